/* hip.c - the sg_gpu_* C ABI (reference surge.h:640-1408) on one MI355X.
 *
 * Replaces the reference's Metal host layer (reference src/metal.m). Plain
 * C11 over the HIP runtime C API; every kernel is launched through the
 * extern "C" launchers of kernels.hip on one stream.
 *
 * Device memory: weights are uploaded once by sg_gpu_load_model and repacked
 * on the device into the GEMV layout, with siblings that read the same input
 * fused into one matrix (q|k|v; qkv|z|b|a; gate/up row-interleaved). State
 * (fp16 K/V caches, DeltaNet conv ring and S) lives in HBM for the life of
 * the state. One decode step is one captured HIP graph replayed per token;
 * the position and token live in a device step descriptor, so the same graph
 * serves every position.
 *
 * Errors follow the reference: sg_err with a static message (or one static
 * format buffer, so not thread-safe), NULL on success. Shapes and sizes are
 * checked on the host before any launch.
 */
#define _GNU_SOURCE
#ifndef __HIP_PLATFORM_AMD__
#define __HIP_PLATFORM_AMD__ 1
#endif
#include <hip/hip_runtime_api.h>

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "kernels.h"
#include "surge.h"

/* ---------------------------------------------------------------------
 * errors
 * --------------------------------------------------------------------- */

static char g_errbuf[512];
static sg_err errf(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_errbuf, sizeof g_errbuf, fmt, ap);
    va_end(ap);
    return (sg_err){g_errbuf};
}
#define HIPCHK(call, what) do { hipError_t _e = (call); \
    if (_e != hipSuccess) return errf("gpu: %s failed: %s", what, hipGetErrorString(_e)); } while (0)

/* ---------------------------------------------------------------------
 * types
 * --------------------------------------------------------------------- */

enum { BUF_ALLOC = 0, BUF_WRAP = 1, BUF_DEVICE = 2 };

typedef struct {
    sg_gpu *g;
    void *dev;
    void *host;          /* ALLOC: owned mirror; WRAP: caller's pointer; DEVICE: NULL */
    uint64_t nbytes;
    int kind;
} gbuf;

typedef struct {          /* a device matrix in the GEMV layout */
    int8_t *qs;
    uint16_t *d;
    uint16_t *dt;            /* the scales block-major [cols/32][rows], for the prefill GEMM (or NULL) */
    float *wf;
    uint32_t rows, cols;
} dmat;

typedef struct {
    bool attn;
    dmat in, out, gu, down;
    float *ln1, *ln2, *qn, *kn, *ssm_norm, *conv_w, *ssm_a, *dt_bias;
    uint16_t *kc, *vc;    /* [n_kv][max_ctx][hd] f16 (head-major: a split's keys are contiguous) */
    float *ring;          /* [4][conv_dim]: last inputs, slot = position % 4 */
    float *S;             /* [n_v][dv][dk] */
} glayer;

typedef struct { void *p; uint64_t n; } alloc_rec;

struct sg_gpu {
    int dev;
    hipStream_t stream;
    alloc_rec *allocs;
    uint32_t n_allocs, cap_allocs;
    uint64_t alloc_bytes;

    /* model */
    const sg_model *model;
    sg_cfg cfg;
    bool q8;
    glayer *ls;
    dmat emb, lm;
    bool lm_is_emb;
    float *out_norm;
    uint32_t key_dim, value_dim, conv_dim, q_width, kv_width, attn_width;

    /* state */
    bool have_state;
    uint32_t max_ctx, used, max_splits;
    uint32_t split_cap;     /* resolved decode split cap (SURGE_SPLITK_GQA_CAP or SGK_MAX_SPLITS) */
    uint32_t gdn_blocks;    /* DeltaNet step workgroups per value head (1 or SGK_GDN_BLOCKS) */
    float *cs_table;
    float *x, *act, *ctx, *ybuf, *gbuf, *ffg, *logits, *am, *as, *aacc;
    uint32_t *amax_scratch, *hist;
    float *gss;             /* DeltaNet step: per-head row-block sums of squares */
    sgk_step *d_step, *h_step;
    float *h_logits;
    uint32_t *h_tok;
    hipGraphExec_t g_fwd, g_greedy;
    bool use_graph;

    /* prefill chunk scratch */
    uint32_t pf_chunk;
    uint64_t pf_segments;
    sgk_step *pf_steps, *pf_hsteps;
    float *pf_X, *pf_Xn, *pf_IN, *pf_CONV, *pf_Y, *pf_G, *pf_CTX, *pf_FF, *pf_m, *pf_s, *pf_acc;
    uint16_t *pf_XS;        /* the prefill GEMMs' X split into bf16 hi | lo */
    uint16_t *pf_XS2;       /* a second split: gate/up writes the down projection's into it */
    float *pf_PART;         /* split-K partials of the narrow prefill GEMMs: 4 x chunk x hidden */
    float *pf_WY;           /* the chunked DeltaNet scan's per-(head, sub-chunk) workspace */

    /* the pinned step descriptor's upload: the next write to h_step waits
     * for it (event recorded after each upload) */
    hipEvent_t step_ev;
    bool step_pending;

    /* decode attention selection, read from the environment at
     * sg_gpu_state_new (reference surge.h:1179-1254), and what the decode
     * path has encoded since (one per attention layer per step) */
    bool attn_splitk, attn_gqa, attn_online;
    int attn_arm;
    uint64_t n_per_head, n_gqa, n_online;

    /* one-shot scratch */
    void *tmp;
    uint64_t tmp_bytes;

};

/* The decode attention partial a state dispatches (fixed per state: the
 * MI355X policy does not change the arm with depth). */
enum { ARM_SINGLE = 0,      /* SURGE_ATTN_SPLITK=0: one split per head, no split-K */
       ARM_PER_HEAD,        /* split-K, one workgroup per (split, query head) */
       ARM_GQA,             /* split-K, one workgroup per (split, kv head) */
       ARM_ONLINE };        /* SURGE_ATTN_SPLITK_ONLINE=1: the same kernel, counted apart */

/* ---------------------------------------------------------------------
 * allocation bookkeeping
 * --------------------------------------------------------------------- */

static sg_err dalloc(sg_gpu *g, uint64_t n, void **out) {
    *out = NULL;
    if (n == 0) n = 1;
    void *p = NULL;
    hipError_t e = hipMalloc(&p, n);
    if (e != hipSuccess) return errf("gpu: hipMalloc(%llu) failed: %s", (unsigned long long)n, hipGetErrorString(e));
    if (g->n_allocs == g->cap_allocs) {
        uint32_t nc = g->cap_allocs ? 2 * g->cap_allocs : 256;
        alloc_rec *r = realloc(g->allocs, nc * sizeof *r);
        if (!r) { hipFree(p); return (sg_err){"gpu: out of host memory"}; }
        g->allocs = r;
        g->cap_allocs = nc;
    }
    g->allocs[g->n_allocs++] = (alloc_rec){p, n};
    g->alloc_bytes += n;
    *out = p;
    return SG_OK;
}

static sg_err dzalloc(sg_gpu *g, uint64_t n, void **out) {
    sg_err e = dalloc(g, n, out);
    if (sg_failed(e)) return e;
    HIPCHK(hipMemset(*out, 0, n ? n : 1), "hipMemset");
    return SG_OK;
}

static void dfree(sg_gpu *g, void *p) {
    if (!g || !p) return;
    for (uint32_t i = 0; i < g->n_allocs; i++) {
        if (g->allocs[i].p == p) {
            g->alloc_bytes -= g->allocs[i].n;
            g->allocs[i] = g->allocs[--g->n_allocs];
            hipFree(p);
            return;
        }
    }
}

uint64_t sg_gpu_current_alloc_bytes(const sg_gpu *g) { return g ? g->alloc_bytes : 0; }

/* ---------------------------------------------------------------------
 * lifecycle and buffers
 * --------------------------------------------------------------------- */

sg_err sg_gpu_init(sg_gpu **out) {
    if (!out) return (sg_err){"gpu: invalid arguments"};
    *out = NULL;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n < 1) return (sg_err){"gpu: no HIP device available"};
    sg_gpu *g = calloc(1, sizeof *g);
    if (!g) return (sg_err){"gpu: out of memory"};
    g->dev = 0;
    if (hipSetDevice(0) != hipSuccess) { free(g); return (sg_err){"gpu: hipSetDevice failed"}; }
    /* the no-allocation entry points' static workspace: its device address on
     * this device, looked up once with the device current */
    hipError_t se = sgk_scratch_init(g->dev);
    if (se != hipSuccess) {
        free(g);
        return errf("gpu: static workspace lookup failed: %s", hipGetErrorString(se));
    }
    /* Default priority (never a prioritised stream). */
    if (hipStreamCreateWithFlags(&g->stream, hipStreamNonBlocking) != hipSuccess) {
        free(g);
        return (sg_err){"gpu: hipStreamCreate failed"};
    }
    const char *ev = getenv("SURGE_HIP_GRAPH");
    g->use_graph = !(ev && strcmp(ev, "0") == 0);
    g->attn_splitk = g->attn_gqa = true;       /* the defaults until a state reads the environment */
    g->attn_online = false;
    /* The KV module allocates through this library (reference metal.m:627-633). */
    sg_kv_set_backend(sg_gpu_alloc, sg_gpu_buf_free, sg_gpu_buf_host);
    *out = g;
    return SG_OK;
}

static void state_free(sg_gpu *g);
static void model_free(sg_gpu *g);

void sg_gpu_free(sg_gpu *g) {
    if (!g) return;
    hipStreamSynchronize(g->stream);
    state_free(g);
    model_free(g);
    while (g->n_allocs) dfree(g, g->allocs[g->n_allocs - 1].p);
    free(g->allocs);
    hipStreamDestroy(g->stream);
    free(g);
}

sg_err sg_gpu_wrap(sg_gpu *g, const void *ptr, uint64_t nbytes, void **buf_out) {
    if (!g || !ptr || !buf_out || !nbytes) return (sg_err){"gpu: sg_gpu_wrap got an invalid argument"};
    *buf_out = NULL;
    if ((uintptr_t)ptr % 4) return (sg_err){"gpu: sg_gpu_wrap needs a 4-byte aligned pointer"};
    gbuf *b = calloc(1, sizeof *b);
    if (!b) return (sg_err){"gpu: out of memory"};
    sg_err e = dalloc(g, nbytes, &b->dev);
    if (sg_failed(e)) { free(b); return e; }
    if (hipMemcpy(b->dev, ptr, nbytes, hipMemcpyHostToDevice) != hipSuccess) {
        dfree(g, b->dev);
        free(b);
        return (sg_err){"gpu: sg_gpu_wrap upload failed"};
    }
    b->g = g;
    b->host = (void *)ptr;
    b->nbytes = nbytes;
    b->kind = BUF_WRAP;
    *buf_out = b;
    return SG_OK;
}

sg_err sg_gpu_alloc(sg_gpu *g, uint64_t nbytes, void **buf_out, void **host_out) {
    if (!g || !buf_out || !nbytes) return (sg_err){"gpu: sg_gpu_alloc got an invalid argument"};
    *buf_out = NULL;
    if (host_out) *host_out = NULL;
    gbuf *b = calloc(1, sizeof *b);
    if (!b) return (sg_err){"gpu: out of memory"};
    b->host = calloc(1, nbytes);
    if (!b->host) { free(b); return (sg_err){"gpu: out of host memory for the mirror"}; }
    sg_err e = dzalloc(g, nbytes, &b->dev);
    if (sg_failed(e)) { free(b->host); free(b); return e; }
    b->g = g;
    b->nbytes = nbytes;
    b->kind = BUF_ALLOC;
    *buf_out = b;
    if (host_out) *host_out = b->host;
    return SG_OK;
}

sg_err sg_gpu_wrap_device(sg_gpu *g, void *dev_ptr, uint64_t nbytes, void **buf_out) {
    if (!g || !dev_ptr || !buf_out || !nbytes) return (sg_err){"gpu: sg_gpu_wrap_device got an invalid argument"};
    gbuf *b = calloc(1, sizeof *b);
    if (!b) return (sg_err){"gpu: out of memory"};
    b->g = g;
    b->dev = dev_ptr;
    b->nbytes = nbytes;
    b->kind = BUF_DEVICE;
    *buf_out = b;
    return SG_OK;
}

void sg_gpu_buf_free(void *buf) {
    gbuf *b = buf;
    if (!b) return;
    if (b->kind != BUF_DEVICE) dfree(b->g, b->dev);
    if (b->kind == BUF_ALLOC) free(b->host);
    free(b);
}

void *sg_gpu_buf_host(void *buf) { return buf ? ((gbuf *)buf)->host : NULL; }
void *sg_gpu_buf_device(void *buf) { return buf ? ((gbuf *)buf)->dev : NULL; }

sg_err sg_gpu_buf_upload(void *buf) {
    gbuf *b = buf;
    if (!b) return (sg_err){"gpu: NULL buffer"};
    if (b->kind != BUF_ALLOC) return SG_OK;
    HIPCHK(hipMemcpy(b->dev, b->host, b->nbytes, hipMemcpyHostToDevice), "upload");
    return SG_OK;
}

sg_err sg_gpu_buf_download(void *buf) {
    gbuf *b = buf;
    if (!b) return (sg_err){"gpu: NULL buffer"};
    if (b->kind != BUF_ALLOC) return SG_OK;
    HIPCHK(hipMemcpy(b->host, b->dev, b->nbytes, hipMemcpyDeviceToHost), "download");
    return SG_OK;
}

/* ---------------------------------------------------------------------
 * one-shot helpers: size checks, mirror sync, scratch
 * --------------------------------------------------------------------- */

static float fbits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

static sg_err need(const void *buf, uint64_t bytes, const char *what) {
    const gbuf *b = buf;
    if (!b) return errf("gpu: %s is NULL", what);
    if (b->nbytes < bytes) return errf("gpu: %s holds %llu bytes, needs %llu", what,
                                       (unsigned long long)b->nbytes, (unsigned long long)bytes);
    return SG_OK;
}

static bool overlap(const void *a, const void *b) {
    const gbuf *x = a, *y = b;
    if (!x || !y) return false;
    const char *p = x->dev, *q = y->dev;
    return p < q + y->nbytes && q < p + x->nbytes;
}

static sg_err push(void *const *bufs, int n) {
    for (int i = 0; i < n; i++) {
        if (!bufs[i]) continue;
        sg_err e = sg_gpu_buf_upload(bufs[i]);
        if (sg_failed(e)) return e;
    }
    return SG_OK;
}

static sg_err finish(sg_gpu *g, hipError_t launch, void *const *outs, int n) {
    if (launch != hipSuccess) return errf("gpu: kernel launch failed: %s", hipGetErrorString(launch));
    HIPCHK(hipStreamSynchronize(g->stream), "kernel execution");
    for (int i = 0; i < n; i++) {
        if (!outs[i]) continue;
        sg_err e = sg_gpu_buf_download(outs[i]);
        if (sg_failed(e)) return e;
    }
    return SG_OK;
}

static sg_err scratch(sg_gpu *g, uint64_t bytes, void **out) {
    if (g->tmp_bytes < bytes) {
        dfree(g, g->tmp);
        g->tmp = NULL;
        g->tmp_bytes = 0;
        sg_err e = dalloc(g, bytes, &g->tmp);
        if (sg_failed(e)) return e;
        g->tmp_bytes = bytes;
    }
    *out = g->tmp;
    return SG_OK;
}

#define DEV(b) ((b) ? ((gbuf *)(b))->dev : NULL)

/* ---------------------------------------------------------------------
 * sg_gpu_run_op: the per-op oracle hooks (surge.h:666-762)
 * --------------------------------------------------------------------- */

sg_err sg_gpu_run_op(sg_gpu *g, const char *kernel, void *a, void *b, void *out,
                     const uint32_t p[8]) {
    if (!g || !kernel || !a || !out || !p) return (sg_err){"gpu: sg_gpu_run_op got a NULL argument"};
    if (overlap(out, a) || overlap(out, b)) {
        if (strcmp(kernel, "k_delta_step") != 0)
            return errf("gpu: %s: out must not overlap an input", kernel);
    }
    void *ins[3] = {a, b, out};
    void *outs[1] = {out};
    hipStream_t s = g->stream;
    sg_err e;
    const uint32_t n = p[0];

    if (!strcmp(kernel, "k_matvec_q8") || !strcmp(kernel, "k_matvec_f32")) {
        bool q8 = kernel[9] == 'q';
        uint32_t rows = p[0], cols = p[1];
        if (!rows || !cols || (q8 && cols % 32)) return errf("gpu: %s: bad shape %ux%u", kernel, rows, cols);
        uint64_t wbytes = q8 ? (uint64_t)rows * (cols / 32) * 34 : (uint64_t)rows * cols * 4;
        if (sg_failed(e = need(a, wbytes, "w")) || sg_failed(e = need(b, (uint64_t)cols * 4, "x")) ||
            sg_failed(e = need(out, (uint64_t)rows * 4, "y"))) return e;
        if (sg_failed(e = push(ins, 3))) return e;
        sgk_gemv ga = {0};
        ga.rows = rows; ga.cols = cols; ga.x = DEV(b); ga.y = DEV(out);
        ga.pro = SGK_PRO_NONE; ga.epi = SGK_EPI_STORE;
        if (q8) {
            void *t;
            if (sg_failed(e = scratch(g, (uint64_t)rows * cols + (uint64_t)rows * (cols / 32) * 2 + 256, &t))) return e;
            ga.qs = t;
            ga.d = (uint16_t *)((char *)t + (((uint64_t)rows * cols + 255) / 256 * 256));
            hipError_t he = sgk_repack_q8(DEV(a), rows, cols, (int8_t *)ga.qs, (uint16_t *)ga.d, NULL, rows, 0, 1, s);
            if (he != hipSuccess) return finish(g, he, NULL, 0);
        } else {
            ga.wf = DEV(a);
        }
        return finish(g, sgk_gemv_launch(&ga, s), outs, 1);
    }
    if (!strcmp(kernel, "k_rmsnorm") || !strcmp(kernel, "k_rmsnorm_heads")) {
        bool heads = kernel[9] == '_';
        uint32_t nh = heads ? p[1] : 1, stride = heads ? (p[3] ? p[3] : n) : n;
        float eps = fbits(heads ? p[2] : p[1]);
        bool hw = heads ? p[4] != 0 : p[2] != 0;
        if (!n || !nh || stride < n) return errf("gpu: %s: bad shape", kernel);
        uint64_t bytes = ((uint64_t)(nh - 1) * stride + n) * 4;
        if (sg_failed(e = need(a, bytes, "x")) || sg_failed(e = need(out, bytes, "out"))) return e;
        if (hw && sg_failed(e = need(b, (uint64_t)n * 4, "w"))) return e;
        if (sg_failed(e = push(ins, 3))) return e;
        return finish(g, sgk_rmsnorm_heads(DEV(a), hw ? DEV(b) : NULL, DEV(out), n, nh, stride, eps, s), outs, 1);
    }
    if (!strcmp(kernel, "k_rope") || !strcmp(kernel, "k_rope_heads")) {
        bool heads = kernel[6] == '_';
        uint32_t hd = p[0], rd = p[1], nh = heads ? p[2] : 1, stride = heads ? (p[3] ? p[3] : hd) : hd;
        if (!hd || hd > 256 || rd < 2 || rd > hd || rd % 2 || !nh || stride < hd)
            return errf("gpu: %s: bad shape", kernel);
        uint64_t bytes = ((uint64_t)(nh - 1) * stride + hd) * 4;
        if (sg_failed(e = need(a, bytes, "x")) || sg_failed(e = need(b, (uint64_t)rd * 4, "cs")) ||
            sg_failed(e = need(out, bytes, "out"))) return e;
        if (sg_failed(e = push(ins, 3))) return e;
        return finish(g, sgk_rope_heads(DEV(a), DEV(b), DEV(out), hd, rd, nh, stride, s), outs, 1);
    }
    if (!strcmp(kernel, "k_softmax")) {
        if (!n) return (sg_err){"gpu: k_softmax: n is zero"};
        if (sg_failed(e = need(a, (uint64_t)n * 4, "x")) || sg_failed(e = need(out, (uint64_t)n * 4, "out"))) return e;
        if (sg_failed(e = push(ins, 3))) return e;
        return finish(g, sgk_softmax(DEV(a), DEV(out), n, s), outs, 1);
    }
    struct { const char *name; int op; bool needs_b; } ew[] = {
        {"k_swiglu", SGK_EW_SWIGLU, true}, {"k_silu", SGK_EW_SILU, false},
        {"k_gate_sigmoid", SGK_EW_GATE_SIGMOID, true}, {"k_add", SGK_EW_ADD, true},
        {"k_scale", SGK_EW_SCALE, false},
    };
    for (size_t i = 0; i < sizeof ew / sizeof *ew; i++) {
        if (strcmp(kernel, ew[i].name)) continue;
        if (!n) return errf("gpu: %s: n is zero", kernel);
        if (sg_failed(e = need(a, (uint64_t)n * 4, "a")) || sg_failed(e = need(out, (uint64_t)n * 4, "out"))) return e;
        if (ew[i].needs_b && sg_failed(e = need(b, (uint64_t)n * 4, "b"))) return e;
        if (sg_failed(e = push(ins, 3))) return e;
        return finish(g, sgk_elementwise(ew[i].op, DEV(a), DEV(b), DEV(out), n, fbits(p[1]), s), outs, 1);
    }
    if (!strcmp(kernel, "k_kv_store_f16")) {
        uint64_t off = p[1];
        if (!n) return (sg_err){"gpu: k_kv_store_f16: n is zero"};
        if (sg_failed(e = need(a, (uint64_t)n * 4, "x")) || sg_failed(e = need(out, (off + n) * 2, "cache"))) return e;
        if (sg_failed(e = push(ins, 3))) return e;
        return finish(g, sgk_elementwise(SGK_EW_TO_F16, DEV(a), NULL, (uint16_t *)DEV(out) + off, n, 0.0f, s), outs, 1);
    }
    if (!strcmp(kernel, "k_conv1d_step")) {
        uint32_t ch = p[0], ks = p[1];
        if (!ch || !ks) return (sg_err){"gpu: k_conv1d_step: bad shape"};
        if (sg_failed(e = need(a, (uint64_t)ch * 4, "x")) || sg_failed(e = need(b, (uint64_t)ch * ks * 4, "w")) ||
            sg_failed(e = need(out, (uint64_t)ch * ks * 4, "out"))) return e;
        if (sg_failed(e = push(ins, 3))) return e;
        float *o = DEV(out);
        return finish(g, sgk_conv1d_step(DEV(a), DEV(b), o, o + ch, ch, ks, s), outs, 1);
    }
    if (!strcmp(kernel, "k_delta_step")) {
        uint32_t dk = p[0], dv = p[1];
        if (!dk || !dv) return (sg_err){"gpu: k_delta_step: bad shape"};
        if (sg_failed(e = need(a, (uint64_t)dk * dv * 4, "S")) || sg_failed(e = need(b, (uint64_t)(2 * dk + dv) * 4, "qkv")) ||
            sg_failed(e = need(out, (uint64_t)dv * 4, "out"))) return e;
        void *t;
        if (sg_failed(e = scratch(g, 8, &t))) return e;
        float gates[2] = {fbits(p[2]), fbits(p[3])};
        if (sg_failed(e = push(ins, 3))) return e;
        HIPCHK(hipMemcpy(t, gates, 8, hipMemcpyHostToDevice), "gates upload");
        void *o2[2] = {out, a};
        return finish(g, sgk_delta_multi(DEV(a), DEV(b), DEV(out), t, dk, dv, 1, 1, dk, 1, s), o2, 2);
    }
    if (!strcmp(kernel, "k_rmsnorm_gated")) {
        uint32_t dv = p[0], nh = p[1];
        if (!dv || !nh) return (sg_err){"gpu: k_rmsnorm_gated: bad shape"};
        uint64_t nb = (uint64_t)dv * nh * 4;
        if (sg_failed(e = need(a, nb, "y")) || sg_failed(e = need(b, nb + (uint64_t)dv * 4, "z|w")) ||
            sg_failed(e = need(out, nb, "out"))) return e;
        if (sg_failed(e = push(ins, 3))) return e;
        const float *zb = DEV(b);
        return finish(g, sgk_rmsnorm_gated(DEV(a), zb, zb + (uint64_t)dv * nh, DEV(out), dv, nh, fbits(p[2]), s), outs, 1);
    }
    if (!strcmp(kernel, "k_argmax")) {
        /* the greedy loop's device argmax: out[0] = sg_argmax_f32(a, n) */
        if (!n) return (sg_err){"gpu: k_argmax: n is zero"};
        if (sg_failed(e = need(a, (uint64_t)n * 4, "v")) || sg_failed(e = need(out, 4, "out"))) return e;
        if (sg_failed(e = push(ins, 3))) return e;
        void *t;
        if (sg_failed(e = scratch(g, 4096, &t))) return e;
        return finish(g, sgk_argmax(DEV(a), n, DEV(out), t, s), outs, 1);
    }
    if (!strcmp(kernel, "k_matmul_q8")) {
        uint32_t N = p[0], M = p[1], K = p[2];
        if (!N || !M || !K || K % 32) return (sg_err){"gpu: k_matmul_q8: bad shape (K must be a nonzero multiple of 32)"};
        if (sg_failed(e = need(a, (uint64_t)N * K * 4, "X")) || sg_failed(e = need(b, (uint64_t)M * (K / 32) * 34, "W")) ||
            sg_failed(e = need(out, (uint64_t)N * M * 4, "Y"))) return e;
        if (sg_failed(e = push(ins, 3))) return e;
        void *t;
        const uint64_t qb = ((uint64_t)M * K + 255) / 256 * 256, db = ((uint64_t)M * (K / 32) * 2 + 255) / 256 * 256;
        const uint64_t xb = ((uint64_t)N * K * 4 + 255) / 256 * 256, pc = (uint64_t)4 * N * M;   /* split-K partials */
        if (sg_failed(e = scratch(g, qb + 2 * db + xb + pc * 4, &t))) return e;
        int8_t *qs = t;
        uint16_t *d = (uint16_t *)((char *)t + qb), *dt = (uint16_t *)((char *)t + qb + db);
        uint16_t *xs = (uint16_t *)((char *)t + qb + 2 * db);
        float *part = (float *)((char *)t + qb + 2 * db + xb);
        hipError_t he = sgk_repack_q8(DEV(b), M, K, qs, d, dt, M, 0, 1, s);
        if (he == hipSuccess) he = sgk_gemm_q8(DEV(a), qs, dt, DEV(out), N, M, K, xs, part, pc, s);
        return finish(g, he, outs, 1);
    }
    return errf("gpu: unknown kernel '%s'", kernel);
}

/* ---------------------------------------------------------------------
 * attention one-shots (surge.h:774-980)
 * --------------------------------------------------------------------- */

static sg_err attn_check(const uint32_t p[8], bool need_splits, bool per_head) {
    uint32_t nh = p[0], nkv = p[1], hd = p[2], qs = p[4];
    if (!nh || !nkv || nh % nkv) return (sg_err){"gpu: n_heads must be a nonzero multiple of n_kv_heads"};
    if (!per_head && nh / nkv > 8) return (sg_err){"gpu: GQA group wider than 8 is not supported"};
    if (hd != 16 && hd != 32 && hd != 64 && hd != 128 && hd != 256) return (sg_err){"gpu: head_dim must be 16, 32, 64, 128 or 256"};
    if (qs < hd) return (sg_err){"gpu: q_stride < head_dim"};
    if (need_splits && (!p[6] || p[6] > 1024)) return (sg_err){"gpu: n_splits must be in [1, 1024]"};
    return SG_OK;
}

/* One split-K partial launch over caller buffers: the decode kernel with q
 * taken as given (no norm, RoPE or K/V store). One-shots are not counted in
 * the decode dispatch counters (reference surge.h:1011-1017). */
static sg_err attn_partial_oneshot(sg_gpu *g, void *q, void *k, void *v, void *m, void *s, void *acc,
                                   const uint32_t p[8], bool per_head) {
    if (!g || !q || !k || !v || !m || !s || !acc || !p) return (sg_err){"gpu: attention one-shot got a NULL argument"};
    sg_err e = attn_check(p, true, per_head);
    if (sg_failed(e)) return e;
    uint32_t nh = p[0], nkv = p[1], hd = p[2], seq = p[3], qs = p[4], ns = p[6];
    uint64_t kvb = (uint64_t)seq * nkv * hd * 2;
    if (sg_failed(e = need(q, ((uint64_t)(nh - 1) * qs + hd) * 4, "q")) ||
        (seq && (sg_failed(e = need(k, kvb, "k")) || sg_failed(e = need(v, kvb, "v")))) ||
        sg_failed(e = need(m, (uint64_t)nh * ns * 4, "m")) || sg_failed(e = need(s, (uint64_t)nh * ns * 4, "s")) ||
        sg_failed(e = need(acc, (uint64_t)nh * ns * hd * 4, "acc"))) return e;
    void *outs[3] = {m, s, acc};
    for (int i = 0; i < 3; i++)
        if (overlap(outs[i], q) || overlap(outs[i], k) || overlap(outs[i], v) ||
            overlap(outs[i], outs[(i + 1) % 3])) return (sg_err){"gpu: attention outputs must not overlap"};
    void *ins[3] = {q, k, v};
    if (sg_failed(e = push(ins, 3))) return e;
    sgk_attn A = {0};
    A.q = DEV(q); A.kc = DEV(k); A.vc = DEV(v); A.m = DEV(m); A.s = DEV(s); A.acc = DEV(acc);
    A.n_heads = nh; A.n_kv = nkv; A.hd = hd; A.q_stride = qs; A.seq = seq; A.n_splits = ns; A.max_splits = ns;
    A.ntok = 1; A.scale = fbits(p[5]); A.per_head = per_head;
    return finish(g, sgk_attn_partial(&A, g->stream), outs, 3);
}

sg_err sg_gpu_run_attn_splitk_partial_gqa(sg_gpu *g, void *q, void *k, void *v, void *m,
                                          void *s, void *acc, const uint32_t p[8]) {
    return attn_partial_oneshot(g, q, k, v, m, s, acc, p, false);
}

/* The per-head partial (reference kernels_splitk.metal:156-267): one
 * workgroup per (split, query head). Same bytes as the GQA form. */
sg_err sg_gpu_run_attn_splitk_partial(sg_gpu *g, void *q, void *k, void *v, void *m, void *s,
                                      void *acc, const uint32_t p[8]) {
    return attn_partial_oneshot(g, q, k, v, m, s, acc, p, true);
}

sg_err sg_gpu_run_attn_splitk_combine(sg_gpu *g, void *m, void *s, void *acc, void *out,
                                      const uint32_t p[8]) {
    if (!g || !m || !s || !acc || !out || !p) return (sg_err){"gpu: combine got a NULL argument"};
    uint32_t nh = p[0], hd = p[2], ns = p[6];
    if (!nh || !hd || !ns || ns > 1024) return (sg_err){"gpu: combine: bad shape"};
    sg_err e;
    if (sg_failed(e = need(m, (uint64_t)nh * ns * 4, "m")) || sg_failed(e = need(s, (uint64_t)nh * ns * 4, "s")) ||
        sg_failed(e = need(acc, (uint64_t)nh * ns * hd * 4, "acc")) || sg_failed(e = need(out, (uint64_t)nh * hd * 4, "out")))
        return e;
    if (overlap(out, m) || overlap(out, s) || overlap(out, acc)) return (sg_err){"gpu: combine output overlaps an input"};
    void *ins[3] = {m, s, acc}, *outs[1] = {out};
    if (sg_failed(e = push(ins, 3))) return e;
    sgk_attn A = {0};
    A.m = DEV(m); A.s = DEV(s); A.acc = DEV(acc); A.out = DEV(out);
    A.n_heads = nh; A.hd = hd; A.n_splits = ns; A.max_splits = ns; A.ntok = 1;
    return finish(g, sgk_attn_combine(&A, g->stream), outs, 1);
}

/* Single-pass decode attention: the split-K pair with the decode policy's
 * split count, combined, in one call. p: [0]=nh [1]=nkv [2]=hd [3]=seq
 * [4]=q_stride [5]=scale. The partials go to `ws` when given (the
 * no-allocation variant), else to the gpu's lazily grown one-shot scratch. */
static sg_err attn_decode_oneshot(sg_gpu *g, void *q, void *k, void *v, void *out, const uint32_t p[8],
                                  bool no_alloc) {
    if (!g || !q || !k || !v || !out || !p) return (sg_err){"gpu: attention one-shot got a NULL argument"};
    uint32_t pp[8];
    memcpy(pp, p, sizeof pp);
    pp[6] = sgk_n_splits(p[3]);
    sg_err e = attn_check(pp, true, false);
    if (sg_failed(e)) return e;
    uint32_t nh = pp[0], nkv = pp[1], hd = pp[2], seq = pp[3], qs = pp[4], ns = pp[6];
    uint64_t kvb = (uint64_t)seq * nkv * hd * 2;
    if (sg_failed(e = need(q, ((uint64_t)(nh - 1) * qs + hd) * 4, "q")) ||
        (seq && (sg_failed(e = need(k, kvb, "k")) || sg_failed(e = need(v, kvb, "v")))) ||
        sg_failed(e = need(out, (uint64_t)nh * hd * 4, "out"))) return e;
    const uint64_t wsb = (uint64_t)nh * ns * (2 + hd) * 4;
    void *t;
    if (no_alloc) {
        if (wsb > SGK_SCRATCH_BYTES)
            return errf("gpu: attn_decode_f16_noalloc: %u heads x %u splits x (head_dim %u + 2) partials need %llu "
                        "bytes; the static workspace holds %u", nh, ns, hd, (unsigned long long)wsb,
                        (unsigned)SGK_SCRATCH_BYTES);
        if (!(t = sgk_scratch_ptr(g->dev))) return (sg_err){"gpu: the static workspace is not set up"};
    } else if (sg_failed(e = scratch(g, wsb, &t))) {
        return e;
    }
    float *mm = t, *ss = mm + (uint64_t)nh * ns, *aa = ss + (uint64_t)nh * ns;
    void *ins[3] = {q, k, v}, *outs[1] = {out};
    if (sg_failed(e = push(ins, 3))) return e;
    sgk_attn A = {0};
    A.q = DEV(q); A.kc = DEV(k); A.vc = DEV(v); A.m = mm; A.s = ss; A.acc = aa; A.out = DEV(out);
    A.n_heads = nh; A.n_kv = nkv; A.hd = hd; A.q_stride = qs; A.seq = seq; A.n_splits = ns; A.max_splits = ns;
    A.ntok = 1; A.scale = fbits(pp[5]);
    hipError_t he = sgk_attn_partial(&A, g->stream);
    if (he == hipSuccess) he = sgk_attn_combine(&A, g->stream);
    return finish(g, he, outs, 1);
}

sg_err sg_gpu_run_attn_decode_f16(sg_gpu *g, void *q, void *k, void *v, void *out, const uint32_t p[8]) {
    return attn_decode_oneshot(g, q, k, v, out, p, false);
}

/* The same call with no device allocation (no reference counterpart; for
 * callers that cannot allocate): the partials live in the library's static
 * device workspace (SGK_SCRATCH_BYTES = 4 MiB per GPU, found at sg_gpu_init),
 * so n_heads * n_splits * (head_dim + 2) * 4 bytes must fit in it (24 heads
 * at head_dim 256 and 128 splits do). Calls that overlap on one GPU share
 * that workspace and race; this library's calls are synchronous on one
 * stream, so its own calls never overlap. */
sg_err sg_gpu_run_attn_decode_f16_noalloc(sg_gpu *g, void *q, void *k, void *v, void *out, const uint32_t p[8]) {
    return attn_decode_oneshot(g, q, k, v, out, p, true);
}

/* Split policy (surge.h:1020-1106), re-derived for 256 CUs: see kernels.h. */
uint32_t sg_gpu_splitk_n_splits(uint32_t seq) { return sgk_n_splits(seq); }
uint32_t sg_gpu_splitk_gqa_n_splits(uint32_t seq) { return sgk_n_splits(seq); }
/* The cap a live state dispatches with: its accepted SURGE_SPLITK_GQA_CAP, or
 * the default (also for NULL or a gpu with no live state). */
uint32_t sg_gpu_splitk_gqa_cap(const sg_gpu *g) {
    return (g && g->have_state && g->split_cap) ? g->split_cap : SGK_MAX_SPLITS;
}
uint32_t sg_gpu_splitk_gqa_n_splits_at(const sg_gpu *g, uint32_t seq) {
    return sgk_n_splits_cap(seq, sg_gpu_splitk_gqa_cap(g));
}
/* The selection predicates (reference surge.h:1011-1050) answer from the
 * state's switches (SURGE_ATTN_SPLITK, _GQA, _ONLINE, read at
 * sg_gpu_state_new; before any state, the defaults 1, 1, 0). The group must
 * be in [2, 8]; the online arm also needs head_dim in [1, 256] and, when
 * its switch is on, takes the dispatch from the GQA arm for the state's
 * head_dim, so the two never both claim one. Unlike the reference, whose
 * measured floor of 128 threadgroups leaves short contexts to the per-head
 * partial, the MI355X policy has no floor: `seq` does not change the
 * answer. */
static bool gqa_band(uint32_t n_heads, uint32_t n_kv_heads) {
    return n_kv_heads && n_heads % n_kv_heads == 0 && n_heads / n_kv_heads >= 2 && n_heads / n_kv_heads <= 8;
}
bool sg_gpu_splitk_online_selected(const sg_gpu *g, uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                                   uint32_t seq) {
    (void)seq;
    return g && g->attn_splitk && g->attn_online && gqa_band(n_heads, n_kv_heads) && head_dim >= 1 &&
           head_dim <= 256;
}
bool sg_gpu_splitk_gqa_selected(const sg_gpu *g, uint32_t n_heads, uint32_t n_kv_heads, uint32_t seq) {
    if (!g || !g->attn_splitk || !g->attn_gqa || !gqa_band(n_heads, n_kv_heads)) return false;
    const uint32_t hd = g->model ? g->cfg.head_dim : 0;
    return !sg_gpu_splitk_online_selected(g, n_heads, n_kv_heads, hd, seq);
}
void sg_gpu_splitk_dispatch_counts(const sg_gpu *g, uint64_t *per_head, uint64_t *gqa) {
    if (per_head) *per_head = g ? g->n_per_head : 0;
    if (gqa) *gqa = g ? g->n_gqa : 0;
}
uint64_t sg_gpu_splitk_online_dispatches(const sg_gpu *g) { return g ? g->n_online : 0; }

sg_err sg_gpu_run_delta_multi(sg_gpu *g, void *S, void *qkv, void *out, void *gates,
                              const uint32_t p[8]) {
    if (!g || !S || !qkv || !out || !gates || !p) return (sg_err){"gpu: delta_multi got a NULL argument"};
    uint32_t dk = p[0], dv = p[1], nv = p[2], nk = p[3], kd = p[4];
    if (!dk || !dv || !nv || !nk || nv % nk || kd < nk * dk) return (sg_err){"gpu: delta_multi: bad shape"};
    if (dk != 32 && dk != 64 && dk != 128 && dk != 256) return (sg_err){"gpu: delta_multi: dk must be 32, 64, 128 or 256"};
    sg_err e;
    if (sg_failed(e = need(S, (uint64_t)nv * dv * dk * 4, "S")) ||
        sg_failed(e = need(qkv, ((uint64_t)2 * kd + (uint64_t)nv * dv) * 4, "qkv")) ||
        sg_failed(e = need(out, (uint64_t)nv * dv * 4, "out")) || sg_failed(e = need(gates, (uint64_t)2 * nv * 4, "gates")))
        return e;
    void *ins[4] = {S, qkv, gates, out}, *outs[2] = {S, out};
    if (sg_failed(e = push(ins, 4))) return e;
    return finish(g, sgk_delta_multi(DEV(S), DEV(qkv), DEV(out), DEV(gates), dk, dv, nv, nk, kd, p[5] != 0, g->stream),
                  outs, 2);
}

/* The decode path's fused DeltaNet layer step (k_gdn_step) on caller buffers
 * (no reference counterpart: the reference tests its decode kernels one by
 * one, k_conv1d_step, k_delta_gates, k_delta_multi, k_rmsnorm_gated; here
 * they are one kernel, so it is tested whole). One token:
 *   in    [conv_dim + value_dim + 2 n_v]  the input projection's rows
 *         qkv | z | b | a (qkv before the conv);
 *   w     [conv_dim ksize + 2 n_v + dv]   conv_w | ssm_a | dt_bias | ssm_norm;
 *   state [(ksize-1) conv_dim + n_v dv dk] the conv tail (oldest first) | S,
 *         updated in place;
 *   out   [value_dim]                     silu(z) * rmsnorm(y, ssm_norm).
 * p: [0]=dk [1]=dv [2]=n_v [3]=n_k [4]=ksize [5]=tiled [6]=ssm_a is -exp(A_log)
 * [7]=eps bits. conv_dim = 2 n_k dk + n_v dv. head_v_dim <= 128 (one
 * workgroup per value head, the decode default). */
/* SURGE_DELTA_SCAN, the prefill DeltaNet scan's form: mfma (default) or seq.
 * Any other value is refused, not ignored, so an A/B of scan forms never
 * measures one it did not name. */
static sg_err delta_scan_env(void) {
    if (sgk_delta_scan_env_ok()) return SG_OK;
    return errf("gpu: SURGE_DELTA_SCAN='%s' must be mfma or seq (default mfma)", getenv("SURGE_DELTA_SCAN"));
}

sg_err sg_gpu_run_gdn_step(sg_gpu *g, void *in, void *w, void *state, void *out, const uint32_t p[8]) {
    if (!g || !in || !w || !state || !out || !p) return (sg_err){"gpu: gdn_step got a NULL argument"};
    const uint32_t dk = p[0], dv = p[1], nv = p[2], nk = p[3], ks = p[4];
    if (dk != 32 && dk != 64 && dk != 128 && dk != 256) return (sg_err){"gpu: gdn_step: dk must be 32, 64, 128 or 256"};
    if (!dv || dv > 128 || !nv || !nk || nv % nk || ks < 1 || ks > 4)
        return (sg_err){"gpu: gdn_step: bad shape (dv <= 128, n_v a multiple of n_k, ksize 1..4)"};
    const uint64_t cd = 2ull * nk * dk + (uint64_t)nv * dv, vd = (uint64_t)nv * dv, keep = ks - 1;
    sg_err e;
    if (sg_failed(e = need(in, (cd + vd + 2ull * nv) * 4, "in")) ||
        sg_failed(e = need(w, (cd * ks + 2ull * nv + dv) * 4, "w")) ||
        sg_failed(e = need(state, (keep * cd + vd * dk) * 4, "state")) || sg_failed(e = need(out, vd * 4, "out")))
        return e;
    if (overlap(out, in) || overlap(out, w) || overlap(out, state) || overlap(state, in) || overlap(state, w))
        return (sg_err){"gpu: gdn_step: buffers must not overlap"};
    void *ins[3] = {in, w, state}, *outs[2] = {state, out};
    if (sg_failed(e = push(ins, 3))) return e;
    /* scratch: the step descriptor, then the 4-slot ring. The step runs at
     * position 3, so the taps read slots 3-keep .. 2, which take the conv
     * tail's rows, and the input goes to slot 3. */
    void *t;
    if (sg_failed(e = scratch(g, 256 + 4 * cd * 4, &t))) return e;
    sgk_step st = {0, 3, {0, 0}};
    float *ring = (float *)((char *)t + 256), *dst = DEV(state), *wp = DEV(w);
    hipStream_t s = g->stream;
    HIPCHK(hipMemcpyAsync(t, &st, sizeof st, hipMemcpyHostToDevice, s), "gdn_step descriptor");
    if (keep)
        HIPCHK(hipMemcpyAsync(ring + (3 - keep) * cd, dst, keep * cd * 4, hipMemcpyDeviceToDevice, s), "conv tail in");
    sgk_gdn d = {0};
    d.in = DEV(in); d.z = (const float *)DEV(in) + cd; d.conv_w = wp; d.ssm_a = wp + cd * ks;
    d.dt_bias = d.ssm_a + nv; d.norm_w = d.dt_bias + nv; d.ring = ring; d.S = dst + keep * cd;
    d.step = t; d.n_k = nk; d.n_v = nv; d.dk = dk; d.dv = dv; d.conv_dim = (uint32_t)cd; d.ksize = ks;
    d.tiled = p[5] != 0; d.neg_exp = p[6] != 0; d.out = DEV(out); d.eps = fbits(p[7]); d.blocks = 1;
    hipError_t he = sgk_gdn_step(&d, s);
    if (he == hipSuccess && keep)
        he = hipMemcpyAsync(dst, ring + (4 - keep) * cd, keep * cd * 4, hipMemcpyDeviceToDevice, s);
    return finish(g, he, outs, 2);
}

/* The prefill path's DeltaNet layer core over a chunk of n tokens, with the
 * kernels prefill_chunk runs (sgk_gdn_chunk: the chunk conv with its q/k
 * norm, the conv ring, the gates and the delta-rule scan in the build's
 * default form; then the RMSNormGated rows) on caller buffers (no reference
 * counterpart: the reference's prefill runs its per-token kernels in a loop,
 * kernels.metal:1111-1278). Buffers as sg_gpu_run_gdn_step, with n rows:
 *   in    [n][conv_dim + value_dim + 2 n_v]  qkv | z | b | a per token;
 *   w     [conv_dim ksize + 2 n_v + dv]      conv_w | ssm_a | dt_bias | ssm_norm;
 *   state [(ksize-1) conv_dim + n_v dv dk]   the conv tail (oldest first) | S,
 *         updated in place;
 *   out   [n][value_dim].
 * p: [0]=dk [1]=dv [2]=n_v [3]=n_k [4]=ksize [5]=flags: bit 0 tiled, bit 1
 * ssm_a is -exp(A_log), bits 2-3 the first position mod 4 (the ring slot the
 * chunk starts at) [6]=n [7]=eps bits. */
sg_err sg_gpu_run_gdn_chunk(sg_gpu *g, void *in, void *w, void *state, void *out, const uint32_t p[8]) {
    if (!g || !in || !w || !state || !out || !p) return (sg_err){"gpu: gdn_chunk got a NULL argument"};
    const uint32_t dk = p[0], dv = p[1], nv = p[2], nk = p[3], ks = p[4], n = p[6];
    if (dk != 32 && dk != 64 && dk != 128 && dk != 256) return (sg_err){"gpu: gdn_chunk: dk must be 32, 64, 128 or 256"};
    if (sg_failed(delta_scan_env())) return delta_scan_env();
    if (!dv || !nv || !nk || nv % nk || ks < 1 || ks > 4 || !n)
        return (sg_err){"gpu: gdn_chunk: bad shape (n_v a multiple of n_k, ksize 1..4, n > 0)"};
    const uint64_t cd = 2ull * nk * dk + (uint64_t)nv * dv, vd = (uint64_t)nv * dv, keep = ks - 1;
    const uint64_t row = cd + vd + 2ull * nv;
    sg_err e;
    if (sg_failed(e = need(in, n * row * 4, "in")) || sg_failed(e = need(w, (cd * ks + 2ull * nv + dv) * 4, "w")) ||
        sg_failed(e = need(state, (keep * cd + vd * dk) * 4, "state")) || sg_failed(e = need(out, n * vd * 4, "out")))
        return e;
    if (overlap(out, in) || overlap(out, w) || overlap(out, state) || overlap(state, in) || overlap(state, w))
        return (sg_err){"gpu: gdn_chunk: buffers must not overlap"};
    void *ins[3] = {in, w, state}, *outs[2] = {state, out};
    if (sg_failed(e = push(ins, 3))) return e;
    /* scratch: the chunk's step descriptors, the 4-slot ring, the conv
     * output, the scan readouts and the scan workspace */
    const uint64_t sb = ((uint64_t)n * sizeof(sgk_step) + 255) / 256 * 256, rb = 4 * cd * 4, cb = (uint64_t)n * cd * 4,
                   yb = (uint64_t)n * vd * 4, wsb = (uint64_t)sgk_delta_ws_floats(nv, n) * 4;
    void *t;
    if (sg_failed(e = scratch(g, sb + rb + cb + yb + wsb, &t))) return e;
    const uint32_t pos0 = 4 + ((p[5] >> 2) & 3);
    sgk_step *st = calloc(n, sizeof *st);
    if (!st) return (sg_err){"gpu: gdn_chunk: out of host memory"};
    for (uint32_t z = 0; z < n; z++) st[z].pos = pos0 + z;
    hipStream_t s = g->stream;
    hipError_t he = hipMemcpyAsync(t, st, n * sizeof *st, hipMemcpyHostToDevice, s);
    if (he == hipSuccess) he = hipStreamSynchronize(s);
    free(st);
    HIPCHK(he, "gdn_chunk descriptors");
    float *ring = (float *)((char *)t + sb), *conv = ring + 4 * cd, *y = conv + (uint64_t)n * cd, *ws = y + (uint64_t)n * vd;
    float *dst = DEV(state), *wp = DEV(w);
    /* the tail's row j is the input of position pos0 - keep + j */
    for (uint64_t j = 0; j < keep; j++)
        HIPCHK(hipMemcpyAsync(ring + ((pos0 - keep + j) & 3) * cd, dst + j * cd, cd * 4, hipMemcpyDeviceToDevice, s),
               "conv tail in");
    sgk_gdn d = {0};
    d.in = DEV(in); d.conv_w = wp; d.ssm_a = wp + cd * ks; d.dt_bias = d.ssm_a + nv; d.ring = ring;
    d.S = dst + keep * cd; d.y = y; d.step = t; d.n_k = nk; d.n_v = nv; d.dk = dk; d.dv = dv;
    d.conv_dim = (uint32_t)cd; d.ksize = ks; d.tiled = p[5] & 1; d.neg_exp = (p[5] >> 1) & 1;
    he = sgk_gdn_chunk(&d, conv, (uint32_t)row, n, ws, s);
    if (he == hipSuccess)
        he = sgk_rmsnorm_gated_rows(y, (const float *)DEV(in) + cd, (uint32_t)row, d.ssm_a + 2 * nv, DEV(out), dv, nv, n,
                                    fbits(p[7]), s);
    /* the new tail: the inputs of the last keep positions, which the ring
     * holds (positions before the chunk kept their slots) */
    for (uint64_t j = 0; he == hipSuccess && j < keep; j++)
        he = hipMemcpyAsync(dst + j * cd, ring + ((pos0 + n - keep + j) & 3) * cd, cd * 4, hipMemcpyDeviceToDevice, s);
    return finish(g, he, outs, 2);
}

/* ---------------------------------------------------------------------
 * prefill per-op hooks (surge.h:787-800, 1133-1142): the chunk kernels the
 * prefill path runs, one synchronous call each, with the reference's
 * argument layouts and params.
 * --------------------------------------------------------------------- */

sg_err sg_gpu_run_conv1d_chunk(sg_gpu *g, void *x, void *w, void *out, void *state, const uint32_t p[8]) {
    if (!g || !x || !w || !out || !state || !p) return (sg_err){"gpu: conv1d_chunk got a NULL argument"};
    uint32_t ch = p[0], ks = p[1], n = p[2];
    if (!ch || ks < 1 || ks > 4 || !n) return (sg_err){"gpu: conv1d_chunk: bad shape (ksize 1..4)"};
    sg_err e;
    uint64_t xb = (uint64_t)n * ch * 4;
    if (sg_failed(e = need(x, xb, "x")) || sg_failed(e = need(w, (uint64_t)ch * ks * 4, "w")) ||
        sg_failed(e = need(out, xb, "out")) || sg_failed(e = need(state, (uint64_t)(ks - 1) * ch * 4 + (ks == 1 ? 4 : 0), "state")))
        return e;
    if (overlap(out, x) || overlap(out, w) || overlap(out, state)) return (sg_err){"gpu: conv1d_chunk: out overlaps an input"};
    void *ins[4] = {x, w, out, state}, *outs[2] = {out, state};
    if (sg_failed(e = push(ins, 4))) return e;
    return finish(g, sgk_conv1d_chunk(DEV(x), DEV(w), DEV(out), DEV(state), ch, ks, n, g->stream), outs, 2);
}

sg_err sg_gpu_run_delta_gates_chunk(sg_gpu *g, void *a, void *b, void *gates, void *adt, const uint32_t p[8]) {
    if (!g || !a || !b || !gates || !adt || !p) return (sg_err){"gpu: delta_gates_chunk got a NULL argument"};
    uint32_t n = p[0], n_tok = p[2];
    if (!n || !n_tok) return (sg_err){"gpu: delta_gates_chunk: bad shape"};
    sg_err e;
    uint64_t ab = (uint64_t)n * n_tok * 4;
    if (sg_failed(e = need(a, ab, "a")) || sg_failed(e = need(b, ab, "b")) ||
        sg_failed(e = need(gates, 2 * ab, "gates")) || sg_failed(e = need(adt, (uint64_t)2 * n * 4, "adt"))) return e;
    void *ins[3] = {a, b, adt}, *outs[1] = {gates};
    if (sg_failed(e = push(ins, 3))) return e;
    return finish(g, sgk_delta_gates_chunk(DEV(a), DEV(b), DEV(gates), DEV(adt), n, p[1] != 0, n_tok, g->stream),
                  outs, 1);
}

sg_err sg_gpu_run_delta_chunk(sg_gpu *g, void *S, void *qkv, void *out, void *gates, const uint32_t p[8]) {
    if (!g || !S || !qkv || !out || !gates || !p) return (sg_err){"gpu: delta_chunk got a NULL argument"};
    uint32_t dk = p[0], dv = p[1], nv = p[2], nk = p[3], kd = p[4], n_tok = p[6], cd = p[7];
    if (!dk || !dv || !nv || !nk || nv % nk || kd != nk * dk || cd < 2 * kd + nv * dv || !n_tok)
        return (sg_err){"gpu: delta_chunk: bad shape"};
    if (dk != 32 && dk != 64 && dk != 128 && dk != 256) return (sg_err){"gpu: delta_chunk: dk must be 32, 64, 128 or 256"};
    if (sg_failed(delta_scan_env())) return delta_scan_env();
    sg_err e;
    if (sg_failed(e = need(S, (uint64_t)nv * dv * dk * 4, "S")) || sg_failed(e = need(qkv, (uint64_t)n_tok * cd * 4, "qkv")) ||
        sg_failed(e = need(out, (uint64_t)n_tok * nv * dv * 4, "out")) ||
        sg_failed(e = need(gates, (uint64_t)n_tok * 2 * nv * 4, "gates"))) return e;
    void *ins[4] = {S, qkv, gates, out}, *outs[2] = {S, out};
    if (sg_failed(e = push(ins, 4))) return e;
    sgk_gdn d = {0};
    d.S = DEV(S); d.y = DEV(out); d.n_k = nk; d.n_v = nv; d.dk = dk; d.dv = dv; d.conv_dim = cd; d.tiled = p[5] != 0;
    void *ws = NULL;
    if (sg_failed(e = scratch(g, sgk_delta_ws_floats(nv, n_tok) * 4, &ws))) return e;
    return finish(g, sgk_delta_scan(&d, DEV(qkv), cd, n_tok, DEV(gates), (float *)ws, g->stream), outs, 2);
}

sg_err sg_gpu_run_rmsnorm_gated_chunk(sg_gpu *g, void *y, void *z, void *out, void *w, const uint32_t p[8]) {
    if (!g || !y || !z || !out || !w || !p) return (sg_err){"gpu: rmsnorm_gated_chunk got a NULL argument"};
    uint32_t dv = p[0], nh = p[1], n_tok = p[3];
    if (!dv || !nh || !n_tok) return (sg_err){"gpu: rmsnorm_gated_chunk: bad shape"};
    sg_err e;
    uint64_t nb = (uint64_t)n_tok * nh * dv * 4;
    if (sg_failed(e = need(y, nb, "y")) || sg_failed(e = need(z, nb, "z")) || sg_failed(e = need(out, nb, "out")) ||
        sg_failed(e = need(w, (uint64_t)dv * 4, "w"))) return e;
    void *ins[3] = {y, z, w}, *outs[1] = {out};
    if (sg_failed(e = push(ins, 3))) return e;
    return finish(g, sgk_rmsnorm_gated_rows(DEV(y), DEV(z), nh * dv, DEV(w), DEV(out), dv, nh, n_tok, fbits(p[2]),
                                            g->stream), outs, 1);
}

/* Causal chunk attention (surge.h:787-788): query token t (position base+t)
 * over cache positions 0..base+t, through the split-K kernels with the
 * prefill split policy. */
/* RoPE cos | sin per position for positions 0 .. npos-1, rd = rope_dim
 * floats each: angle and trig in double, stored f32 (reference
 * metal.m:4027-4037, ref.c:561-602). */
static void rope_table(float *t, uint32_t npos, uint32_t rd, float theta) {
    const uint32_t half = rd / 2;
    for (uint32_t p = 0; p < npos; p++)
        for (uint32_t i = 0; i < half; i++) {
            const double ang = (double)p * pow((double)theta, -2.0 * (double)i / (double)rd);
            t[(uint64_t)p * rd + i] = (float)cos(ang);
            t[(uint64_t)p * rd + half + i] = (float)sin(ang);
        }
}

sg_err sg_gpu_run_attn_prefill(sg_gpu *g, void *q, void *k, void *v, void *out, const uint32_t p[8]) {
    if (!g || !q || !k || !v || !out || !p) return (sg_err){"gpu: attn_prefill got a NULL argument"};
    uint32_t pp[8] = {p[0], p[1], p[2], 0, p[5], 0, 1, 0};
    sg_err e = attn_check(pp, false, false);
    if (sg_failed(e)) return e;
    uint32_t nh = p[0], nkv = p[1], hd = p[2], base = p[3], n = p[4], qs = p[5];
    if (!n) return (sg_err){"gpu: attn_prefill: n is zero"};
    uint64_t kvb = (uint64_t)(base + n) * nkv * hd * 2;
    if (sg_failed(e = need(q, (uint64_t)n * nh * qs * 4, "q")) || sg_failed(e = need(k, kvb, "k")) ||
        sg_failed(e = need(v, kvb, "v")) || sg_failed(e = need(out, (uint64_t)n * nh * hd * 4, "out"))) return e;
    uint64_t ah = (uint64_t)n * nh * SGK_PREFILL_SPLITS;
    uint64_t steps_b = ((uint64_t)n * sizeof(sgk_step) + 255) / 256 * 256;
    void *t;
    if (sg_failed(e = scratch(g, steps_b + ah * (2 + hd) * 4, &t))) return e;
    sgk_step *hs = malloc((uint64_t)n * sizeof *hs);
    if (!hs) return (sg_err){"gpu: out of host memory"};
    for (uint32_t z = 0; z < n; z++) { hs[z].token = 0; hs[z].pos = base + z; }
    hipError_t he = hipMemcpy(t, hs, (uint64_t)n * sizeof *hs, hipMemcpyHostToDevice);
    free(hs);
    if (he != hipSuccess) return (sg_err){"gpu: attn_prefill: descriptor upload failed"};
    void *ins[3] = {q, k, v}, *outs[1] = {out};
    if (sg_failed(e = push(ins, 3))) return e;
    float *mm = (float *)((char *)t + steps_b), *ss = mm + ah, *aa = ss + ah;
    sgk_attn A = {0};
    A.q = DEV(q); A.kc = DEV(k); A.vc = DEV(v); A.m = mm; A.s = ss; A.acc = aa; A.out = DEV(out); A.steps = t;
    A.n_heads = nh; A.n_kv = nkv; A.hd = hd; A.q_stride = qs; A.q_tok = nh * qs; A.out_tok = nh * hd;
    A.max_splits = SGK_PREFILL_SPLITS; A.ntok = n; A.scale = fbits(p[6]); A.prefill = 1;
    A.seq = base + n;
    /* The prefill path's kernel: the MFMA flash pass (deep chunks split over
     * keys and merged by the combine) for head_dim 64/128/256 with float4 q
     * rows; the split-K kernels per token otherwise. */
    if ((hd == 64 || hd == 128 || hd == 256) && qs % 4 == 0) {
        he = sgk_attn_flash(&A, g->stream);
    } else {
        he = sgk_attn_partial(&A, g->stream);
        if (he == hipSuccess) he = sgk_attn_combine(&A, g->stream);
    }
    return finish(g, he, outs, 1);
}

/* The prefill path's attention layer core over a chunk of n tokens at
 * positions base .. base+n-1, with the kernels prefill_chunk runs
 * (sgk_attn_prep: q_norm / k_norm, partial RoPE, K and V stored f16 at each
 * token's position; sgk_attn_flash: causal attention over keys 0 .. position,
 * deep chunks split over keys and merged by the combine, sigmoid output
 * gate), on caller buffers (no reference counterpart: the reference's
 * prefill runs its attention kernels per token, kernels.metal:1021-1081;
 * here they are tested whole, as one chunk):
 *   in  [n][n_heads 2 hd + 2 n_kv hd]  the input projection's rows: per
 *       query head q | gate, then k, then v (not modified);
 *   w   [2 hd]                         q_norm | k_norm;
 *   kv  [2][base + n][n_kv][hd] f16    K then V in the reference layout:
 *       positions below base given, the chunk's written;
 *   out [n][n_heads hd].
 * p: [0]=n_heads [1]=n_kv [2]=hd (64, 128 or 256) [3]=rope_dim [4]=base
 * [5]=n [6]=rope_theta bits [7]=eps bits. */
sg_err sg_gpu_run_attn_chunk(sg_gpu *g, void *in, void *w, void *kv, void *out, const uint32_t p[8]) {
    if (!g || !in || !w || !kv || !out || !p) return (sg_err){"gpu: attn_chunk got a NULL argument"};
    const uint32_t nh = p[0], nkv = p[1], hd = p[2], rd = p[3], base = p[4], n = p[5];
    if (!nh || !nkv || nh % nkv || (hd != 64 && hd != 128 && hd != 256) || rd < 2 || rd > hd || (rd & 1) || !n)
        return (sg_err){"gpu: attn_chunk: bad shape (n_heads a multiple of n_kv, hd 64/128/256, even rope_dim <= hd, n > 0)"};
    const uint64_t row = 2ull * nh * hd + 2ull * nkv * hd, cap = (uint64_t)base + n, kvh = cap * nkv * hd;
    sg_err e;
    if (sg_failed(e = need(in, n * row * 4, "in")) || sg_failed(e = need(w, 2ull * hd * 4, "w")) ||
        sg_failed(e = need(kv, 2 * kvh * 2, "kv")) || sg_failed(e = need(out, (uint64_t)n * nh * hd * 4, "out")))
        return e;
    if (overlap(out, in) || overlap(out, w) || overlap(out, kv) || overlap(kv, in) || overlap(kv, w))
        return (sg_err){"gpu: attn_chunk: buffers must not overlap"};
    void *ins[3] = {in, w, kv}, *outs[2] = {kv, out};
    if (sg_failed(e = push(ins, 3))) return e;
    /* scratch: step descriptors, the RoPE table for positions 0 .. cap-1, a
     * working copy of the rows (the prep normalises q in place) and the key
     * splits' partials */
    const uint64_t steps_b = ((uint64_t)n * sizeof(sgk_step) + 255) / 256 * 256, cs_b = (cap * rd * 4 + 255) / 256 * 256;
    const uint64_t work_b = n * row * 4, ah = (uint64_t)n * nh * SGK_PREFILL_SPLITS;
    void *t;
    if (sg_failed(e = scratch(g, steps_b + cs_b + work_b + ah * (2 + hd) * 4, &t))) return e;
    sgk_step *hs = calloc(n, sizeof *hs);
    float *ht = malloc(cap * rd * 4);
    hipError_t he = hs && ht ? hipSuccess : hipErrorOutOfMemory;
    if (he == hipSuccess) {
        for (uint32_t z = 0; z < n; z++) hs[z].pos = base + z;
        rope_table(ht, (uint32_t)cap, rd, fbits(p[6]));
        he = hipMemcpy(t, hs, (uint64_t)n * sizeof *hs, hipMemcpyHostToDevice);
        if (he == hipSuccess) he = hipMemcpy((char *)t + steps_b, ht, cap * rd * 4, hipMemcpyHostToDevice);
    }
    free(hs);
    free(ht);
    HIPCHK(he, "attn_chunk descriptors and RoPE table");
    hipStream_t s = g->stream;
    float *cs = (float *)((char *)t + steps_b), *work = (float *)((char *)t + steps_b + cs_b);
    float *mm = work + n * row, *ss = mm + ah, *aa = ss + ah;
    HIPCHK(hipMemcpyAsync(work, DEV(in), work_b, hipMemcpyDeviceToDevice, s), "attn_chunk rows");
    const float *wn = DEV(w);
    uint16_t *kc = DEV(kv);
    sgk_attn A = {0};
    A.q = work; A.kc = kc; A.vc = kc + kvh; A.m = mm; A.s = ss; A.acc = aa; A.out = DEV(out);
    A.gate = work + hd; A.steps = t; A.n_heads = nh; A.n_kv = nkv; A.hd = hd; A.rope_dim = rd;
    A.q_stride = 2 * hd; A.q_tok = (uint32_t)row; A.out_tok = nh * hd; A.max_splits = SGK_PREFILL_SPLITS;
    A.ntok = n; A.seq = (uint32_t)cap; A.scale = (float)(1.0 / sqrt((double)hd)); A.prefill = 1;
    he = sgk_attn_prep(&A, wn, wn + hd, cs, fbits(p[7]), s);
    if (he == hipSuccess) he = sgk_attn_flash(&A, s);
    return finish(g, he, outs, 2);
}

/* The online-softmax partial (surge.h:974-1050). The partial kernel here is
 * the online form already (running max, sum and accumulator rescaled across
 * key rounds), so this is the GQA one-shot: the same bytes, where the
 * reference's online kernel differs from its four-pass one in the last bits. */
sg_err sg_gpu_run_attn_splitk_partial_gqa_online(sg_gpu *g, void *q, void *k, void *v, void *m, void *s,
                                                 void *acc, const uint32_t p[8]) {
    return attn_partial_oneshot(g, q, k, v, m, s, acc, p, false);
}

/* ---------------------------------------------------------------------
 * model load
 * --------------------------------------------------------------------- */

static void mat_free(sg_gpu *g, dmat *M) {
    dfree(g, M->qs);
    dfree(g, M->d);
    dfree(g, M->dt);
    dfree(g, M->wf);
    *M = (dmat){0};
}

/* Releases the loaded model's device weights and clears every handle to
 * them, so a model loaded next (of either weight type) starts clean. */
static void model_free(sg_gpu *g) {
    for (uint32_t i = 0; g->ls && i < g->cfg.n_layers; i++) {
        glayer *L = &g->ls[i];
        mat_free(g, &L->in); mat_free(g, &L->out); mat_free(g, &L->gu); mat_free(g, &L->down);
        float *sm[] = {L->ln1, L->ln2, L->qn, L->kn, L->ssm_norm, L->conv_w, L->ssm_a, L->dt_bias};
        for (size_t k = 0; k < sizeof sm / sizeof *sm; k++) dfree(g, sm[k]);
    }
    free(g->ls);
    g->ls = NULL;
    if (!g->lm_is_emb) mat_free(g, &g->lm);
    g->lm = (dmat){0};
    mat_free(g, &g->emb);
    dfree(g, g->out_norm);
    g->out_norm = NULL;
    g->model = NULL;
}

/* gemm: the prefill GEMM also multiplies by it (a block-major scale copy). */
static sg_err mat_alloc(sg_gpu *g, dmat *M, uint32_t rows, uint32_t cols, bool gemm) {
    *M = (dmat){0};
    M->rows = rows;
    M->cols = cols;
    sg_err e;
    if (g->q8) {
        if (sg_failed(e = dalloc(g, (uint64_t)rows * cols, (void **)&M->qs))) return e;
        if (gemm && sg_failed(e = dalloc(g, (uint64_t)rows * (cols / 32) * 2, (void **)&M->dt))) return e;
        return dalloc(g, (uint64_t)rows * (cols / 32) * 2, (void **)&M->d);
    }
    return dalloc(g, (uint64_t)rows * cols * 4, (void **)&M->wf);
}

/* Uploads one [rows, cols] weight from host memory into rows row0,
 * row0+step, ... of a device matrix. */
static sg_err mat_put(sg_gpu *g, dmat *M, const void *host, uint32_t rows, uint32_t row0,
                      uint32_t step, void *stage) {
    uint32_t cols = M->cols;
    if (g->q8) {
        uint64_t raw = (uint64_t)rows * (cols / 32) * 34;
        HIPCHK(hipMemcpyAsync(stage, host, raw, hipMemcpyHostToDevice, g->stream), "weight upload");
        HIPCHK(sgk_repack_q8(stage, rows, cols, M->qs, M->d, M->dt, M->rows, row0, step, g->stream), "repack");
        HIPCHK(hipStreamSynchronize(g->stream), "repack");
        return SG_OK;
    }
    for (uint32_t r = 0; r < rows; r++)
        HIPCHK(hipMemcpy(M->wf + (uint64_t)(row0 + (uint64_t)r * step) * cols, (const float *)host + (uint64_t)r * cols,
                         (uint64_t)cols * 4, hipMemcpyHostToDevice), "weight upload");
    return SG_OK;
}

static float bf16f(uint16_t h) { uint32_t u = (uint32_t)h << 16; float f; memcpy(&f, &u, 4); return f; }

static sg_err small_put(sg_gpu *g, float **dst, const void *src, sg_tensor_type t, uint64_t n, float shift) {
    float *tmp = malloc(n * 4);
    if (!tmp) return (sg_err){"gpu: out of host memory"};
    for (uint64_t i = 0; i < n; i++)
        tmp[i] = (t == SG_T_BF16 ? bf16f(((const uint16_t *)src)[i]) : ((const float *)src)[i]) + shift;
    sg_err e = dalloc(g, n * 4, (void **)dst);
    if (!sg_failed(e) && hipMemcpy(*dst, tmp, n * 4, hipMemcpyHostToDevice) != hipSuccess)
        e = (sg_err){"gpu: small tensor upload failed"};
    free(tmp);
    return e;
}

static sg_err check_model(const sg_model *m) {
    const sg_cfg *c = &m->cfg;
    if (!m->layers || !m->tok_emb || !m->out_norm || !m->lm_head) return (sg_err){"gpu: model is missing tensors"};
    if (!c->n_layers || !c->hidden || !c->ffn_hidden || !c->vocab || !c->head_dim || !c->n_heads || !c->n_kv_heads ||
        !c->full_attn_interval)
        return (sg_err){"gpu: model config has a zero dimension"};
    if (m->wtype != SG_T_Q8_0 && m->wtype != SG_T_F32) return (sg_err){"gpu: matmul weights must be Q8_0 or F32"};
    if (c->n_heads % c->n_kv_heads || c->n_heads / c->n_kv_heads > 8) return (sg_err){"gpu: GQA group must divide and be at most 8"};
    if (c->head_dim != 16 && c->head_dim != 32 && c->head_dim != 64 && c->head_dim != 128 && c->head_dim != 256)
        return (sg_err){"gpu: head_dim must be 16, 32, 64, 128 or 256"};
    for (uint32_t i = 0; i < c->n_layers; i++) {
        bool is_attn = m->layers[i].q_proj != NULL;
        if (is_attn != ((i + 1) % c->full_attn_interval == 0))
            return (sg_err){"gpu: layer kind disagrees with full_attn_interval"};
        if (!is_attn) {
            if (!c->n_k_heads || !c->n_v_heads || c->n_v_heads % c->n_k_heads || c->conv_kernel < 1 || c->conv_kernel > 4)
                return (sg_err){"gpu: DeltaNet dims unsupported (conv_kernel 1..4, n_v multiple of n_k)"};
            if (c->head_k_dim != 32 && c->head_k_dim != 64 && c->head_k_dim != 128 && c->head_k_dim != 256)
                return (sg_err){"gpu: head_k_dim must be 32, 64, 128 or 256"};
            if (!c->head_v_dim || c->head_v_dim > SGK_GDN_MAX_DV || c->head_v_dim % 4)
                return (sg_err){"gpu: head_v_dim must be a multiple of 4 in [4, 256]"};
            if (c->n_v_heads > SGK_GATED_MAX_HEADS) return (sg_err){"gpu: at most 256 DeltaNet value heads"};
            if (c->head_v_dim > 128 && c->n_v_heads * c->head_v_dim > 8192)
                return (sg_err){"gpu: DeltaNet value_dim above 8192 needs head_v_dim <= 128"};
        } else if (c->rope_dim < 2 || c->rope_dim > c->head_dim || c->rope_dim % 2) {
            return (sg_err){"gpu: rope_dim must be even and in [2, head_dim]"};
        }
    }
    if (m->wtype == SG_T_Q8_0) {
        uint32_t w[] = { c->hidden, c->ffn_hidden, c->n_heads * c->head_dim, c->n_v_heads * c->head_v_dim };
        for (int i = 0; i < 4; i++) if (w[i] % 32) return (sg_err){"gpu: a Q8_0 matmul width is not a multiple of 32"};
    }
    return SG_OK;
}

sg_err sg_gpu_load_model(sg_gpu *g, const sg_model *m) {
    if (!g || !m) return (sg_err){"gpu: sg_gpu_load_model got a NULL argument"};
    sg_err e = check_model(m);
    if (sg_failed(e)) return e;
    if (g->have_state) state_free(g);
    model_free(g);
    const sg_cfg *c = &m->cfg;
    g->cfg = *c;
    g->q8 = m->wtype == SG_T_Q8_0;
    g->key_dim = c->n_k_heads * c->head_k_dim;
    g->value_dim = c->n_v_heads * c->head_v_dim;
    g->conv_dim = 2 * g->key_dim + g->value_dim;
    g->attn_width = c->n_heads * c->head_dim;
    g->q_width = c->attn_output_gate ? 2 * g->attn_width : g->attn_width;
    g->kv_width = c->n_kv_heads * c->head_dim;
    g->ls = calloc(c->n_layers, sizeof *g->ls);
    if (!g->ls) return (sg_err){"gpu: out of memory"};

    /* staging for the largest single weight */
    uint64_t H = c->hidden, F = c->ffn_hidden;
    uint64_t maxrows = c->vocab;
    if (F > maxrows) maxrows = F;
    uint64_t maxelems = maxrows * (H > F ? H : F);
    uint64_t big[] = { (uint64_t)g->q_width * H, (uint64_t)g->conv_dim * H, (uint64_t)g->value_dim * H, H * g->attn_width };
    for (int i = 0; i < 4; i++) if (big[i] > maxelems) maxelems = big[i];
    void *stage = NULL;
    if (g->q8 && sg_failed(e = dalloc(g, maxelems / 32 * 34 + 256, &stage))) return e;

    float sh = m->norms_are_residual ? 1.0f : 0.0f;
    for (uint32_t i = 0; i < c->n_layers && !sg_failed(e); i++) {
        const sg_layer_w *w = &m->layers[i];
        glayer *L = &g->ls[i];
        L->attn = w->q_proj != NULL;
        if (sg_failed(e = small_put(g, &L->ln1, w->ln1, m->dense_type, H, sh))) break;
        if (sg_failed(e = small_put(g, &L->ln2, w->ln2, m->dense_type, H, sh))) break;
        if (sg_failed(e = mat_alloc(g, &L->gu, 2 * c->ffn_hidden, c->hidden, true))) break;
        if (sg_failed(e = mat_put(g, &L->gu, w->gate_proj, c->ffn_hidden, 0, 2, stage))) break;
        if (sg_failed(e = mat_put(g, &L->gu, w->up_proj, c->ffn_hidden, 1, 2, stage))) break;
        if (sg_failed(e = mat_alloc(g, &L->down, c->hidden, c->ffn_hidden, true))) break;
        if (sg_failed(e = mat_put(g, &L->down, w->down_proj, c->hidden, 0, 1, stage))) break;
        if (L->attn) {
            uint32_t rows = g->q_width + 2 * g->kv_width;
            if (sg_failed(e = mat_alloc(g, &L->in, rows, c->hidden, true))) break;
            if (sg_failed(e = mat_put(g, &L->in, w->q_proj, g->q_width, 0, 1, stage))) break;
            if (sg_failed(e = mat_put(g, &L->in, w->k_proj, g->kv_width, g->q_width, 1, stage))) break;
            if (sg_failed(e = mat_put(g, &L->in, w->v_proj, g->kv_width, g->q_width + g->kv_width, 1, stage))) break;
            if (sg_failed(e = mat_alloc(g, &L->out, c->hidden, g->attn_width, true))) break;
            if (sg_failed(e = mat_put(g, &L->out, w->o_proj, c->hidden, 0, 1, stage))) break;
            if (sg_failed(e = small_put(g, &L->qn, w->q_norm, m->dense_type, c->head_dim, sh))) break;
            if (sg_failed(e = small_put(g, &L->kn, w->k_norm, m->dense_type, c->head_dim, sh))) break;
        } else {
            uint32_t nv = c->n_v_heads, rows = g->conv_dim + g->value_dim + 2 * nv;
            if (sg_failed(e = mat_alloc(g, &L->in, rows, c->hidden, true))) break;
            if (sg_failed(e = mat_put(g, &L->in, w->ssm_in_qkv, g->conv_dim, 0, 1, stage))) break;
            if (sg_failed(e = mat_put(g, &L->in, w->ssm_in_z, g->value_dim, g->conv_dim, 1, stage))) break;
            if (sg_failed(e = mat_put(g, &L->in, w->ssm_in_b, nv, g->conv_dim + g->value_dim, 1, stage))) break;
            if (sg_failed(e = mat_put(g, &L->in, w->ssm_in_a, nv, g->conv_dim + g->value_dim + nv, 1, stage))) break;
            if (sg_failed(e = mat_alloc(g, &L->out, c->hidden, g->value_dim, true))) break;
            if (sg_failed(e = mat_put(g, &L->out, w->ssm_out, c->hidden, 0, 1, stage))) break;
            if (sg_failed(e = small_put(g, &L->ssm_norm, w->ssm_norm, m->ssm_norm_type, c->head_v_dim, 0.0f))) break;
            if (sg_failed(e = small_put(g, &L->ssm_a, w->ssm_a, m->ssm_a_type, nv, 0.0f))) break;
            if (sg_failed(e = small_put(g, &L->dt_bias, w->ssm_dt_bias, m->dense_type, nv, 0.0f))) break;
            if (sg_failed(e = small_put(g, &L->conv_w, w->ssm_conv1d, m->dense_type, (uint64_t)g->conv_dim * c->conv_kernel, 0.0f))) break;
        }
    }
    if (!sg_failed(e)) e = mat_alloc(g, &g->emb, c->vocab, c->hidden, false);
    if (!sg_failed(e)) e = mat_put(g, &g->emb, m->tok_emb, c->vocab, 0, 1, stage);
    g->lm_is_emb = m->lm_head == m->tok_emb;
    if (!sg_failed(e)) {
        if (g->lm_is_emb) {
            g->lm = g->emb;
        } else {
            e = mat_alloc(g, &g->lm, c->vocab, c->hidden, false);
            if (!sg_failed(e)) e = mat_put(g, &g->lm, m->lm_head, c->vocab, 0, 1, stage);
        }
    }
    if (!sg_failed(e)) e = small_put(g, &g->out_norm, m->out_norm, m->dense_type, H, sh);
    dfree(g, stage);
    if (sg_failed(e)) { model_free(g); return e; }
    g->model = m;
    return SG_OK;
}

/* ---------------------------------------------------------------------
 * decode state and the per-token graph
 * --------------------------------------------------------------------- */

static void state_free(sg_gpu *g) {
    if (!g->have_state) return;
    if (g->g_fwd) hipGraphExecDestroy(g->g_fwd);
    if (g->g_greedy) hipGraphExecDestroy(g->g_greedy);
    g->g_fwd = g->g_greedy = NULL;
    if (g->step_ev) hipEventDestroy(g->step_ev);
    g->step_ev = NULL;
    g->step_pending = false;
    if (g->h_step) hipHostFree(g->h_step);
    if (g->h_logits) hipHostFree(g->h_logits);
    if (g->h_tok) hipHostFree(g->h_tok);
    if (g->pf_hsteps) hipHostFree(g->pf_hsteps);
    g->pf_hsteps = NULL;
    {
        void **pb[] = { (void **)&g->pf_steps, (void **)&g->pf_X, (void **)&g->pf_Xn, (void **)&g->pf_IN,
                        (void **)&g->pf_CONV, (void **)&g->pf_Y, (void **)&g->pf_G, (void **)&g->pf_CTX,
                        (void **)&g->pf_FF, (void **)&g->pf_m, (void **)&g->pf_s, (void **)&g->pf_acc,
                        (void **)&g->pf_XS, (void **)&g->pf_PART, (void **)&g->pf_WY, (void **)&g->pf_XS2 };
        for (size_t i = 0; i < sizeof pb / sizeof *pb; i++) { dfree(g, *pb[i]); *pb[i] = NULL; }
        g->pf_chunk = 0;
    }
    g->h_step = NULL;
    g->h_logits = NULL;
    g->h_tok = NULL;
    for (uint32_t i = 0; g->ls && i < g->cfg.n_layers; i++) {
        glayer *L = &g->ls[i];
        dfree(g, L->kc); dfree(g, L->vc); dfree(g, L->ring); dfree(g, L->S);
        L->kc = L->vc = NULL; L->ring = L->S = NULL;
    }
    void *bufs[] = { g->cs_table, g->x, g->act, g->ctx, g->ybuf, g->gbuf, g->ffg, g->logits, g->am, g->as,
                     g->aacc, g->amax_scratch, g->hist, g->d_step, g->gss };
    for (size_t i = 0; i < sizeof bufs / sizeof *bufs; i++) dfree(g, bufs[i]);
    g->cs_table = g->x = g->act = g->ctx = g->ybuf = g->gbuf = g->ffg = g->logits = g->am = g->as = g->aacc = NULL;
    g->amax_scratch = g->hist = NULL;
    g->gss = NULL;
    g->d_step = NULL;
    g->have_state = false;
}

/* The attention layer's split-K partial and combine of a decode step, q the
 * layer's fused q|gate|k|v projection rows. */
static hipError_t enqueue_attn(sg_gpu *g, const glayer *L, float *q) {
    const sg_cfg *c = &g->cfg;
    const uint32_t hd = c->head_dim, qs = c->attn_output_gate ? 2 * hd : hd;
    sgk_attn A = {0};
    A.q = q; A.kc = L->kc; A.vc = L->vc; A.m = g->am; A.s = g->as; A.acc = g->aacc; A.out = g->ctx;
    A.gate = c->attn_output_gate ? q + hd : NULL; A.steps = g->d_step;
    A.n_heads = c->n_heads; A.n_kv = c->n_kv_heads; A.hd = hd; A.rope_dim = c->rope_dim; A.q_stride = qs;
    A.max_splits = g->max_splits; A.ntok = 1; A.scale = (float)(1.0 / sqrt((double)hd));
    A.kv_ps = hd; A.kv_hs = (uint64_t)g->max_ctx * hd;
    A.fuse_prep = 1; A.qn = L->qn; A.kn = L->kn; A.cs = g->cs_table; A.eps = c->rms_eps;
    A.split_cap = g->attn_arm == ARM_SINGLE ? 1 : g->split_cap;
    A.per_head = g->attn_arm == ARM_PER_HEAD;
    hipError_t e = sgk_attn_partial(&A, g->stream);
    return e != hipSuccess ? e : sgk_attn_combine(&A, g->stream);
}

/* Enqueues one decode step (everything after the step descriptor is set). */
static hipError_t enqueue_step(sg_gpu *g, bool greedy) {
    const sg_cfg *c = &g->cfg;
    hipStream_t s = g->stream;
    hipError_t e;
    const int8_t *eq = g->emb.qs;
    if ((e = sgk_embed(eq, g->emb.d, g->emb.wf, c->hidden, g->d_step, 0, g->x, s)) != hipSuccess) return e;
    for (uint32_t i = 0; i < c->n_layers; i++) {
        glayer *L = &g->ls[i];
        sgk_gemv a = {0};
        a.qs = L->in.qs; a.d = L->in.d; a.wf = L->in.wf; a.rows = L->in.rows; a.cols = L->in.cols;
        a.x = g->x; a.nw = L->ln1; a.eps = c->rms_eps; a.y = g->act;
        a.pro = SGK_PRO_RMS; a.epi = SGK_EPI_STORE;
        if ((e = sgk_gemv_launch(&a, s)) != hipSuccess) return e;
        sgk_gemv o = {0};
        o.qs = L->out.qs; o.d = L->out.d; o.wf = L->out.wf; o.rows = L->out.rows; o.cols = L->out.cols;
        o.y = g->x; o.epi = SGK_EPI_ADD; o.eps = c->rms_eps;
        if (L->attn) {
            if ((e = enqueue_attn(g, L, g->act)) != hipSuccess) return e;
            o.x = g->ctx; o.pro = SGK_PRO_NONE;
        } else {
            sgk_gdn d = {0};
            d.in = g->act; d.conv_w = L->conv_w; d.ring = L->ring; d.ssm_a = L->ssm_a; d.dt_bias = L->dt_bias;
            d.S = L->S; d.y = g->ybuf; d.step = g->d_step; d.n_k = c->n_k_heads; d.n_v = c->n_v_heads;
            d.dk = c->head_k_dim; d.dv = c->head_v_dim; d.conv_dim = g->conv_dim; d.ksize = c->conv_kernel;
            d.tiled = g->model->v_heads_tiled; d.neg_exp = g->model->ssm_a_form == SG_SSM_A_NEG_EXP;
            d.z = g->act + g->conv_dim; d.norm_w = L->ssm_norm; d.out = g->gbuf; d.eps = c->rms_eps;
            d.ss = g->gss; d.blocks = g->gdn_blocks;
            if ((e = sgk_gdn_step(&d, s)) != hipSuccess) return e;
            if (g->gdn_blocks == 1) {
                o.x = g->gbuf; o.pro = SGK_PRO_NONE;          /* the step finished RMSNormGated */
            } else {                  /* each head's RMS factor applied in the out projection's prologue */
                o.x = g->gbuf; o.gss = g->gss; o.gdv = c->head_v_dim;
                o.pro = SGK_PRO_GATED;
            }
        }
        if ((e = sgk_gemv_launch(&o, s)) != hipSuccess) return e;
        sgk_gemv f = {0};
        f.qs = L->gu.qs; f.d = L->gu.d; f.wf = L->gu.wf; f.rows = L->gu.rows; f.cols = L->gu.cols;
        f.x = g->x; f.nw = L->ln2; f.eps = c->rms_eps; f.y = g->ffg; f.pro = SGK_PRO_RMS; f.epi = SGK_EPI_SWIGLU;
        if ((e = sgk_gemv_launch(&f, s)) != hipSuccess) return e;
        sgk_gemv dn = {0};
        dn.qs = L->down.qs; dn.d = L->down.d; dn.wf = L->down.wf; dn.rows = L->down.rows; dn.cols = L->down.cols;
        dn.x = g->ffg; dn.y = g->x; dn.pro = SGK_PRO_NONE; dn.epi = SGK_EPI_ADD;
        if ((e = sgk_gemv_launch(&dn, s)) != hipSuccess) return e;
    }
    sgk_gemv lm = {0};
    lm.qs = g->lm.qs; lm.d = g->lm.d; lm.wf = g->lm.wf; lm.rows = g->lm.rows; lm.cols = g->lm.cols;
    lm.x = g->x; lm.nw = g->out_norm; lm.eps = c->rms_eps; lm.y = g->logits; lm.pro = SGK_PRO_RMS; lm.epi = SGK_EPI_STORE;
    if ((e = sgk_gemv_launch(&lm, s)) != hipSuccess) return e;
    if (greedy) {
        /* next token = argmax, written straight into the descriptor, then
         * recorded and the position advanced (sgk_step_advance). */
        if ((e = sgk_argmax(g->logits, c->vocab, (uint32_t *)&g->d_step->token, g->amax_scratch, s)) != hipSuccess)
            return e;
        if ((e = sgk_step_advance(g->d_step, g->hist, s)) != hipSuccess) return e;
    }
    return hipSuccess;
}

static bool graphed(const sg_gpu *g) { return g->use_graph; }

static sg_err capture(sg_gpu *g, bool greedy, hipGraphExec_t *out) {
    hipGraph_t graph = NULL;
    HIPCHK(hipStreamBeginCapture(g->stream, hipStreamCaptureModeRelaxed), "graph capture begin");
    hipError_t le = enqueue_step(g, greedy);
    hipError_t ce = hipStreamEndCapture(g->stream, &graph);
    if (le != hipSuccess) { if (graph) hipGraphDestroy(graph); return errf("gpu: capture launch failed: %s", hipGetErrorString(le)); }
    if (ce != hipSuccess) return errf("gpu: graph capture failed: %s", hipGetErrorString(ce));
    hipError_t ie = hipGraphInstantiate(out, graph, NULL, NULL, 0);
    hipGraphDestroy(graph);
    if (ie != hipSuccess) return errf("gpu: graph instantiate failed: %s", hipGetErrorString(ie));
    return SG_OK;
}

sg_err sg_gpu_state_new(sg_gpu *g, const sg_model *m, uint32_t max_ctx) {
    if (!g || !m) return (sg_err){"gpu: sg_gpu_state_new got a NULL argument"};
    if (m != g->model) return (sg_err){"gpu: this gpu was loaded with a different sg_model"};
    if (!max_ctx || max_ctx > SG_KV_CAP_MAX) return (sg_err){"gpu: max_ctx must be in [1, 262144]"};
    state_free(g);
    /* The decode-selection switches, read here as the reference reads them
     * (surge.h:1179-1254, metal.m state_new): SURGE_KV_DTYPE f16 (default);
     * f32 names the reference's f32 cache, which is not built here, so it is
     * refused; anything else warns and keeps f16. SURGE_ATTN_SPLITK and
     * SURGE_ATTN_SPLITK_GQA: "0" turns off, anything else but "1" warns and
     * keeps the default 1. SURGE_ATTN_SPLITK_ONLINE: exactly "0" or "1", else
     * refused. */
    const char *dt_env = getenv("SURGE_KV_DTYPE");
    if (dt_env && strcmp(dt_env, "f32") == 0)
        return (sg_err){"gpu: SURGE_KV_DTYPE=f32 selects an f32 K/V cache, which this build does not have "
                        "(f16 is the only KV dtype on MI355X)"};
    if (dt_env && dt_env[0] && strcmp(dt_env, "f16") != 0)
        fprintf(stderr, "gpu: SURGE_KV_DTYPE='%s' not recognized (want f16); using f16\n", dt_env);
    bool sw[2] = {true, true};
    const char *sw_name[2] = {"SURGE_ATTN_SPLITK", "SURGE_ATTN_SPLITK_GQA"};
    for (int k = 0; k < 2; k++) {
        const char *v = getenv(sw_name[k]);
        if (v && strcmp(v, "0") == 0) sw[k] = false;
        else if (v && v[0] && strcmp(v, "1") != 0)
            fprintf(stderr, "gpu: %s='%s' not recognized (want 0 or 1); using 1\n", sw_name[k], v);
    }
    bool online = false;
    const char *on_env = getenv("SURGE_ATTN_SPLITK_ONLINE");
    if (on_env && on_env[0]) {
        if (strcmp(on_env, "1") == 0) online = true;
        else if (strcmp(on_env, "0") != 0)
            return errf("gpu: SURGE_ATTN_SPLITK_ONLINE='%s' must be exactly 0 or 1 (default 0)", on_env);
    }
    /* SURGE_SPLITK_GQA_CAP (reference surge.h:1239-1256): plain decimal digits
     * in [4, 1024], else the state is refused. Unset, the cap is the split
     * count that gives one partial workgroup per CU (CUs / n_kv_heads, within
     * [SGK_SPLIT_CAP_MIN, SGK_MAX_SPLITS]). */
    const uint32_t nkv = g->cfg.n_kv_heads ? g->cfg.n_kv_heads : 1;
    uint32_t cap = sgk_device_cus() / nkv;
    cap = cap < SGK_SPLIT_CAP_MIN ? SGK_SPLIT_CAP_MIN : cap > SGK_MAX_SPLITS ? SGK_MAX_SPLITS : cap;
    if (sg_failed(delta_scan_env())) return delta_scan_env();
    const char *cap_env = getenv("SURGE_SPLITK_GQA_CAP");
    if (cap_env && cap_env[0] != '\0') {
        uint64_t v = 0;
        const char *ch = cap_env;
        for (; *ch >= '0' && *ch <= '9' && v <= SGK_SPLIT_CAP_MAX; ch++) v = v * 10 + (uint64_t)(*ch - '0');
        if (*ch != '\0' || v < SGK_SPLIT_CAP_MIN || v > SGK_SPLIT_CAP_MAX)
            return errf("gpu: SURGE_SPLITK_GQA_CAP='%s' is not an integer in [%u, %u]", cap_env,
                        SGK_SPLIT_CAP_MIN, SGK_SPLIT_CAP_MAX);
        cap = (uint32_t)v;
    }
    const sg_cfg *c = &g->cfg;
    g->max_ctx = max_ctx;
    g->split_cap = cap;
    g->attn_splitk = sw[0];
    g->attn_gqa = sw[1];
    g->attn_online = online;
    g->n_per_head = g->n_gqa = g->n_online = 0;
    if (!g->attn_splitk) g->attn_arm = ARM_SINGLE;
    else if (sg_gpu_splitk_online_selected(g, c->n_heads, c->n_kv_heads, c->head_dim, max_ctx)) g->attn_arm = ARM_ONLINE;
    else if (sg_gpu_splitk_gqa_selected(g, c->n_heads, c->n_kv_heads, max_ctx)) g->attn_arm = ARM_GQA;
    else g->attn_arm = ARM_PER_HEAD;
    /* The DeltaNet step runs SGK_GDN_BLOCKS row-block workgroups per value
     * head, the out projection's gated prologue finishing RMSNormGated
     * (measured faster than one workgroup per head finishing it itself).
     * SURGE_GDN_BLOCKS=1 (head_v_dim <= 128) | 4 overrides. */
    g->gdn_blocks = SGK_GDN_BLOCKS;
    {
        const char *gb = getenv("SURGE_GDN_BLOCKS");
        if (gb && gb[0]) {
            if (!strcmp(gb, "4")) g->gdn_blocks = SGK_GDN_BLOCKS;
            else if (!strcmp(gb, "1") && c->head_v_dim <= 128) g->gdn_blocks = 1;
            else return errf("gpu: SURGE_GDN_BLOCKS='%s' must be 1 (head_v_dim <= 128) or 4", gb);
        }
    }
    g->max_splits = g->attn_arm == ARM_SINGLE ? 1 : sgk_n_splits_cap(max_ctx, cap);
    sg_err e = SG_OK;
    uint32_t act_rows = 0;
    for (uint32_t i = 0; i < c->n_layers; i++) if (g->ls[i].in.rows > act_rows) act_rows = g->ls[i].in.rows;
    for (uint32_t i = 0; i < c->n_layers && !sg_failed(e); i++) {
        glayer *L = &g->ls[i];
        if (L->attn) {
            uint64_t kvb = (uint64_t)max_ctx * g->kv_width * 2;
            if (!sg_failed(e = dzalloc(g, kvb, (void **)&L->kc))) e = dzalloc(g, kvb, (void **)&L->vc);
        } else {
            if (!sg_failed(e = dzalloc(g, (uint64_t)4 * g->conv_dim * 4, (void **)&L->ring)))
                e = dzalloc(g, (uint64_t)c->n_v_heads * c->head_v_dim * c->head_k_dim * 4, (void **)&L->S);
        }
    }
    uint64_t ah = (uint64_t)c->n_heads * g->max_splits;
    struct { void **p; uint64_t n; } al[] = {
        {(void **)&g->x, (uint64_t)c->hidden * 4}, {(void **)&g->act, (uint64_t)act_rows * 4},
        {(void **)&g->ctx, (uint64_t)g->attn_width * 4 + 4}, {(void **)&g->ybuf, (uint64_t)g->value_dim * 4 + 4},
        {(void **)&g->gbuf, (uint64_t)g->value_dim * 4 + 4},
        {(void **)&g->ffg, (uint64_t)c->ffn_hidden * 4}, {(void **)&g->logits, (uint64_t)c->vocab * 4},
        {(void **)&g->am, ah * 4}, {(void **)&g->as, ah * 4}, {(void **)&g->aacc, ah * c->head_dim * 4},
        {(void **)&g->amax_scratch, 4096}, {(void **)&g->hist, ((uint64_t)max_ctx + 2) * 4},
        {(void **)&g->gss, (uint64_t)c->n_v_heads * SGK_GDN_BLOCKS * 4 + 4},
        {(void **)&g->d_step, sizeof(sgk_step)},
    };
    for (size_t i = 0; i < sizeof al / sizeof *al && !sg_failed(e); i++) e = dzalloc(g, al[i].n, al[i].p);
    /* RoPE cos|sin per position, angle and trig in double, stored f32
     * (reference metal.m:4027-4037, ref.c:561-602). */
    uint32_t rd = c->rope_dim ? c->rope_dim : 2;
    if (!sg_failed(e)) e = dalloc(g, (uint64_t)max_ctx * rd * 4, (void **)&g->cs_table);
    if (!sg_failed(e)) {
        float *t = malloc((uint64_t)max_ctx * rd * 4);
        if (!t) e = (sg_err){"gpu: out of host memory"};
        else {
            rope_table(t, max_ctx, rd, c->rope_theta);
            if (hipMemcpy(g->cs_table, t, (uint64_t)max_ctx * rd * 4, hipMemcpyHostToDevice) != hipSuccess)
                e = (sg_err){"gpu: RoPE table upload failed"};
            free(t);
        }
    }
    if (!sg_failed(e) && hipHostMalloc((void **)&g->h_step, sizeof(sgk_step), 0) != hipSuccess) e = (sg_err){"gpu: hipHostMalloc failed"};
    if (!sg_failed(e) && hipHostMalloc((void **)&g->h_logits, (uint64_t)c->vocab * 4, 0) != hipSuccess) e = (sg_err){"gpu: hipHostMalloc failed"};
    if (!sg_failed(e) && hipHostMalloc((void **)&g->h_tok, ((uint64_t)max_ctx + 2) * 4, 0) != hipSuccess) e = (sg_err){"gpu: hipHostMalloc failed"};
    if (!sg_failed(e) && hipEventCreateWithFlags(&g->step_ev, hipEventDisableTiming) != hipSuccess)
        e = (sg_err){"gpu: hipEventCreate failed"};
    g->have_state = true;
    if (!sg_failed(e) && graphed(g)) {
        e = capture(g, false, &g->g_fwd);
        if (!sg_failed(e)) e = capture(g, true, &g->g_greedy);
    }
    if (sg_failed(e)) { state_free(g); return e; }
    g->used = 0;
    return SG_OK;
}

void sg_gpu_state_reset(sg_gpu *g) {
    if (!g || !g->have_state) return;
    hipStreamSynchronize(g->stream);
    const sg_cfg *c = &g->cfg;
    for (uint32_t i = 0; i < c->n_layers; i++) {
        glayer *L = &g->ls[i];
        if (L->ring) sgk_fill_f32(L->ring, 0.0f, (uint64_t)4 * g->conv_dim, g->stream);
        if (L->S) sgk_fill_f32(L->S, 0.0f, (uint64_t)c->n_v_heads * c->head_v_dim * c->head_k_dim, g->stream);
    }
    hipStreamSynchronize(g->stream);
    g->used = 0;
}

uint32_t sg_gpu_used(const sg_gpu *g) { return (g && g->have_state) ? g->used : 0; }

static sg_err step_checks(sg_gpu *g, const sg_model *m, int32_t token, uint32_t pos) {
    if (!g || !m) return (sg_err){"gpu: sg_gpu_forward got a NULL argument"};
    if (!g->have_state) return (sg_err){"gpu: call sg_gpu_state_new first"};
    if (m != g->model) return (sg_err){"gpu: this gpu was loaded with a different sg_model"};
    if (token < 0 || (uint32_t)token >= g->cfg.vocab) return (sg_err){"gpu: token id out of range"};
    if (pos >= g->max_ctx) return (sg_err){"gpu: position exceeds max_ctx"};
    if (pos != g->used) return (sg_err){"gpu: positions must be presented in order"};
    return SG_OK;
}

static uint32_t n_attn_layers(const sg_gpu *g) {
    uint32_t n = 0;
    for (uint32_t i = 0; i < g->cfg.n_layers; i++) n += g->ls[i].attn;
    return n;
}

/* Writes the pinned step descriptor and queues its upload. The previous
 * upload of the same pinned bytes may not have run yet (forward_nosync and
 * the greedy loop return without waiting), so the write waits for it. */
static sg_err step_upload(sg_gpu *g, int32_t token, uint32_t pos) {
    if (g->step_pending) HIPCHK(hipEventSynchronize(g->step_ev), "previous step upload");
    g->h_step->token = token;
    g->h_step->pos = pos;
    HIPCHK(hipMemcpyAsync(g->d_step, g->h_step, sizeof(sgk_step), hipMemcpyHostToDevice, g->stream), "step upload");
    HIPCHK(hipEventRecord(g->step_ev, g->stream), "step upload event");
    g->step_pending = true;
    return SG_OK;
}

/* Counts what one decode step encodes: one partial per attention layer, in
 * the counter of the state's arm (the single-pass arm counts in neither). */
static void count_step(sg_gpu *g, uint64_t steps) {
    const uint64_t n = steps * n_attn_layers(g);
    if (g->attn_arm == ARM_PER_HEAD) g->n_per_head += n;
    else if (g->attn_arm == ARM_GQA) g->n_gqa += n;
    else if (g->attn_arm == ARM_ONLINE) g->n_online += n;
}

static sg_err launch_step(sg_gpu *g, int32_t token, uint32_t pos, bool greedy) {
    sg_err se = step_upload(g, token, pos);
    if (sg_failed(se)) return se;
    count_step(g, 1);
    if (graphed(g)) {
        HIPCHK(hipGraphLaunch(greedy ? g->g_greedy : g->g_fwd, g->stream), "graph launch");
    } else {
        hipError_t e = enqueue_step(g, greedy);
        if (e != hipSuccess) return errf("gpu: decode step launch failed: %s", hipGetErrorString(e));
    }
    return SG_OK;
}

sg_err sg_gpu_forward(sg_gpu *g, const sg_model *m, int32_t token, uint32_t pos, const float **logits) {
    sg_err e = step_checks(g, m, token, pos);
    if (sg_failed(e)) return e;
    if (sg_failed(e = launch_step(g, token, pos, false))) return e;
    HIPCHK(hipMemcpyAsync(g->h_logits, g->logits, (uint64_t)g->cfg.vocab * 4, hipMemcpyDeviceToHost, g->stream), "logits download");
    HIPCHK(hipStreamSynchronize(g->stream), "decode step");
    g->used = pos + 1;
    if (logits) *logits = g->h_logits;
    return SG_OK;
}

sg_err sg_gpu_forward_nosync(sg_gpu *g, const sg_model *m, int32_t token, uint32_t pos) {
    sg_err e = step_checks(g, m, token, pos);
    if (sg_failed(e)) return e;
    if (sg_failed(e = launch_step(g, token, pos, false))) return e;
    g->used = pos + 1;
    return SG_OK;
}

sg_err sg_gpu_sync(sg_gpu *g) {
    if (!g) return (sg_err){"gpu: NULL gpu"};
    HIPCHK(hipStreamSynchronize(g->stream), "stream synchronize");
    return SG_OK;
}

sg_err sg_gpu_argmax(sg_gpu *g, uint32_t *token_out) {
    if (!g || !token_out || !g->have_state) return (sg_err){"gpu: sg_gpu_argmax needs a live state"};
    HIPCHK(sgk_argmax(g->logits, g->cfg.vocab, g->hist + g->max_ctx + 1, g->amax_scratch, g->stream), "argmax");
    HIPCHK(hipMemcpyAsync(g->h_tok, g->hist + g->max_ctx + 1, 4, hipMemcpyDeviceToHost, g->stream), "argmax download");
    HIPCHK(hipStreamSynchronize(g->stream), "argmax");
    *token_out = g->h_tok[0];
    return SG_OK;
}

/* Device-resident greedy decode (no reference counterpart): feeds `token` at
 * position `pos`, then n_steps-1 more tokens each chosen on the device by
 * argmax, with no host round trip in between. out_tokens receives the n
 * argmax tokens (the token after each step). */
sg_err sg_gpu_decode_greedy(sg_gpu *g, const sg_model *m, int32_t token, uint32_t pos,
                            uint32_t n_steps, int32_t *out_tokens) {
    sg_err e = step_checks(g, m, token, pos);
    if (sg_failed(e)) return e;
    if (!n_steps || (uint64_t)pos + n_steps > g->max_ctx) return (sg_err){"gpu: greedy decode runs past max_ctx"};
    if (sg_failed(e = step_upload(g, token, pos))) return e;
    count_step(g, n_steps);
    for (uint32_t i = 0; i < n_steps; i++) {
        if (graphed(g)) {
            HIPCHK(hipGraphLaunch(g->g_greedy, g->stream), "graph launch");
        } else {
            hipError_t he = enqueue_step(g, true);
            if (he != hipSuccess) return errf("gpu: decode step launch failed: %s", hipGetErrorString(he));
        }
    }
    HIPCHK(hipMemcpyAsync(g->h_tok, g->hist + pos + 1, (uint64_t)n_steps * 4, hipMemcpyDeviceToHost, g->stream), "tokens download");
    HIPCHK(hipStreamSynchronize(g->stream), "greedy decode");
    if (out_tokens) memcpy(out_tokens, g->h_tok, (uint64_t)n_steps * 4);
    g->used = pos + n_steps;
    return SG_OK;
}

/* sg_gpu_decode_greedy with per-token timestamps (no reference counterpart):
 * t_cum[i] = seconds from just before the first step to the end of step i,
 * from HIP events recorded between the steps on the GPU's clock, the series
 * surge-bench fits by slope (sg_bench_slope, reference cli_bench.c:627-693)
 * without a host round trip per token. */
sg_err sg_gpu_decode_greedy_timed(sg_gpu *g, const sg_model *m, int32_t token, uint32_t pos, uint32_t n_steps,
                                  int32_t *out_tokens, double *t_cum) {
    sg_err e = step_checks(g, m, token, pos);
    if (sg_failed(e)) return e;
    if (!t_cum || !n_steps || (uint64_t)pos + n_steps > g->max_ctx)
        return (sg_err){"gpu: timed greedy decode needs t_cum and must stay within max_ctx"};
    hipEvent_t *ev = calloc((size_t)n_steps + 1, sizeof *ev);
    if (!ev) return (sg_err){"gpu: out of host memory"};
    hipError_t he = hipSuccess;
    for (uint32_t i = 0; i <= n_steps && he == hipSuccess; i++) he = hipEventCreate(&ev[i]);
    if (he == hipSuccess && sg_failed(e = step_upload(g, token, pos))) he = hipErrorUnknown;
    if (he == hipSuccess) he = hipEventRecord(ev[0], g->stream);
    for (uint32_t i = 0; i < n_steps && he == hipSuccess; i++) {
        he = graphed(g) ? hipGraphLaunch(g->g_greedy, g->stream) : enqueue_step(g, true);
        if (he == hipSuccess) he = hipEventRecord(ev[i + 1], g->stream);
    }
    if (he == hipSuccess)
        he = hipMemcpyAsync(g->h_tok, g->hist + pos + 1, (uint64_t)n_steps * 4, hipMemcpyDeviceToHost, g->stream);
    if (he == hipSuccess) he = hipStreamSynchronize(g->stream);
    for (uint32_t i = 0; i < n_steps && he == hipSuccess; i++) {
        float ms = 0.0f;
        he = hipEventElapsedTime(&ms, ev[0], ev[i + 1]);
        t_cum[i] = (double)ms * 1e-3;
    }
    for (uint32_t i = 0; i <= n_steps; i++) if (ev[i]) hipEventDestroy(ev[i]);
    free(ev);
    if (sg_failed(e)) return e;
    if (he != hipSuccess) return errf("gpu: timed greedy decode: %s", hipGetErrorString(he));
    count_step(g, n_steps);
    if (out_tokens) memcpy(out_tokens, g->h_tok, (uint64_t)n_steps * 4);
    g->used = pos + n_steps;
    return SG_OK;
}

sg_err sg_gpu_state_fill_synthetic(sg_gpu *g, uint32_t n_tokens, uint32_t seed) {
    if (!g || !g->have_state) return (sg_err){"gpu: sg_gpu_state_fill_synthetic needs a live state"};
    if (n_tokens >= g->max_ctx) return (sg_err){"gpu: sg_gpu_state_fill_synthetic: n_tokens must be < max_ctx"};
    const sg_cfg *c = &g->cfg;
    hipStream_t s = g->stream;
    HIPCHK(hipStreamSynchronize(s), "fill: previous work");
    const uint32_t nkv = c->n_kv_heads, hd = c->head_dim;
    for (uint32_t i = 0; i < c->n_layers; i++) {
        glayer *L = &g->ls[i];
        const uint32_t ls = seed * 2654435761u + 97u * i;
        if (L->attn) {
            /* head-major [n_kv][max_ctx][hd]: head h's first n_tokens rows are contiguous */
            for (uint32_t h = 0; h < nkv; h++) {
                const uint64_t off = (uint64_t)h * g->max_ctx * hd, n = (uint64_t)n_tokens * hd;
                HIPCHK(sgk_fill_hash((uint16_t *)L->kc + off, n, 1, ls + 2 * h, 2.0f, s), "fill K");
                HIPCHK(sgk_fill_hash((uint16_t *)L->vc + off, n, 1, ls + 2 * h + 1, 2.0f, s), "fill V");
            }
        } else {
            HIPCHK(sgk_fill_hash(L->S, (uint64_t)c->n_v_heads * c->head_v_dim * c->head_k_dim, 0, ls + 7, 0.05f, s),
                   "fill S");
            HIPCHK(sgk_fill_hash(L->ring, (uint64_t)4 * g->conv_dim, 0, ls + 11, 0.05f, s), "fill ring");
        }
    }
    HIPCHK(hipStreamSynchronize(s), "fill");
    g->used = n_tokens;
    return SG_OK;
}

/* ---------------------------------------------------------------------
 * prefill (surge.h:1276-1309)
 * --------------------------------------------------------------------- */

/* Chunk scratch, sized for `chunk` tokens on first use (and regrown). */
static sg_err prefill_alloc(sg_gpu *g, uint32_t chunk) {
    if (g->pf_chunk >= chunk) return SG_OK;
    void **bufs[] = { (void **)&g->pf_steps, (void **)&g->pf_X, (void **)&g->pf_Xn, (void **)&g->pf_IN,
                      (void **)&g->pf_CONV, (void **)&g->pf_Y, (void **)&g->pf_G, (void **)&g->pf_CTX,
                      (void **)&g->pf_FF, (void **)&g->pf_m, (void **)&g->pf_s, (void **)&g->pf_acc,
                      (void **)&g->pf_XS, (void **)&g->pf_PART, (void **)&g->pf_WY, (void **)&g->pf_XS2 };
    for (size_t i = 0; i < sizeof bufs / sizeof *bufs; i++) { dfree(g, *bufs[i]); *bufs[i] = NULL; }
    if (g->pf_hsteps) { hipHostFree(g->pf_hsteps); g->pf_hsteps = NULL; }
    g->pf_chunk = 0;
    const sg_cfg *c = &g->cfg;
    uint32_t in_rows = 0;
    for (uint32_t i = 0; i < c->n_layers; i++) if (g->ls[i].in.rows > in_rows) in_rows = g->ls[i].in.rows;
    uint64_t n = chunk, ah = n * c->n_heads * SGK_PREFILL_SPLITS;
    uint64_t kmax = c->hidden;                      /* widest GEMM input row */
    if (c->ffn_hidden > kmax) kmax = c->ffn_hidden;
    if (g->attn_width > kmax) kmax = g->attn_width;
    if (g->value_dim > kmax) kmax = g->value_dim;
    uint64_t sizes[] = { n * sizeof(sgk_step), n * c->hidden * 4, n * c->hidden * 4, n * in_rows * 4,
                         n * g->conv_dim * 4 + 4, n * g->value_dim * 4 + 4, n * g->value_dim * 4 + 4,
                         n * g->attn_width * 4 + 4, n * c->ffn_hidden * 4, ah * 4, ah * 4, ah * c->head_dim * 4,
                         n * kmax * 4, 4 * n * c->hidden * 4, sgk_delta_ws_floats(c->n_v_heads, chunk) * 4 + 4,
                         n * kmax * 4 };
    sg_err e = SG_OK;
    for (size_t i = 0; i < sizeof bufs / sizeof *bufs && !sg_failed(e); i++) e = dzalloc(g, sizes[i], bufs[i]);
    if (!sg_failed(e) && hipHostMalloc((void **)&g->pf_hsteps, n * sizeof(sgk_step), 0) != hipSuccess)
        e = (sg_err){"gpu: hipHostMalloc failed"};
    if (sg_failed(e)) return e;
    g->pf_chunk = chunk;
    return SG_OK;
}

/* Y = X W^T with the GEMM epilogue `epi`. post_nw (SGK_EPI_ADD only): the
 * next product over Y's rows takes RMSNorm(Y) with this weight on Q8
 * weights; when this product splits K its reduce writes that split into
 * pf_XS and sets *ready, and the next call passes it on (gemm_rows_norm). */
static hipError_t gemm_rows_x(sg_gpu *g, const dmat *M, const float *X, uint32_t ldx, float *Y, uint32_t ldy,
                              uint32_t n, int epi, const float *post_nw, int *ready, int xs_ready, uint16_t *xs) {
    sgk_gemm_args a = { X, M->qs, M->dt, M->wf, Y, n, M->rows, M->cols, ldx, ldy, epi, xs, g->pf_PART,
                        (uint64_t)4 * g->pf_chunk * g->cfg.hidden, NULL, 0.0f, xs_ready, post_nw, g->cfg.rms_eps,
                        post_nw ? ready : NULL, NULL };
    if (ready) *ready = 0;
    return sgk_gemm(&a, g->stream);
}

static hipError_t gemm_rows(sg_gpu *g, const dmat *M, const float *X, uint32_t ldx, float *Y, uint32_t ldy,
                            uint32_t n, int epi, const float *post_nw, int *ready) {
    return gemm_rows_x(g, M, X, ldx, Y, ldy, n, epi, post_nw, ready, 0, g->pf_XS);
}

/* RMSNorm(X) (weight nw) then the GEMM: Q8 weights take the norm inside the
 * GEMM's bf16 split (one pass over X), or find it in pf_XS already when
 * xs_ready (written by the previous product's reduce); f32 weights normalise
 * into pf_Xn. */
static hipError_t gemm_rows_norm_x(sg_gpu *g, const dmat *M, const float *X, const float *nw, float *Y,
                                   uint32_t ldy, uint32_t n, int epi, int xs_ready, uint16_t *xs, uint16_t *ys) {
    const uint32_t H = g->cfg.hidden;
    if (!M->qs || !nw) {
        hipError_t e = sgk_rmsnorm_heads(X, nw, g->pf_Xn, H, n, H, g->cfg.rms_eps, g->stream);
        return e != hipSuccess ? e : gemm_rows(g, M, g->pf_Xn, H, Y, ldy, n, epi, NULL, NULL);
    }
    sgk_gemm_args a = { X, M->qs, M->dt, M->wf, Y, n, M->rows, M->cols, H, ldy, epi, xs, g->pf_PART,
                        (uint64_t)4 * g->pf_chunk * H, nw, g->cfg.rms_eps, xs_ready, NULL, 0.0f, NULL, ys };
    return sgk_gemm(&a, g->stream);
}

static hipError_t gemm_rows_norm(sg_gpu *g, const dmat *M, const float *X, const float *nw, float *Y,
                                 uint32_t ldy, uint32_t n, int epi, int xs_ready) {
    return gemm_rows_norm_x(g, M, X, nw, Y, ldy, n, epi, xs_ready, g->pf_XS, NULL);
}

static sg_err timed(sg_gpu *g, hipEvent_t a, hipEvent_t b, uint32_t reps, double *us);

sg_err sg_gpu_time_gemm(sg_gpu *g, uint32_t layer, uint32_t which, uint32_t n, uint32_t reps, double *us) {
    if (!g || !g->have_state || !us || !reps || !n) return (sg_err){"gpu: sg_gpu_time_gemm got an invalid argument"};
    const sg_cfg *c = &g->cfg;
    if (layer >= c->n_layers || which > 3) return (sg_err){"gpu: sg_gpu_time_gemm: layer or which out of range"};
    sg_err e = prefill_alloc(g, n);
    if (sg_failed(e)) return e;
    hipStream_t s = g->stream;
    const glayer *L = &g->ls[layer];
    const uint32_t H = c->hidden, ow = L->attn ? g->attn_width : g->value_dim;
    float *ox = L->attn ? g->pf_CTX : g->pf_Y;          /* the output projection's input rows */
    hipError_t he = sgk_fill_hash(g->pf_X, (uint64_t)n * H, 0, 11, 1.0f, s);
    if (he == hipSuccess) he = sgk_fill_hash(g->pf_FF, (uint64_t)n * c->ffn_hidden, 0, 12, 1.0f, s);
    if (he == hipSuccess) he = sgk_fill_hash(ox, (uint64_t)n * ow, 0, 13, 1.0f, s);
    hipEvent_t a = NULL, b = NULL;
    if (he == hipSuccess) he = hipEventCreate(&a);
    if (he == hipSuccess) he = hipEventCreate(&b);
    for (uint32_t r = 0; r < reps + 1 && he == hipSuccess; r++) {      /* product 0 warms up, untimed */
        if (r == 1) he = hipEventRecord(a, s);
        if (he != hipSuccess) break;
        switch (which) {
        case 0: he = gemm_rows_norm(g, &L->in, g->pf_X, L->ln1, g->pf_IN, L->in.rows, n, SGK_EPI_STORE, 0); break;
        case 1: he = gemm_rows(g, &L->out, ox, ow, g->pf_X, H, n, SGK_EPI_ADD, NULL, NULL); break;
        case 2: he = gemm_rows_norm(g, &L->gu, g->pf_X, L->ln2, g->pf_FF, c->ffn_hidden, n, SGK_EPI_SWIGLU, 0); break;
        default: he = gemm_rows(g, &L->down, g->pf_FF, c->ffn_hidden, g->pf_X, H, n, SGK_EPI_ADD, NULL, NULL); break;
        }
    }
    if (he == hipSuccess) he = hipEventRecord(b, s);
    if (he == hipSuccess) e = timed(g, a, b, reps, us);
    else e = errf("gpu: sg_gpu_time_gemm: %s", hipGetErrorString(he));
    hipStreamSynchronize(s);
    if (a) hipEventDestroy(a);
    if (b) hipEventDestroy(b);
    return e;
}

/* One chunk of n tokens at positions base..base+n-1 through every layer. */
static hipError_t prefill_chunk(sg_gpu *g, uint32_t base, uint32_t n) {
    const sg_cfg *c = &g->cfg;
    hipStream_t s = g->stream;
    hipError_t e;
    const uint32_t H = c->hidden, hd = c->head_dim, qs = c->attn_output_gate ? 2 * hd : hd;
    if ((e = sgk_embed_rows(g->emb.qs, g->emb.d, g->emb.wf, H, g->pf_steps, n, g->pf_X, s)) != hipSuccess) return e;
    /* ready: rxs holds the next product's normed split (written by the reduce
     * of the product before). Splits go to pf_XS, except the down projection's
     * input, which gate/up writes into pf_XS2 (it reads pf_XS meanwhile), and
     * what the down projection's reduce writes into its own split, pf_XS2. */
    int ready = 0;
    uint16_t *rxs = g->pf_XS;
    for (uint32_t i = 0; i < c->n_layers; i++) {
        glayer *L = &g->ls[i];
        const glayer *Ln = i + 1 < c->n_layers ? &g->ls[i + 1] : NULL;
        const uint32_t in_rows = L->in.rows;
        if ((e = gemm_rows_norm_x(g, &L->in, g->pf_X, L->ln1, g->pf_IN, in_rows, n, SGK_EPI_STORE, ready,
                                  ready ? rxs : g->pf_XS, NULL)) != hipSuccess)
            return e;
        if (L->attn) {
            sgk_attn A = {0};
            A.q = g->pf_IN; A.kc = L->kc; A.vc = L->vc; A.m = g->pf_m; A.s = g->pf_s; A.acc = g->pf_acc;
            A.out = g->pf_CTX; A.gate = c->attn_output_gate ? g->pf_IN + hd : NULL; A.steps = g->pf_steps;
            A.n_heads = c->n_heads; A.n_kv = c->n_kv_heads; A.hd = hd; A.rope_dim = c->rope_dim; A.q_stride = qs;
            A.q_tok = in_rows; A.out_tok = g->attn_width; A.max_splits = SGK_PREFILL_SPLITS; A.ntok = n;
            A.seq = base + n;       /* keys of the chunk's last token: the flash pass splits deep chunks */
            A.scale = (float)(1.0 / sqrt((double)hd)); A.prefill = 1;
            A.kv_ps = hd; A.kv_hs = (uint64_t)g->max_ctx * hd;
            if ((e = sgk_attn_prep(&A, L->qn, L->kn, g->cs_table, c->rms_eps, s)) != hipSuccess) return e;
            if (hd == 64 || hd == 128 || hd == 256) {
                if ((e = sgk_attn_flash(&A, s)) != hipSuccess) return e;
            } else {
                if ((e = sgk_attn_partial(&A, s)) != hipSuccess) return e;
                if ((e = sgk_attn_combine(&A, s)) != hipSuccess) return e;
            }
            if ((e = gemm_rows(g, &L->out, g->pf_CTX, g->attn_width, g->pf_X, H, n, SGK_EPI_ADD, L->gu.qs ? L->ln2 : NULL,
                               &ready)) != hipSuccess)
                return e;
            rxs = g->pf_XS;
        } else {
            sgk_gdn d = {0};
            d.in = g->pf_IN; d.conv_w = L->conv_w; d.ring = L->ring; d.ssm_a = L->ssm_a; d.dt_bias = L->dt_bias;
            d.S = L->S; d.y = g->pf_Y; d.step = g->pf_steps; d.n_k = c->n_k_heads; d.n_v = c->n_v_heads;
            d.dk = c->head_k_dim; d.dv = c->head_v_dim; d.conv_dim = g->conv_dim; d.ksize = c->conv_kernel;
            d.tiled = g->model->v_heads_tiled; d.neg_exp = g->model->ssm_a_form == SG_SSM_A_NEG_EXP;
            if ((e = sgk_gdn_chunk(&d, g->pf_CONV, in_rows, n, g->pf_WY, s)) != hipSuccess) return e;
            /* RMSNormGated; with Q8 output weights written straight as their GEMM's bf16 split */
            const int gsplit = L->out.qs != NULL;
            if (gsplit) e = sgk_rmsnorm_gated_split(g->pf_Y, g->pf_IN + g->conv_dim, in_rows, L->ssm_norm, g->pf_XS,
                                                    c->head_v_dim, c->n_v_heads, n, c->rms_eps, s);
            else e = sgk_rmsnorm_gated_rows(g->pf_Y, g->pf_IN + g->conv_dim, in_rows, L->ssm_norm, g->pf_G,
                                            c->head_v_dim, c->n_v_heads, n, c->rms_eps, s);
            if (e != hipSuccess) return e;
            if ((e = gemm_rows_x(g, &L->out, g->pf_G, g->value_dim, g->pf_X, H, n, SGK_EPI_ADD,
                                 L->gu.qs ? L->ln2 : NULL, &ready, gsplit, g->pf_XS)) != hipSuccess)
                return e;
            rxs = g->pf_XS;
        }
        /* gate/up with Q8 down weights writes its SwiGLU output as the down projection's split */
        uint16_t *ys = L->gu.qs && L->down.qs ? g->pf_XS2 : NULL;
        if ((e = gemm_rows_norm_x(g, &L->gu, g->pf_X, L->ln2, g->pf_FF, c->ffn_hidden, n, SGK_EPI_SWIGLU, ready,
                                  ready ? rxs : g->pf_XS, ys)) != hipSuccess)
            return e;
        if ((e = gemm_rows_x(g, &L->down, g->pf_FF, c->ffn_hidden, g->pf_X, H, n, SGK_EPI_ADD,
                             Ln && Ln->in.qs ? Ln->ln1 : NULL, &ready, ys != NULL, ys ? ys : g->pf_XS)) != hipSuccess)
            return e;
        rxs = ys ? ys : g->pf_XS;
    }
    return hipSuccess;
}

/* Chunked prompt ingest (surge.h:1276-1309): every projection of a chunk is
 * one MFMA GEMM; attention is one MFMA pass per (64-token block, head) over
 * the causal prefix (head_dim 64/128/256; other sizes run the decode split-K
 * kernels per token); the DeltaNet conv and delta
 * rule scan the chunk in order with the state threaded through, exactly as
 * decode would. Only the last row gets out_norm + lm_head. */
sg_err sg_gpu_prefill(sg_gpu *g, const sg_model *m, const int32_t *tokens, uint32_t n_tokens,
                      uint32_t chunk_size, const float **out_last_logits) {
    if (!g || !m || !tokens) return (sg_err){"gpu: sg_gpu_prefill got a NULL argument"};
    if (!g->have_state) return (sg_err){"gpu: call sg_gpu_state_new first"};
    if (m != g->model) return (sg_err){"gpu: this gpu was loaded with a different sg_model"};
    if (!n_tokens || n_tokens > g->max_ctx) return (sg_err){"gpu: n_tokens must be in [1, max_ctx]"};
    if (sg_failed(delta_scan_env())) return delta_scan_env();
    for (uint32_t i = 0; i < n_tokens; i++)
        if (tokens[i] < 0 || (uint32_t)tokens[i] >= g->cfg.vocab) return (sg_err){"gpu: token id out of range"};
    uint32_t chunk = chunk_size ? chunk_size : SG_PREFILL_CHUNK_DEFAULT;
    if (chunk > n_tokens) chunk = n_tokens;
    sg_err e = prefill_alloc(g, chunk);
    if (sg_failed(e)) return e;
    sg_gpu_state_reset(g);
    g->pf_segments = 0;
    for (uint32_t base = 0; base < n_tokens; base += chunk) {
        uint32_t n = n_tokens - base < chunk ? n_tokens - base : chunk;
        for (uint32_t z = 0; z < n; z++) {
            g->pf_hsteps[z].token = tokens[base + z];
            g->pf_hsteps[z].pos = base + z;
        }
        HIPCHK(hipMemcpyAsync(g->pf_steps, g->pf_hsteps, (uint64_t)n * sizeof(sgk_step), hipMemcpyHostToDevice,
                              g->stream), "chunk descriptors");
        hipError_t he = prefill_chunk(g, base, n);
        if (he != hipSuccess) return errf("gpu: prefill launch failed: %s", hipGetErrorString(he));
        if (base + n >= n_tokens) {
            sgk_gemv lm = {0};
            lm.qs = g->lm.qs; lm.d = g->lm.d; lm.wf = g->lm.wf; lm.rows = g->lm.rows; lm.cols = g->lm.cols;
            lm.x = g->pf_X + (uint64_t)(n - 1) * g->cfg.hidden; lm.nw = g->out_norm; lm.eps = g->cfg.rms_eps;
            lm.y = g->logits; lm.pro = SGK_PRO_RMS; lm.epi = SGK_EPI_STORE;
            HIPCHK(sgk_gemv_launch(&lm, g->stream), "lm_head");
            HIPCHK(hipMemcpyAsync(g->h_logits, g->logits, (uint64_t)g->cfg.vocab * 4, hipMemcpyDeviceToHost,
                                  g->stream), "logits download");
        }
        /* the pinned descriptor buffer is reused by the next chunk */
        HIPCHK(hipStreamSynchronize(g->stream), "prefill chunk");
        g->pf_segments++;
    }
    g->used = n_tokens;
    if (out_last_logits) *out_last_logits = g->h_logits;
    return SG_OK;
}

void sg_gpu_set_prefill_rest(sg_gpu *g, uint32_t work_budget_ms, uint32_t rest_ms) {
    (void)g; (void)work_budget_ms; (void)rest_ms;
}
uint64_t sg_gpu_prefill_rest_ms(const sg_gpu *g) { (void)g; return 0; }
void sg_gpu_set_prefill_max_burst(sg_gpu *g, uint32_t max_burst_ms) { (void)g; (void)max_burst_ms; }
uint64_t sg_gpu_prefill_segments(const sg_gpu *g) { return g ? g->pf_segments : 0; }

/* ---------------------------------------------------------------------
 * measurement hooks (no reference counterpart)
 * --------------------------------------------------------------------- */

void *sg_gpu_stream(const sg_gpu *g) { return g ? (void *)g->stream : NULL; }

/* Enqueues (asynchronously, on the library stream) exactly one of the decode
 * step's GEMV launches for `layer`, against the live state's activation
 * buffers: which = 0 input projection, 1 output projection, 2 gate/up,
 * 3 down, 4 lm_head (layer ignored). Used to time one kernel in isolation
 * with events on sg_gpu_stream; it mutates the activation buffers. */
sg_err sg_gpu_enqueue_gemv(sg_gpu *g, uint32_t layer, uint32_t which) {
    return sg_gpu_enqueue_gemv_tuned(g, layer, which, 0, 0);
}

sg_err sg_gpu_enqueue_gemv_tuned(sg_gpu *g, uint32_t layer, uint32_t which, uint32_t tune_r, uint32_t tune_blocks) {
    if (!g || !g->have_state) return (sg_err){"gpu: sg_gpu_enqueue_gemv needs a live state"};
    if (which != 4 && layer >= g->cfg.n_layers) return (sg_err){"gpu: layer out of range"};
    const sg_cfg *c = &g->cfg;
    sgk_gemv a = {0};
    const dmat *M;
    a.eps = c->rms_eps;
    if (which == 4) {
        M = &g->lm;
        a.x = g->x; a.nw = g->out_norm; a.y = g->logits; a.pro = SGK_PRO_RMS; a.epi = SGK_EPI_STORE;
    } else {
        glayer *L = &g->ls[layer];
        switch (which) {
        case 0: M = &L->in; a.x = g->x; a.nw = L->ln1; a.y = g->act; a.pro = SGK_PRO_RMS; a.epi = SGK_EPI_STORE; break;
        case 1:
            M = &L->out; a.y = g->x; a.epi = SGK_EPI_ADD;
            if (L->attn) { a.x = g->ctx; a.pro = SGK_PRO_NONE; }
            else if (g->gdn_blocks == 1) { a.x = g->gbuf; a.pro = SGK_PRO_NONE; }
            else { a.x = g->gbuf; a.gss = g->gss; a.gdv = c->head_v_dim; a.pro = SGK_PRO_GATED; }
            break;
        case 2: M = &L->gu; a.x = g->x; a.nw = L->ln2; a.y = g->ffg; a.pro = SGK_PRO_RMS; a.epi = SGK_EPI_SWIGLU; break;
        case 3: M = &L->down; a.x = g->ffg; a.y = g->x; a.pro = SGK_PRO_NONE; a.epi = SGK_EPI_ADD; break;
        default: return (sg_err){"gpu: which must be 0..4"};
        }
    }
    a.qs = M->qs; a.d = M->d; a.wf = M->wf; a.rows = M->rows; a.cols = M->cols;
    a.tune_r = tune_r; a.tune_blocks = tune_blocks;
    HIPCHK(sgk_gemv_launch(&a, g->stream), "gemv launch");
    return SG_OK;
}

/* ---------------------------------------------------------------------
 * timing hooks for the per-kernel micro configs (no reference counterpart)
 *
 * Each runs one product kernel `reps` times back to back on the library
 * stream and reports the average microseconds per launch from HIP events
 * around the launches. Launch i reads input copy i % n, the n copies laid out
 * one after another in a scratch allocation of at least `rotate_bytes`, so a
 * timed launch does not find its inputs in the 256 MB MALL left there by the
 * launch before; rotate_bytes 0 keeps one copy (the cache-resident figure).
 * Inputs come from caller buffers (uploaded from their host mirrors).
 * --------------------------------------------------------------------- */

static uint64_t n_copies(uint64_t unit, uint64_t rotate_bytes) {
    uint64_t n = rotate_bytes ? (rotate_bytes + unit - 1) / unit : 1;
    return n < 1 ? 1 : n;
}

static sg_err timed(sg_gpu *g, hipEvent_t a, hipEvent_t b, uint32_t reps, double *us) {
    HIPCHK(hipEventSynchronize(b), "timing");
    float ms = 0.0f;
    HIPCHK(hipEventElapsedTime(&ms, a, b), "timing");
    *us = (double)ms * 1e3 / reps;
    (void)g;
    return SG_OK;
}

/* The decode GEMV (k_gemv_q8, no prologue, plain store) on a Q8_0 matrix
 * [rows][cols/32] of 34-byte blocks: y = W x. */
sg_err sg_gpu_time_read(sg_gpu *g, uint64_t bytes, uint64_t rotate_bytes, uint32_t reps, double *us) {
    if (!g || !us || !reps || !bytes || bytes % 16) return (sg_err){"gpu: sg_gpu_time_read got an invalid argument"};
    const uint64_t unit = (bytes + 255) / 256 * 256, n = n_copies(unit, rotate_bytes);
    char *base;
    float *out;
    sg_err e;
    if (sg_failed(e = dzalloc(g, n * unit, (void **)&base))) return e;
    const uint32_t blocks = 4 * (uint32_t)sgk_device_cus();
    if (sg_failed(e = dalloc(g, (uint64_t)blocks * 4, (void **)&out))) { dfree(g, base); return e; }
    hipStream_t s = g->stream;
    hipEvent_t a = NULL, b = NULL;
    hipError_t he = hipEventCreate(&a);
    if (he == hipSuccess) he = hipEventCreate(&b);
    for (uint32_t r = 0; r < reps + 1 && he == hipSuccess; r++) {     /* launch 0 warms up, untimed */
        if (r == 1) he = hipEventRecord(a, s);
        if (he == hipSuccess) he = sgk_read(base + (uint64_t)((r + n - 1) % n) * unit, bytes, out, blocks, s);
    }
    if (he == hipSuccess) he = hipEventRecord(b, s);
    if (he == hipSuccess) e = timed(g, a, b, reps, us);
    else e = errf("gpu: sg_gpu_time_read: %s", hipGetErrorString(he));
    hipStreamSynchronize(s);
    if (a) hipEventDestroy(a);
    if (b) hipEventDestroy(b);
    dfree(g, out);
    dfree(g, base);
    return e;
}

sg_err sg_gpu_time_empty(sg_gpu *g, uint32_t reps, int graph, double *us) {
    if (!g || !us || !reps) return (sg_err){"gpu: sg_gpu_time_empty got an invalid argument"};
    hipStream_t s = g->stream;
    hipEvent_t a = NULL, b = NULL;
    hipGraph_t gr = NULL;
    hipGraphExec_t ge = NULL;
    hipError_t he = hipEventCreate(&a);
    if (he == hipSuccess) he = hipEventCreate(&b);
    if (he == hipSuccess && graph) {
        he = hipStreamBeginCapture(s, hipStreamCaptureModeRelaxed);
        for (uint32_t r = 0; r < reps && he == hipSuccess; r++) he = sgk_empty(s);
        hipError_t ce = hipStreamEndCapture(s, &gr);
        if (he == hipSuccess) he = ce;
        if (he == hipSuccess) he = hipGraphInstantiate(&ge, gr, NULL, NULL, 0);
        if (he == hipSuccess) he = hipGraphLaunch(ge, s);              /* warm-up */
        if (he == hipSuccess) he = hipEventRecord(a, s);
        if (he == hipSuccess) he = hipGraphLaunch(ge, s);
    } else if (he == hipSuccess) {
        he = sgk_empty(s);
        if (he == hipSuccess) he = hipEventRecord(a, s);
        for (uint32_t r = 0; r < reps && he == hipSuccess; r++) he = sgk_empty(s);
    }
    if (he == hipSuccess) he = hipEventRecord(b, s);
    sg_err e = he == hipSuccess ? timed(g, a, b, reps, us) : errf("gpu: sg_gpu_time_empty: %s", hipGetErrorString(he));
    hipStreamSynchronize(s);
    if (ge) hipGraphExecDestroy(ge);
    if (gr) hipGraphDestroy(gr);
    if (a) hipEventDestroy(a);
    if (b) hipEventDestroy(b);
    return e;
}

/* Algorithmic bytes of each kernel of one greedy decode token at `ctx` keys,
 * in the launch order of enqueue_step (greedy, per-kernel path): embedding;
 * per layer the input projection, the attention partial and combine or the
 * DeltaNet step, the output projection, gate/up and down; lm_head, the two
 * argmax passes and the step advance. Returns the kernel count (b may be NULL
 * to count). Every figure is rounded up to 16 bytes. */
static uint32_t floor_plan(const sg_gpu *g, uint32_t ctx, uint64_t *b) {
    const sg_cfg *c = &g->cfg;
    const uint64_t H = c->hidden, hd = c->head_dim, nh = c->n_heads, nkv = c->n_kv_heads;
    const uint64_t ns = sgk_n_splits_cap(ctx, g->split_cap ? g->split_cap : SGK_MAX_SPLITS);
    uint32_t n = 0;
#define FL_ADD(v) do { const uint64_t v_ = (v); if (b) b[n] = (v_ + 15) & ~(uint64_t)15; n++; } while (0)
#define FL_GEMV(M, rms, orows) FL_ADD((uint64_t)(M).rows * (M).cols / 32 * 34 + (uint64_t)(M).cols * 4 * ((rms) ? 2 : 1) \
                                      + (uint64_t)(orows) * 4)
    FL_ADD(H + H / 16 + 4 * H);
    for (uint32_t i = 0; i < c->n_layers; i++) {
        const glayer *L = &g->ls[i];
        FL_GEMV(L->in, 1, L->in.rows);
        if (L->attn) {
            FL_ADD(2 * (uint64_t)ctx * nkv * hd * 2 + (uint64_t)L->in.rows * 4 + nh * ns * (hd + 2) * 4);
            FL_ADD(nh * ns * (hd + 2) * 4 + 2 * nh * hd * 4);
        } else {
            const uint64_t nv = c->n_v_heads, dv = c->head_v_dim, dk = c->head_k_dim, cd = g->conv_dim;
            FL_ADD(2 * nv * dv * dk * 4 + 5 * cd * 4 + (uint64_t)L->in.rows * 4 + cd * c->conv_kernel * 4 + nv * dv * 4);
        }
        FL_GEMV(L->out, 0, L->out.rows);
        FL_GEMV(L->gu, 1, L->gu.rows / 2);
        FL_GEMV(L->down, 0, L->down.rows);
    }
    FL_GEMV(g->lm, 1, g->lm.rows);
    FL_ADD((uint64_t)c->vocab * 4);
    FL_ADD(256 * 4);
    FL_ADD(16);
#undef FL_GEMV
#undef FL_ADD
    return n;
}

sg_err sg_gpu_time_floor(sg_gpu *g, uint32_t ctx, uint32_t mode, uint32_t reps, double *us, uint32_t *n_kernels,
                         uint64_t *bytes) {
    if (!g || !us || !reps || mode > 2 || !ctx) return (sg_err){"gpu: sg_gpu_time_floor got an invalid argument"};
    if (!g->have_state || !g->q8) return (sg_err){"gpu: sg_gpu_time_floor needs a Q8_0 model and a state"};
    const uint32_t n = floor_plan(g, ctx, NULL);
    uint64_t *b = malloc((uint64_t)n * sizeof *b);
    if (!b) return (sg_err){"gpu: out of host memory"};
    floor_plan(g, ctx, b);
    uint64_t tot = 0;
    for (uint32_t i = 0; i < n; i++) tot += (b[i] + 255) & ~(uint64_t)255;
    char *base = NULL;
    float *out = NULL;
    const uint32_t maxb = 4 * (uint32_t)sgk_device_cus();
    sg_err e = SG_OK;
    if (mode != 0) e = dalloc(g, tot, (void **)&base);
    if (!sg_failed(e)) e = dalloc(g, (uint64_t)maxb * 4, (void **)&out);
    hipStream_t s = g->stream;
    hipEvent_t ea = NULL, eb = NULL;
    hipGraph_t gr = NULL;
    hipGraphExec_t ge = NULL;
    /* one token's launches: empty kernels, or each kernel's bytes read from
     * its own region (about one workgroup per 16 KB, at most 4 per CU) */
    hipError_t he;
#define FL_TOKEN() do {                                                                        \
        uint64_t off_ = 0;                                                                     \
        for (uint32_t i_ = 0; i_ < n && he == hipSuccess; i_++) {                             \
            if (mode == 0) { he = sgk_empty(s); continue; }                                    \
            uint64_t blocks_ = b[i_] / 16384;                                                  \
            blocks_ = blocks_ < 1 ? 1 : blocks_ > maxb ? maxb : blocks_;                       \
            he = sgk_read(base + off_, b[i_], out, (uint32_t)blocks_, s);                      \
            off_ += (b[i_] + 255) & ~(uint64_t)255;                                            \
        }                                                                                      \
    } while (0)
    he = sg_failed(e) ? hipErrorOutOfMemory : hipEventCreate(&ea);
    if (he == hipSuccess) he = hipEventCreate(&eb);
    if (mode == 2) {                          /* launched one by one, as the profiler sees them */
        if (he == hipSuccess) FL_TOKEN();
        if (he == hipSuccess) he = hipEventRecord(ea, s);
        for (uint32_t r = 0; r < reps && he == hipSuccess; r++) FL_TOKEN();
    } else {
        if (he == hipSuccess) he = hipStreamBeginCapture(s, hipStreamCaptureModeRelaxed);
        if (he == hipSuccess) {
            FL_TOKEN();
            hipError_t ce = hipStreamEndCapture(s, &gr);
            if (he == hipSuccess) he = ce;
        }
        if (he == hipSuccess) he = hipGraphInstantiate(&ge, gr, NULL, NULL, 0);
        if (he == hipSuccess) he = hipGraphLaunch(ge, s);                     /* warm-up, untimed */
        if (he == hipSuccess) he = hipEventRecord(ea, s);
        for (uint32_t r = 0; r < reps && he == hipSuccess; r++) he = hipGraphLaunch(ge, s);
    }
#undef FL_TOKEN
    if (he == hipSuccess) he = hipEventRecord(eb, s);
    if (!sg_failed(e)) e = he == hipSuccess ? timed(g, ea, eb, reps, us) : errf("gpu: sg_gpu_time_floor: %s", hipGetErrorString(he));
    hipStreamSynchronize(s);
    if (ge) hipGraphExecDestroy(ge);
    if (gr) hipGraphDestroy(gr);
    if (ea) hipEventDestroy(ea);
    if (eb) hipEventDestroy(eb);
    if (n_kernels) *n_kernels = n;
    if (bytes) { uint64_t t = 0; for (uint32_t i = 0; i < n; i++) t += b[i]; *bytes = t; }
    free(b);
    dfree(g, out);
    dfree(g, base);
    return e;
}

sg_err sg_gpu_time_matvec_q8(sg_gpu *g, void *w, void *x, void *y, uint32_t rows, uint32_t cols,
                             uint64_t rotate_bytes, uint32_t reps, double *us) {
    if (!g || !w || !x || !y || !us || !reps || !rows || !cols || cols % 32)
        return (sg_err){"gpu: sg_gpu_time_matvec_q8 got an invalid argument"};
    sg_err e;
    if (sg_failed(e = need(w, (uint64_t)rows * (cols / 32) * 34, "w")) || sg_failed(e = need(x, (uint64_t)cols * 4, "x")) ||
        sg_failed(e = need(y, (uint64_t)rows * 4, "y"))) return e;
    void *ins[2] = {w, x};
    if (sg_failed(e = push(ins, 2))) return e;
    const uint64_t qb = ((uint64_t)rows * cols + 255) / 256 * 256, db = ((uint64_t)rows * (cols / 32) * 2 + 255) / 256 * 256;
    const uint64_t n = n_copies(qb + db, rotate_bytes);
    char *base;
    if (sg_failed(e = dalloc(g, n * (qb + db), (void **)&base))) return e;
    hipStream_t s = g->stream;
    hipEvent_t a = NULL, b = NULL;
    hipError_t he = sgk_repack_q8(DEV(w), rows, cols, (int8_t *)base, (uint16_t *)(base + qb), NULL, rows, 0, 1, s);
    for (uint64_t i = 1; i < n && he == hipSuccess; i++)
        he = hipMemcpyAsync(base + i * (qb + db), base, qb + db, hipMemcpyDeviceToDevice, s);
    if (he == hipSuccess) he = hipEventCreate(&a);
    if (he == hipSuccess) he = hipEventCreate(&b);
    sgk_gemv ga = {0};
    ga.rows = rows; ga.cols = cols; ga.x = DEV(x); ga.y = DEV(y); ga.pro = SGK_PRO_NONE; ga.epi = SGK_EPI_STORE;
    for (uint32_t r = 0; r < reps + 1 && he == hipSuccess; r++) {     /* launch 0 warms up, untimed */
        const uint64_t c = (uint64_t)(r + n - 1) % n;
        ga.qs = (const int8_t *)(base + c * (qb + db));
        ga.d = (const uint16_t *)(base + c * (qb + db) + qb);
        if (r == 1) he = hipEventRecord(a, s);
        if (he == hipSuccess) he = sgk_gemv_launch(&ga, s);
    }
    if (he == hipSuccess) he = hipEventRecord(b, s);
    if (he == hipSuccess) e = timed(g, a, b, reps, us);
    else e = errf("gpu: sg_gpu_time_matvec_q8: %s", hipGetErrorString(he));
    hipStreamSynchronize(s);
    if (a) hipEventDestroy(a);
    if (b) hipEventDestroy(b);
    dfree(g, base);
    if (!sg_failed(e)) e = sg_gpu_buf_download(y);
    return e;
}

/* The decode split-K attention (the partial on q as given, then the LSE
 * combine), p as sg_gpu_run_attn_splitk_partial_gqa with p[6] = n_splits (0 =
 * the decode policy's count). K and V [seq][n_kv][hd] f16 are rotated;
 * us[0] = partial, us[1] = combine (each timed over its own reps launches). */
sg_err sg_gpu_time_attn(sg_gpu *g, void *q, void *k, void *v, void *out, const uint32_t p[8],
                        uint64_t rotate_bytes, uint32_t reps, double *us) {
    if (!g || !q || !k || !v || !out || !p || !us || !reps) return (sg_err){"gpu: sg_gpu_time_attn got an invalid argument"};
    uint32_t pp[8];
    memcpy(pp, p, sizeof pp);
    if (!pp[6]) pp[6] = sgk_n_splits(pp[3]);
    sg_err e = attn_check(pp, true, false);
    if (sg_failed(e)) return e;
    const uint32_t nh = pp[0], nkv = pp[1], hd = pp[2], seq = pp[3], qs = pp[4], ns = pp[6];
    if (!seq) return (sg_err){"gpu: sg_gpu_time_attn needs seq >= 1"};
    const uint64_t kvb = (uint64_t)seq * nkv * hd * 2, unit = (2 * kvb + 255) / 256 * 256;
    if (sg_failed(e = need(q, ((uint64_t)(nh - 1) * qs + hd) * 4, "q")) || sg_failed(e = need(k, kvb, "k")) ||
        sg_failed(e = need(v, kvb, "v")) || sg_failed(e = need(out, (uint64_t)nh * hd * 4, "out"))) return e;
    void *ins[3] = {q, k, v};
    if (sg_failed(e = push(ins, 3))) return e;
    const uint64_t n = n_copies(unit, rotate_bytes), part = (uint64_t)nh * ns * (2 + hd) * 4;
    char *base;
    if (sg_failed(e = dalloc(g, n * unit + part, (void **)&base))) return e;
    hipStream_t s = g->stream;
    hipEvent_t ev[4] = {0};
    hipError_t he = hipSuccess;
    for (uint64_t i = 0; i < n && he == hipSuccess; i++) {
        he = hipMemcpyAsync(base + i * unit, DEV(k), kvb, hipMemcpyDeviceToDevice, s);
        if (he == hipSuccess) he = hipMemcpyAsync(base + i * unit + kvb, DEV(v), kvb, hipMemcpyDeviceToDevice, s);
    }
    for (int i = 0; i < 4 && he == hipSuccess; i++) he = hipEventCreate(&ev[i]);
    float *mm = (float *)(base + n * unit), *ss = mm + (uint64_t)nh * ns, *aa = ss + (uint64_t)nh * ns;
    sgk_attn A = {0};
    A.q = DEV(q); A.m = mm; A.s = ss; A.acc = aa; A.out = DEV(out);
    A.n_heads = nh; A.n_kv = nkv; A.hd = hd; A.q_stride = qs; A.seq = seq; A.n_splits = ns; A.max_splits = ns;
    A.ntok = 1; A.scale = fbits(pp[5]);
    for (uint32_t r = 0; r < reps + 1 && he == hipSuccess; r++) {
        const uint64_t c = (uint64_t)(r + n - 1) % n;
        A.kc = (uint16_t *)(base + c * unit);
        A.vc = (uint16_t *)(base + c * unit + kvb);
        if (r == 1) he = hipEventRecord(ev[0], s);
        if (he == hipSuccess) he = sgk_attn_partial(&A, s);
    }
    if (he == hipSuccess) he = hipEventRecord(ev[1], s);
    for (uint32_t r = 0; r < reps + 1 && he == hipSuccess; r++) {
        if (r == 1) he = hipEventRecord(ev[2], s);
        if (he == hipSuccess) he = sgk_attn_combine(&A, s);
    }
    if (he == hipSuccess) he = hipEventRecord(ev[3], s);
    if (he == hipSuccess) e = timed(g, ev[0], ev[1], reps, &us[0]);
    else e = errf("gpu: sg_gpu_time_attn: %s", hipGetErrorString(he));
    if (!sg_failed(e)) e = timed(g, ev[2], ev[3], reps, &us[1]);
    hipStreamSynchronize(s);
    for (int i = 0; i < 4; i++) if (ev[i]) hipEventDestroy(ev[i]);
    dfree(g, base);
    if (!sg_failed(e)) e = sg_gpu_buf_download(out);
    return e;
}

/* The fused DeltaNet decode step (k_gdn_step, one workgroup per value head)
 * with buffers and p as sg_gpu_run_gdn_step; the rotated copies are the
 * state S and the 4-slot conv ring (the per-layer state a decode step reads
 * and writes). */
sg_err sg_gpu_time_gdn_step(sg_gpu *g, void *in, void *w, void *out, const uint32_t p[8], uint64_t rotate_bytes,
                            uint32_t reps, double *us) {
    if (!g || !in || !w || !out || !p || !us || !reps) return (sg_err){"gpu: sg_gpu_time_gdn_step got an invalid argument"};
    const uint32_t dk = p[0], dv = p[1], nv = p[2], nk = p[3], ks = p[4];
    if ((dk != 32 && dk != 64 && dk != 128 && dk != 256) || !dv || dv > 128 || !nv || !nk || nv % nk || ks < 1 || ks > 4)
        return (sg_err){"gpu: sg_gpu_time_gdn_step: bad shape"};
    const uint64_t cd = 2ull * nk * dk + (uint64_t)nv * dv, vd = (uint64_t)nv * dv;
    sg_err e;
    if (sg_failed(e = need(in, (cd + vd + 2ull * nv) * 4, "in")) || sg_failed(e = need(w, (cd * ks + 2ull * nv + dv) * 4, "w")) ||
        sg_failed(e = need(out, vd * 4, "out"))) return e;
    void *ins[2] = {in, w};
    if (sg_failed(e = push(ins, 2))) return e;
    const uint64_t unit = ((4 * cd + vd * dk) * 4 + 255) / 256 * 256, n = n_copies(unit, rotate_bytes);
    char *base;
    if (sg_failed(e = dzalloc(g, 256 + n * unit, (void **)&base))) return e;
    hipStream_t s = g->stream;
    sgk_step st = {0, 3, {0, 0}};
    hipEvent_t a = NULL, b = NULL;
    hipError_t he = hipMemcpyAsync(base, &st, sizeof st, hipMemcpyHostToDevice, s);
    if (he == hipSuccess) he = sgk_fill_hash(base + 256, n * unit / 4, 0, 5, 0.05f, s);
    if (he == hipSuccess) he = hipEventCreate(&a);
    if (he == hipSuccess) he = hipEventCreate(&b);
    const float *wp = DEV(w);
    sgk_gdn d = {0};
    d.in = DEV(in); d.z = (const float *)DEV(in) + cd; d.conv_w = wp; d.ssm_a = wp + cd * ks;
    d.dt_bias = d.ssm_a + nv; d.norm_w = d.dt_bias + nv; d.step = (const sgk_step *)base;
    d.n_k = nk; d.n_v = nv; d.dk = dk; d.dv = dv; d.conv_dim = (uint32_t)cd; d.ksize = ks;
    d.tiled = p[5] != 0; d.neg_exp = p[6] != 0; d.out = DEV(out); d.eps = fbits(p[7]); d.blocks = 1;
    for (uint32_t r = 0; r < reps + 1 && he == hipSuccess; r++) {
        char *c = base + 256 + (uint64_t)((r + n - 1) % n) * unit;
        d.ring = (float *)c;
        d.S = (float *)c + 4 * cd;
        if (r == 1) he = hipEventRecord(a, s);
        if (he == hipSuccess) he = sgk_gdn_step(&d, s);
    }
    if (he == hipSuccess) he = hipEventRecord(b, s);
    if (he == hipSuccess) e = timed(g, a, b, reps, us);
    else e = errf("gpu: sg_gpu_time_gdn_step: %s", hipGetErrorString(he));
    hipStreamSynchronize(s);
    if (a) hipEventDestroy(a);
    if (b) hipEventDestroy(b);
    dfree(g, base);
    if (!sg_failed(e)) e = sg_gpu_buf_download(out);
    return e;
}
