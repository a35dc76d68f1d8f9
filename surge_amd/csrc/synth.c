/* synth.c - seeded random-init qwen35-shaped models, in memory or as GGUF.
 *
 * No reference counterpart in C: the reference writes its test models from
 * Python (reference tools/make_fixtures.py:561-582 for the Q8_0 rule and
 * :1242-1416 for the GGUF writer). The file format, tensor names and GGUF
 * semantics below are therefore the format's own (they must match what
 * sg_model_from_gguf reads): Q8_0 blocks are a little-endian f16 scale then
 * 32 int8; small tensors are F32; ssm_a holds -exp(A_log) (< 0); norms are
 * absolute (near 1); value heads are tiled.
 *
 * Random values (matching the benchmark configs):
 *   Q8_0 matmul blocks: 32 int8 uniform in [-127, 127] and the scale
 *     f16(|N(0, 0.02)| / 127);
 *   F32 matmul weights: uniform in [-0.02*sqrt(3), 0.02*sqrt(3)];
 *   norms 1 + U(-0.1, 0.1); conv1d U(-0.5, 0.5); dt_bias U(-0.5, 0.5);
 *   ssm_a = -exp(U(-1, 1)).
 * Every 64-row slab of every tensor starts its own splitmix64 stream at a
 * hash of (seed, tensor index, slab), so the bytes do not depend on the
 * thread count and no two slabs share a stream.
 */
#define _GNU_SOURCE
#include "surge.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>

typedef enum { INIT_MAT, INIT_NORM, INIT_CONV, INIT_DT, INIT_NEG_A } init_kind;

typedef struct {
    char name[64];
    sg_tensor_type type;
    uint64_t rows, cols;   /* 1-D tensors have rows == 1 */
    uint64_t offset, nbytes;
    init_kind init;
} stensor;

struct sg_synth {
    sg_cfg cfg;
    sg_tensor_type wtype;
    uint64_t seed;
    stensor *t;
    uint32_t nt, cap;
    uint8_t *blob;
    uint64_t blob_bytes;
    sg_model model;
};

static uint64_t splitmix(uint64_t *s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
/* splitmix64's output mix, used to hash (seed, tensor, slab) into
 * well-separated starting states (splitmix is a counter generator: streams
 * started from nearby states would be shifted copies of each other). */
static uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static double unif(uint64_t *s) { return (double)(splitmix(s) >> 11) * (1.0 / 9007199254740992.0); }
static double normal(uint64_t *s) {
    double u1 = unif(s), u2 = unif(s);
    if (u1 < 1e-300) u1 = 1e-300;
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

static uint64_t row_bytes(sg_tensor_type t, uint64_t cols) {
    return t == SG_T_Q8_0 ? cols / 32 * 34 : cols * 4;
}

static int add(sg_synth *s, const char *name, sg_tensor_type t, uint64_t rows, uint64_t cols,
               init_kind init) {
    if (s->nt == s->cap) {
        uint32_t nc = s->cap ? 2 * s->cap : 64;
        stensor *n = realloc(s->t, nc * sizeof *n);
        if (!n) return -1;
        s->t = n;
        s->cap = nc;
    }
    stensor *x = &s->t[s->nt++];
    memset(x, 0, sizeof *x);
    snprintf(x->name, sizeof x->name, "%s", name);
    x->type = t;
    x->rows = rows;
    x->cols = cols;
    x->init = init;
    x->nbytes = rows * row_bytes(t, cols);
    x->offset = s->blob_bytes;
    s->blob_bytes += (x->nbytes + 255) / 256 * 256;
    return (int)(s->nt - 1);
}

/* f32 -> f16 for the scale (RNE via the library routine). */
static void fill_slab(const sg_synth *s, uint32_t ti, uint64_t r0, uint64_t r1) {
    const stensor *x = &s->t[ti];
    uint64_t st = mix64(mix64(mix64(s->seed + 0x5EEDull) ^ ti) ^ (r0 / 64));
    uint8_t *base = s->blob + x->offset;
    uint64_t rb = row_bytes(x->type, x->cols);
    for (uint64_t r = r0; r < r1; r++) {
        uint8_t *row = base + r * rb;
        if (x->type == SG_T_Q8_0) {
            for (uint64_t b = 0; b < x->cols / 32; b++) {
                uint8_t *blk = row + b * 34;
                float d = (float)(fabs(normal(&st) * 0.02) / 127.0);
                uint16_t h = sg_f32_to_f16(d);
                blk[0] = (uint8_t)(h & 0xFF);
                blk[1] = (uint8_t)(h >> 8);
                for (int k = 0; k < 32; k += 8) {
                    uint64_t v = splitmix(&st);
                    for (int j = 0; j < 8; j++) {
                        int8_t q = (int8_t)(v >> (8 * j));
                        if (q == -128) q = -127;
                        blk[2 + k + j] = (uint8_t)q;
                    }
                }
            }
        } else {
            float *f = (float *)row;
            for (uint64_t c = 0; c < x->cols; c++) {
                double u = 2.0 * unif(&st) - 1.0;
                switch (x->init) {
                case INIT_MAT: f[c] = (float)(u * 0.02 * 1.7320508075688772); break;
                case INIT_NORM: f[c] = (float)(1.0 + 0.1 * u); break;
                case INIT_CONV: f[c] = (float)(0.5 * u); break;
                case INIT_DT: f[c] = (float)(0.5 * u); break;
                case INIT_NEG_A: f[c] = (float)(-exp(u)); break;
                }
            }
        }
    }
}

const sg_model *sg_synth_model(const sg_synth *s) { return s ? &s->model : NULL; }
uint64_t sg_synth_bytes(const sg_synth *s) { return s ? s->blob_bytes : 0; }

void sg_synth_free(sg_synth *s) {
    if (!s) return;
    if (s->blob) munmap(s->blob, s->blob_bytes ? s->blob_bytes : 1);
    free(s->model.layers);
    free(s->t);
    free(s);
}

sg_err sg_synth_new(const sg_cfg *cfg, sg_tensor_type wtype, uint64_t seed, sg_synth **out) {
    if (!out || !cfg) return (sg_err){"synth: invalid arguments"};
    *out = NULL;
    const sg_cfg *c = cfg;
    if (wtype != SG_T_Q8_0 && wtype != SG_T_F32) return (sg_err){"synth: wtype must be Q8_0 or F32"};
    if (!c->n_layers || !c->hidden || !c->ffn_hidden || !c->vocab || !c->head_dim ||
        !c->n_heads || !c->n_kv_heads || !c->full_attn_interval)
        return (sg_err){"synth: config has a zero dimension"};
    uint64_t H = c->hidden, F = c->ffn_hidden, hd = c->head_dim;
    uint64_t attn_w = c->n_heads * hd, kv_w = c->n_kv_heads * hd;
    uint64_t q_w = c->attn_output_gate ? 2 * attn_w : attn_w;
    uint64_t kd = (uint64_t)c->n_k_heads * c->head_k_dim, vd = (uint64_t)c->n_v_heads * c->head_v_dim;
    uint64_t conv = 2 * kd + vd;
    if (wtype == SG_T_Q8_0 && (H % 32 || F % 32 || attn_w % 32 || vd % 32))
        return (sg_err){"synth: a Q8_0 matmul width is not a multiple of 32"};

    sg_synth *s = calloc(1, sizeof *s);
    if (!s) return (sg_err){"synth: out of memory"};
    s->cfg = *c;
    s->wtype = wtype;
    s->seed = seed;
    char nm[64];
    bool ok = true;
#define ADD(n, t, r, cc, k) ok = ok && add(s, n, t, r, cc, k) >= 0
    ADD("token_embd.weight", wtype, c->vocab, H, INIT_MAT);
    ADD("output_norm.weight", SG_T_F32, 1, H, INIT_NORM);
    if (!c->tied_embeddings) ADD("output.weight", wtype, c->vocab, H, INIT_MAT);
    for (uint32_t i = 0; i < c->n_layers; i++) {
        bool attn = (i + 1) % c->full_attn_interval == 0;
#define L(suffix, t, r, cc, k) (snprintf(nm, sizeof nm, "blk.%u." suffix, i), ADD(nm, t, r, cc, k))
        L("attn_norm.weight", SG_T_F32, 1, H, INIT_NORM);
        L("post_attention_norm.weight", SG_T_F32, 1, H, INIT_NORM);
        L("ffn_gate.weight", wtype, F, H, INIT_MAT);
        L("ffn_up.weight", wtype, F, H, INIT_MAT);
        L("ffn_down.weight", wtype, H, F, INIT_MAT);
        if (attn) {
            L("attn_q.weight", wtype, q_w, H, INIT_MAT);
            L("attn_k.weight", wtype, kv_w, H, INIT_MAT);
            L("attn_v.weight", wtype, kv_w, H, INIT_MAT);
            L("attn_output.weight", wtype, H, attn_w, INIT_MAT);
            L("attn_q_norm.weight", SG_T_F32, 1, hd, INIT_NORM);
            L("attn_k_norm.weight", SG_T_F32, 1, hd, INIT_NORM);
        } else {
            L("attn_qkv.weight", wtype, conv, H, INIT_MAT);
            L("attn_gate.weight", wtype, vd, H, INIT_MAT);
            L("ssm_beta.weight", wtype, c->n_v_heads, H, INIT_MAT);
            L("ssm_alpha.weight", wtype, c->n_v_heads, H, INIT_MAT);
            L("ssm_a", SG_T_F32, 1, c->n_v_heads, INIT_NEG_A);
            L("ssm_dt.bias", SG_T_F32, 1, c->n_v_heads, INIT_DT);
            L("ssm_conv1d.weight", SG_T_F32, conv, c->conv_kernel, INIT_CONV);
            L("ssm_norm.weight", SG_T_F32, 1, c->head_v_dim, INIT_NORM);
            L("ssm_out.weight", wtype, H, vd, INIT_MAT);
        }
#undef L
    }
#undef ADD
    if (!ok) { sg_synth_free(s); return (sg_err){"synth: out of memory"}; }
    void *blob = mmap(NULL, s->blob_bytes, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS, -1, 0);
    if (blob == MAP_FAILED) { s->blob_bytes = 0; sg_synth_free(s); return (sg_err){"synth: out of memory for the weights"}; }
    s->blob = blob;

    /* Fill: every (tensor, 64-row slab) is independent. */
    uint64_t nslab = 0;
    for (uint32_t i = 0; i < s->nt; i++) nslab += (s->t[i].rows + 63) / 64;
    uint64_t *work = malloc(nslab * sizeof *work);
    if (!work) { sg_synth_free(s); return (sg_err){"synth: out of memory"}; }
    uint64_t k = 0;
    for (uint32_t i = 0; i < s->nt; i++)
        for (uint64_t r = 0; r < s->t[i].rows; r += 64) work[k++] = ((uint64_t)i << 40) | (r / 64);
#pragma omp parallel for schedule(dynamic, 16)
    for (int64_t w = 0; w < (int64_t)nslab; w++) {
        uint32_t ti = (uint32_t)(work[w] >> 40);
        uint64_t r0 = (work[w] & ((1ull << 40) - 1)) * 64;
        uint64_t r1 = r0 + 64 < s->t[ti].rows ? r0 + 64 : s->t[ti].rows;
        fill_slab(s, ti, r0, r1);
    }
    free(work);

    /* Point an sg_model at the blob, exactly as sg_model_from_gguf would. */
    sg_model *m = &s->model;
    m->cfg = *c;
    m->layers = calloc(c->n_layers, sizeof *m->layers);
    if (!m->layers) { sg_synth_free(s); return (sg_err){"synth: out of memory"}; }
    uint32_t ti = 0;
#define NEXT() ((const void *)(s->blob + s->t[ti++].offset))
    m->tok_emb = NEXT();
    m->out_norm = NEXT();
    m->lm_head = c->tied_embeddings ? m->tok_emb : NEXT();
    for (uint32_t i = 0; i < c->n_layers; i++) {
        sg_layer_w *w = &m->layers[i];
        w->ln1 = NEXT(); w->ln2 = NEXT();
        w->gate_proj = NEXT(); w->up_proj = NEXT(); w->down_proj = NEXT();
        if ((i + 1) % c->full_attn_interval == 0) {
            w->q_proj = NEXT(); w->k_proj = NEXT(); w->v_proj = NEXT(); w->o_proj = NEXT();
            w->q_norm = NEXT(); w->k_norm = NEXT();
        } else {
            w->ssm_in_qkv = NEXT(); w->ssm_in_z = NEXT(); w->ssm_in_b = NEXT();
            w->ssm_in_a = NEXT(); w->ssm_a = NEXT(); w->ssm_dt_bias = NEXT();
            w->ssm_conv1d = NEXT(); w->ssm_norm = NEXT(); w->ssm_out = NEXT();
        }
    }
#undef NEXT
    m->wtype = wtype;
    m->ssm_a_form = SG_SSM_A_NEG_EXP;
    m->v_heads_tiled = true;
    m->ssm_a_type = SG_T_F32;
    m->ssm_norm_type = SG_T_F32;
    m->dense_type = SG_T_F32;
    m->norms_are_residual = false;
    *out = s;
    return SG_OK;
}

/* ---------------------------------------------------------------------
 * GGUF v3 writer for the same model.
 * --------------------------------------------------------------------- */

static void wr(FILE *f, const void *p, size_t n, bool *ok) { if (*ok && fwrite(p, 1, n, f) != n) *ok = false; }
static void wu32(FILE *f, uint32_t v, bool *ok) { wr(f, &v, 4, ok); }
static void wu64(FILE *f, uint64_t v, bool *ok) { wr(f, &v, 8, ok); }
static void wstr(FILE *f, const char *s, bool *ok) { wu64(f, strlen(s), ok); wr(f, s, strlen(s), ok); }
static void kv_u32(FILE *f, const char *k, uint32_t v, bool *ok) { wstr(f, k, ok); wu32(f, SG_GGUF_U32, ok); wu32(f, v, ok); }
static void kv_f32(FILE *f, const char *k, float v, bool *ok) { wstr(f, k, ok); wu32(f, SG_GGUF_F32, ok); wr(f, &v, 4, ok); }

sg_err sg_synth_write_gguf(const sg_synth *s, const char *path) {
    if (!s || !path) return (sg_err){"synth: invalid arguments"};
    FILE *f = fopen(path, "wb");
    if (!f) return (sg_err){"synth: cannot create the gguf file"};
    bool ok = true;
    const sg_cfg *c = &s->cfg;
    const char *A = "qwen35";
    char k[128];
    uint32_t n_kv = 2 + 17 + 1;
    wr(f, "GGUF", 4, &ok);
    wu32(f, 3, &ok);
    wu64(f, s->nt, &ok);
    wu64(f, n_kv, &ok);
    wstr(f, "general.architecture", &ok); wu32(f, SG_GGUF_STR, &ok); wstr(f, A, &ok);
    kv_u32(f, "general.alignment", 32, &ok);
#define KU(suffix, v) (snprintf(k, sizeof k, "%s." suffix, A), kv_u32(f, k, v, &ok))
#define KF(suffix, v) (snprintf(k, sizeof k, "%s." suffix, A), kv_f32(f, k, v, &ok))
    KU("block_count", c->n_layers);
    KU("attention.head_count", c->n_heads);
    KU("attention.head_count_kv", c->n_kv_heads);
    KU("attention.key_length", c->head_dim);
    KU("attention.value_length", c->head_dim);
    KU("embedding_length", c->hidden);
    KU("feed_forward_length", c->ffn_hidden);
    KF("rope.freq_base", c->rope_theta);
    KF("attention.layer_norm_rms_epsilon", c->rms_eps);
    KU("rope.dimension_count", c->rope_dim);
    KU("full_attention_interval", c->full_attn_interval);
    KU("ssm.group_count", c->n_k_heads);
    KU("ssm.state_size", c->head_k_dim);
    KU("ssm.time_step_rank", c->n_v_heads);
    KU("ssm.inner_size", c->n_v_heads * c->head_v_dim);
    KU("ssm.conv_kernel", c->conv_kernel);
    KU("vocab_size", c->vocab);
#undef KU
#undef KF
    wstr(f, "tokenizer.ggml.tokens", &ok);
    wu32(f, SG_GGUF_ARR, &ok);
    wu32(f, SG_GGUF_STR, &ok);
    wu64(f, c->vocab, &ok);
    for (uint32_t i = 0; i < c->vocab && ok; i++) {
        char tok[24];
        snprintf(tok, sizeof tok, "<%u>", i);
        wstr(f, tok, &ok);
    }
    /* Tensor infos: GGUF lists dims fastest-first (cols, rows). Offsets are
     * relative to the data section and 256-aligned (a multiple of 32). */
    for (uint32_t i = 0; i < s->nt; i++) {
        const stensor *x = &s->t[i];
        wstr(f, x->name, &ok);
        bool two = x->rows > 1 || strstr(x->name, "weight") != NULL;
        if (two && x->rows > 1) { wu32(f, 2, &ok); wu64(f, x->cols, &ok); wu64(f, x->rows, &ok); }
        else { wu32(f, 1, &ok); wu64(f, x->cols, &ok); }
        wu32(f, x->type, &ok);
        wu64(f, x->offset, &ok);
    }
    long pos = ftell(f);
    static const uint8_t zeros[32] = {0};
    if (pos % 32) wr(f, zeros, 32 - pos % 32, &ok);
    for (uint32_t i = 0; i < s->nt && ok; i++) {
        const stensor *x = &s->t[i];
        uint64_t pad = x->offset - (i ? s->t[i - 1].offset + s->t[i - 1].nbytes : 0);
        for (uint64_t z = 0; z < pad && ok; z += 32) wr(f, zeros, pad - z < 32 ? pad - z : 32, &ok);
        wr(f, s->blob + x->offset, x->nbytes, &ok);
    }
    if (fclose(f) != 0) ok = false;
    return ok ? SG_OK : (sg_err){"synth: writing the gguf file failed"};
}
