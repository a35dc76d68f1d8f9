/* kv.c - KV-cache / DeltaNet-state size math, the f16 conversions and the
 * sg_kv allocation module.
 *
 * Interface: sg_kv_bytes, sg_kv_state_bytes, sg_f32_to_f16, sg_f16_to_f32
 * (reference surge.h:1456-1464; behaviour of reference src/kv.c:88-224), and
 * sg_kv_set_backend / sg_kv_new ... sg_kv_s (surge.h:1466-1501, kv.c:227-447).
 * The sizes are pure functions of the config: full-attention layers
 * ((L+1) % full_attn_interval == 0) hold separate K and V of
 * [cap, n_kv_heads, head_dim]; DeltaNet layers hold a conv tail
 * [conv_kernel-1, conv_dim] and S [n_v_heads, head_v_dim, head_k_dim] in f32.
 * Both return 0 for an invalid dtype, cap > SG_KV_CAP_MAX, a dimension above
 * 2^24 or a u64 overflow. The GPU state in hip.c allocates exactly these
 * byte counts (plus the conv ring slot it keeps for in-place updates).
 */
#include "surge.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define DIM_MAX (1u << 24)

static bool mul_ok(uint64_t a, uint64_t b, uint64_t *o) {
    if (a && b > UINT64_MAX / a) return false;
    *o = a * b;
    return true;
}

static bool is_attn_layer(const sg_cfg *c, uint32_t l) {
    return c->full_attn_interval && (l + 1) % c->full_attn_interval == 0;
}

uint64_t sg_kv_bytes(const sg_cfg *c, uint32_t cap, sg_tensor_type dtype) {
    if (!c || !c->n_layers || cap > SG_KV_CAP_MAX) return 0;
    uint64_t esz = dtype == SG_T_F16 ? 2 : dtype == SG_T_F32 ? 4 : 0;
    uint64_t width = (uint64_t)c->n_kv_heads * c->head_dim;
    if (!esz || !width || width > DIM_MAX) return 0;
    uint64_t one, total = 0;
    if (!mul_ok(width * esz, cap, &one) || !mul_ok(one, 2, &one)) return 0;
    for (uint32_t l = 0; l < c->n_layers; l++) {
        if (!is_attn_layer(c, l)) continue;
        if (total > UINT64_MAX - one) return 0;
        total += one;
    }
    return total;
}

uint64_t sg_kv_state_bytes(const sg_cfg *c) {
    if (!c || !c->n_layers || !c->conv_kernel) return 0;
    uint64_t kd = (uint64_t)c->n_k_heads * c->head_k_dim, vd = (uint64_t)c->n_v_heads * c->head_v_dim;
    if (kd > DIM_MAX || vd > DIM_MAX) return 0;
    uint64_t conv = (2 * kd + vd) * (c->conv_kernel - 1), s, per, total = 0;
    if (!mul_ok(vd, c->head_k_dim, &s)) return 0;
    if (!mul_ok(conv + s, 4, &per)) return 0;
    for (uint32_t l = 0; l < c->n_layers; l++) {
        if (is_attn_layer(c, l)) continue;
        if (total > UINT64_MAX - per) return 0;
        total += per;
    }
    return total;
}

/* binary16 -> f32, exact for every pattern including subnormals: the f16
 * value is re-biased into f32's exponent; a subnormal is normalised first. */
float sg_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, bits;
    if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else if (e) {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    } else if (!m) {
        bits = sign;
    } else {
        int lz = __builtin_clz(m) - 21;      /* shifts that bring bit 10 up */
        bits = sign | ((uint32_t)(113 - lz) << 23) | (((m << lz) & 0x3FFu) << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* f32 -> binary16 with round-to-nearest-even; overflow to +-inf, NaN to the
 * quiet 0x7E00 with the sign kept. */
uint16_t sg_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
    if (ax < 0x33000001u) return (uint16_t)sign;      /* <= 2^-25 rounds to zero */
    uint32_t e = ax >> 23, mant = (ax & 0x7FFFFFu) | 0x800000u;
    uint32_t shift = e < 113 ? 126 - e : 13;          /* drop to the f16 ulp */
    uint32_t q = mant >> shift, rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
    q += (rem > half) || (rem == half && (q & 1u));
    if (e < 113) return (uint16_t)(sign | q);
    return (uint16_t)(sign | (((e - 112u) << 10) + q - 0x400u));
}

/* ---------------------------------------------------------------------
 * The standalone KV / DeltaNet-state module (reference surge.h:1466-1501,
 * src/kv.c:227-447): per-layer buffers allocated through an injected
 * backend, so the module itself needs no GPU. sg_gpu_init registers
 * sg_gpu_alloc / sg_gpu_buf_free / sg_gpu_buf_host; a pure-C caller
 * registers a malloc-backed one. Layout: a full-attention layer has separate
 * K and V of [cap, n_kv_heads, head_dim] in kv_dtype; a DeltaNet layer has a
 * conv tail [conv_kernel-1, conv_dim] and S [n_v_heads, head_v_dim,
 * head_k_dim], both f32. (The decode state of sg_gpu_state_new keeps its own
 * head-major cache; this module is the reference's allocator, for callers
 * that manage buffers themselves.)
 * --------------------------------------------------------------------- */
static struct { sg_kv_alloc_fn alloc; sg_kv_free_fn free_; sg_kv_host_fn host; } kv_be;

void sg_kv_set_backend(sg_kv_alloc_fn alloc, sg_kv_free_fn free_, sg_kv_host_fn host) {
    kv_be.alloc = alloc;
    kv_be.free_ = free_;
    kv_be.host = host;
}

struct sg_kv {
    sg_cfg cfg;
    uint32_t cap, used;
    sg_tensor_type dtype;
    sg_kv_free_fn free_;        /* the backend the buffers came from */
    sg_kv_host_fn host;
    uint64_t conv_bytes, s_bytes;
    void **buf;                 /* [n_layers][4]: k, v, conv, s (NULL where the layer has none) */
};

enum { KV_K = 0, KV_V, KV_CONV, KV_S };

void sg_kv_free(sg_kv *kv) {
    if (!kv) return;
    for (uint64_t i = 0; kv->buf && i < (uint64_t)kv->cfg.n_layers * 4; i++)
        if (kv->buf[i] && kv->free_) kv->free_(kv->buf[i]);
    free(kv->buf);
    free(kv);
}

sg_err sg_kv_new(sg_gpu *g, const sg_cfg *c, uint32_t cap, sg_tensor_type kv_dtype, sg_kv **out) {
    if (!out) return (sg_err){"kv: sg_kv_new got a NULL out"};
    *out = NULL;
    if (!c) return (sg_err){"kv: sg_kv_new got a NULL cfg"};
    if (!kv_be.alloc || !kv_be.free_ || !kv_be.host)
        return (sg_err){"kv: no allocation backend registered (call sg_kv_set_backend)"};
    if (!c->n_layers) return (sg_err){"kv: cfg has zero layers"};
    if (!c->full_attn_interval) return (sg_err){"kv: full_attn_interval is zero"};
    const uint64_t esz = kv_dtype == SG_T_F16 ? 2 : kv_dtype == SG_T_F32 ? 4 : 0;
    if (!esz) return (sg_err){"kv: kv_dtype must be SG_T_F16 or SG_T_F32"};
    if (!cap) cap = SG_KV_CAP_DEFAULT;
    if (cap > SG_KV_CAP_MAX) return (sg_err){"kv: cap exceeds SG_KV_CAP_MAX (262144)"};

    uint32_t n_attn = 0;
    for (uint32_t l = 0; l < c->n_layers; l++) n_attn += is_attn_layer(c, l);
    const uint32_t n_gdn = c->n_layers - n_attn;
    uint64_t one = 0, conv_bytes = 0, s_bytes = 0, cd = 0;
    if (n_attn) {
        const uint64_t width = (uint64_t)c->n_kv_heads * c->head_dim;
        if (!width || width > DIM_MAX || !mul_ok(width * esz, cap, &one) || !one)
            return (sg_err){"kv: attention KV size is zero, implausible or overflows"};
    }
    if (n_gdn) {
        if (!c->n_v_heads || !c->head_v_dim || !c->head_k_dim || !c->conv_kernel)
            return (sg_err){"kv: model has DeltaNet layers but no DeltaNet dims"};
        const uint64_t kd = (uint64_t)c->n_k_heads * c->head_k_dim, vd = (uint64_t)c->n_v_heads * c->head_v_dim;
        if (kd > DIM_MAX || vd > DIM_MAX || !(cd = 2 * kd + vd) || cd > DIM_MAX)
            return (sg_err){"kv: conv_dim is zero or implausibly large"};
        uint64_t se;
        if (!mul_ok(vd, c->head_k_dim, &se) || !mul_ok(se, 4, &s_bytes) ||
            !mul_ok(cd * 4, (uint64_t)c->conv_kernel - 1, &conv_bytes))
            return (sg_err){"kv: DeltaNet state size overflows"};
        if (!s_bytes) return (sg_err){"kv: DeltaNet state S size is zero"};
    }

    sg_kv *kv = calloc(1, sizeof *kv);
    if (!kv) return (sg_err){"kv: out of memory"};
    kv->cfg = *c;
    kv->cap = cap;
    kv->dtype = kv_dtype;
    kv->free_ = kv_be.free_;
    kv->host = kv_be.host;
    kv->conv_bytes = conv_bytes;
    kv->s_bytes = s_bytes;
    kv->buf = calloc((size_t)c->n_layers * 4, sizeof *kv->buf);
    if (!kv->buf) { free(kv); return (sg_err){"kv: out of memory"}; }
    for (uint32_t l = 0; l < c->n_layers; l++) {
        void **b = kv->buf + (size_t)l * 4;
        const uint64_t sz[4] = {is_attn_layer(c, l) ? one : 0, is_attn_layer(c, l) ? one : 0,
                                is_attn_layer(c, l) ? 0 : conv_bytes, is_attn_layer(c, l) ? 0 : s_bytes};
        for (int k = 0; k < 4; k++) {
            if (!sz[k]) continue;
            sg_err e = kv_be.alloc(g, sz[k], &b[k], NULL);
            if (sg_failed(e)) { sg_kv_free(kv); return e; }
        }
    }
    const uint64_t kv_total = (uint64_t)n_attn * 2 * one, st_total = (uint64_t)n_gdn * (conv_bytes + s_bytes);
    fprintf(stderr, "kv: cap=%u dtype=%s layers=%u (full-attn=%u deltanet=%u)\n", cap,
            kv_dtype == SG_T_F16 ? "f16" : "f32", c->n_layers, n_attn, n_gdn);
    if (n_attn)
        fprintf(stderr, "kv: per full-attn layer: K=%llu V=%llu bytes\n", (unsigned long long)one,
                (unsigned long long)one);
    if (n_gdn)
        fprintf(stderr, "kv: per deltanet layer: conv=%llu S=%llu bytes (conv_dim=%llu)\n",
                (unsigned long long)conv_bytes, (unsigned long long)s_bytes, (unsigned long long)cd);
    fprintf(stderr, "kv: totals: K+V=%llu (%.2f GiB) deltanet=%llu bytes\n", (unsigned long long)kv_total,
            (double)kv_total / (1u << 30), (unsigned long long)st_total);
    *out = kv;
    return SG_OK;
}

/* Back to position 0. The conv tails and S are zeroed through their host
 * views (what the DeltaNet step reads unconditionally); K/V are left as they
 * are, since nothing reads past `used`. With the GPU backend the host view is
 * sg_gpu_alloc's mirror, which the one-shots upload before each launch. */
void sg_kv_reset(sg_kv *kv) {
    if (!kv) return;
    kv->used = 0;
    for (uint32_t l = 0; l < kv->cfg.n_layers; l++) {
        void **b = kv->buf + (size_t)l * 4;
        void *h;
        if (b[KV_CONV] && (h = kv->host(b[KV_CONV]))) memset(h, 0, (size_t)kv->conv_bytes);
        if (b[KV_S] && (h = kv->host(b[KV_S]))) memset(h, 0, (size_t)kv->s_bytes);
    }
}

sg_err sg_kv_advance(sg_kv *kv, uint32_t n) {
    if (!kv) return (sg_err){"kv: sg_kv_advance got a NULL kv"};
    if ((uint64_t)kv->used + n > kv->cap) return (sg_err){"kv: advance would exceed cap"};
    kv->used += n;
    return SG_OK;
}

uint32_t sg_kv_used(const sg_kv *kv) { return kv ? kv->used : 0; }
uint32_t sg_kv_cap(const sg_kv *kv) { return kv ? kv->cap : 0; }

static void *kv_get(const sg_kv *kv, uint32_t layer, int which) {
    return (kv && layer < kv->cfg.n_layers) ? kv->buf[(size_t)layer * 4 + which] : NULL;
}
void *sg_kv_k(const sg_kv *kv, uint32_t layer) { return kv_get(kv, layer, KV_K); }
void *sg_kv_v(const sg_kv *kv, uint32_t layer) { return kv_get(kv, layer, KV_V); }
void *sg_kv_conv(const sg_kv *kv, uint32_t layer) { return kv_get(kv, layer, KV_CONV); }
void *sg_kv_s(const sg_kv *kv, uint32_t layer) { return kv_get(kv, layer, KV_S); }
