/* kv.c - KV-cache / DeltaNet-state size math and the f16 conversions.
 *
 * Interface: sg_kv_bytes, sg_kv_state_bytes, sg_f32_to_f16, sg_f16_to_f32
 * (reference surge.h:1456-1464; behaviour of reference src/kv.c:88-224).
 * The sizes are pure functions of the config: full-attention layers
 * ((L+1) % full_attn_interval == 0) hold separate K and V of
 * [cap, n_kv_heads, head_dim]; DeltaNet layers hold a conv tail
 * [conv_kernel-1, conv_dim] and S [n_v_heads, head_v_dim, head_k_dim] in f32.
 * Both return 0 for an invalid dtype, cap > SG_KV_CAP_MAX, a dimension above
 * 2^24 or a u64 overflow. The GPU state in hip.c allocates exactly these
 * byte counts (plus the conv ring slot it keeps for in-place updates).
 */
#include "surge.h"

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
