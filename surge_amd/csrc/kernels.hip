// kernels.hip - hand-written CDNA4 (gfx950) kernels for the batch-1 decode
// hot path, with extern "C" launchers for the C host layer (hip.c).
//
// Reference behaviour each kernel reproduces (reference files):
//   Q8_0 GEMV            src/ref.c:638-663, src/kernels.metal:227-250
//   RMSNorm / per-head   src/ref.c:113-125, src/kernels.metal:82-104, :611-635
//   RoPE (half split)    src/ref.c:561-606, src/kernels.metal:641-663
//   fp16 KV store        src/kv.c:152-190, src/kernels.metal:432-441
//   split-K attention    src/ref.c:416-555, src/kernels_splitk.metal:473-683
//   LSE combine          src/ref.c:256-373, src/kernels_splitk.metal:308-364
//   output gate          src/ref.c:185-188, src/kernels.metal:668-679
//   conv1d step          src/ref.c:669-706, src/kernels.metal:520-548
//   DeltaNet gates/step  src/ref.c:127-170,708-739, src/kernels.metal:742-805
//   RMSNormGated         src/ref.c:1322-1330, src/kernels.metal:109-134
//   argmax               src/greedy.c:17-27
//
// Design rules (MI355X, 64-wide waves):
//   - every reduction is a fixed tree (xor butterflies inside a wave, then a
//     fixed-order fold across waves), no atomics: reruns are bit-identical;
//   - fp32 arithmetic with IEEE division/sqrt and libm-accurate exp/log (no
//     fast-math); f16 denormal scales decode exactly;
//   - the GEMV streams 16-byte loads of int8 weights, coalesced along a row,
//     with the input vector staged once per workgroup in LDS.
#include <type_traits>
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <string.h>

#include "kernels.h"

#define TPB 256

// ---------------------------------------------------------------------------
// helpers
// ---------------------------------------------------------------------------

// Cross-lane moves without the LDS crossbar (gfx950): DPP lane selects inside
// a row of 16 lanes and the permlane swaps across rows / half-waves.
//   xor1: quad_perm [1,0,3,2]      xor2: quad_perm [2,3,0,1]
//   mir8: row_half_mirror (i <-> 7-i in each 8 lanes; flips bits 0..2)
//   xor8: row_ror:8 (i <-> i^8 in each row)
//   xor16 / xor32: v_permlane16_swap / v_permlane32_swap of v with itself
template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_xor1(float v) { return dppf<0xB1>(v); }
__device__ __forceinline__ float lane_xor2(float v) { return dppf<0x4E>(v); }
__device__ __forceinline__ float lane_mir8(float v) { return dppf<0x141>(v); }
__device__ __forceinline__ float lane_xor8(float v) { return dppf<0x128>(v); }
__device__ __forceinline__ float lane_xor16(float v) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false, false);
    return __int_as_float((threadIdx.x & 16) ? p[0] : p[1]);
}
__device__ __forceinline__ float lane_xor32(float v) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
    return __int_as_float((threadIdx.x & 32) ? p[0] : p[1]);
}
// Exact partner l ^ O for any power-of-two O.
template <int O>
__device__ __forceinline__ float lane_xor(float v) {
    if (O == 1) return lane_xor1(v);
    if (O == 2) return lane_xor2(v);
    if (O == 8) return lane_xor8(v);
    if (O == 16) return lane_xor16(v);
    if (O == 32) return lane_xor32(v);
    return __shfl_xor(v, O, 64);
}
__device__ __forceinline__ float lane_read(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
// Butterfly sum / max over the 64 lanes; every lane ends with the same bits
// (each step adds a pair in both orders, and + / max commute).
__device__ __forceinline__ float wave_sum(float v) {
    v += lane_xor1(v);
    v += lane_xor2(v);
    v += lane_mir8(v);
    v += lane_xor8(v);
    v += lane_xor16(v);
    v += lane_xor32(v);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, lane_xor1(v));
    v = fmaxf(v, lane_xor2(v));
    v = fmaxf(v, lane_mir8(v));
    v = fmaxf(v, lane_xor8(v));
    v = fmaxf(v, lane_xor16(v));
    v = fmaxf(v, lane_xor32(v));
    return v;
}
// Sum over all 256 threads of a workgroup; every thread gets the same value.
__device__ __forceinline__ float block_sum(float v, float *red) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
// Streaming (non-temporal) 16-byte load: weights are read once per token.
__device__ __forceinline__ uint4 ldnt(const uint4 *p) {
    const v4u v = __builtin_nontemporal_load((const v4u *)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }
__device__ __forceinline__ uint16_t f2h(float f) { return __half_as_ushort(__float2half_rn(f)); }

// sigmoid split on the sign so exp never overflows (ref.c:127-134).
__device__ __forceinline__ float sigm(float x) {
    if (x >= 0.0f) return 1.0f / (1.0f + expf(-x));
    float e = expf(x);
    return e / (1.0f + e);
}
__device__ __forceinline__ float silu(float x) { return x * sigm(x); }
// max(x,0) + log1p(e^-|x|) (ref.c:136-142).
__device__ __forceinline__ float softplus(float x) { return fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x))); }

__device__ __forceinline__ uint32_t dev_n_splits(uint32_t seq, uint32_t cap) {
    uint32_t n = (seq + SGK_KEYS_PER_SPLIT - 1) / SGK_KEYS_PER_SPLIT;
    n = n < 1 ? 1 : n;
    cap = cap ? cap : SGK_MAX_SPLITS;
    return n > cap ? cap : n;
}

// ---------------------------------------------------------------------------
// GEMV: input staging prologue
// ---------------------------------------------------------------------------

// Stage the input vector in LDS with 16-byte loads, in two phases so a
// kernel can put its first weight loads between them: stage_issue requests
// every float4 of x (and of the norm weight w for PRO_RMS) this thread stages,
// all in flight at once (K per thread cover rows up to K*NT*4 columns; wider
// rows finish with a strided loop); stage_finish stores them to LDS. The
// loads are unconditional with the index clamped to the last float4, so no
// branch separates them and each waits only for its own data. PRO_RMS stages
// x*w and returns the RMS factor 1/sqrt(mean(x^2) + eps) (ref.c:113-125) for
// the epilogue to apply to each row sum: W(x*r*w) = r * W(x*w). Other
// prologues return 1. Needs x and w 16-byte aligned (every buffer of this
// library is).
// PRO_GATED keeps the step's gated product silu(z) * (y * w) in v and the
// per-block sums of y^2 of head t (thread t < heads) in gs.
template <int PRO, int NT, int K>
struct xstage {
    float4 v[K], g[PRO == SGK_PRO_RMS ? K : 1];
    float gs[PRO == SGK_PRO_GATED ? SGK_GDN_BLOCKS : 1];
};

template <int PRO, int NT, int K>
__device__ __forceinline__ void stage_issue(const sgk_gemv &a, xstage<PRO, NT, K> &st) {
    const uint32_t n4 = a.cols >> 2, t = threadIdx.x;
    if (!n4) return;
    const float4 *x4 = (const float4 *)a.x, *w4 = (const float4 *)a.nw;
    if (PRO == SGK_PRO_GATED) {
        const uint32_t nh = a.cols / a.gdv, hh = min(t, nh - 1);
#pragma unroll
        for (uint32_t b = 0; b < SGK_GDN_BLOCKS; b++) st.gs[b] = a.gss[hh * SGK_GDN_BLOCKS + b];
#pragma unroll
        for (int k = 0; k < K; k++) st.v[k] = x4[min(t + (uint32_t)k * NT, n4 - 1)];
        return;
    }
#pragma unroll
    for (int k = 0; k < K; k++) {
        const uint32_t i = min(t + (uint32_t)k * NT, n4 - 1);
        st.v[k] = x4[i];
        if (PRO == SGK_PRO_RMS) st.g[k] = w4[i];
    }
}

// Staged x layout of the Q8_0 GEMVs (CH): chunks of 16 columns go in blocks
// of 64; block b holds four planes of 65 float4s, float4 j of chunk c (x
// columns 16c+4j .. +3) at (c/64)*260 + j*65 + c%64. The 64 lanes of a wave,
// reading chunks c..c+63, then read 1 KB of consecutive LDS per float4 (no
// bank conflicts; the linear layout puts lanes 64 bytes apart) at constant
// offsets from one address, and the staging writes of one chunk's four
// float4s land in different banks (the 65th float4 of a plane is padding).
// Without CH (the f32 GEMV) x is linear.
#define XS_CH_BLK 260
// k_gemv_q8 stages x chunked behind the RMSNorm prologue and linearly
// otherwise: the output projections (prologue-less, or the gated one after a
// multi-block DeltaNet step) and, at 2B, the down projections run about one
// row group per wave, and were 5-8% slower chunked (the conflict-free inner
// loop gains nothing there).
#define GEMV_CH(PRO) ((PRO) == SGK_PRO_RMS)
__host__ __device__ __forceinline__ uint32_t xs_ch_floats(uint32_t cols) {
    return ((cols / 16 + 63) / 64) * XS_CH_BLK * 4;
}
template <bool CH>
__device__ __forceinline__ uint32_t xs4_at(uint32_t i) {
    const uint32_t c = i >> 2;
    return CH ? (c >> 6) * XS_CH_BLK + (i & 3) * 65 + (c & 63) : i;
}

template <int PRO, int NT, int K, bool CH = false>
__device__ __forceinline__ float stage_finish(const sgk_gemv &a, xstage<PRO, NT, K> &st, float *xs) {
    __shared__ float red[NT / 64];
    const uint32_t n = a.cols, t = threadIdx.x, n4 = n >> 2;
    if (PRO == SGK_PRO_GATED) {
        // RMSNormGated of the DeltaNet readout (ref.c:1322-1330) finished:
        // head hh's factor r = rsqrt(mean y^2 + eps) from its row blocks' sums
        // of squares (added in block order), then x = (silu(z) * (y * w)) * r,
        // the step having written the product in parentheses.
        // The loads were issued by stage_issue (K float4s per thread cover
        // every column: the launcher holds cols <= K*NT*4 and heads <=
        // SGK_GATED_MAX_HEADS <= NT).
        __shared__ float rh[SGK_GATED_MAX_HEADS];
        const uint32_t nh = n / a.gdv;
        if (t < nh) {
            float tot = 0.0f;
#pragma unroll
            for (uint32_t b = 0; b < SGK_GDN_BLOCKS; b++) tot += st.gs[b];
            rh[t] = 1.0f / sqrtf(tot / (float)a.gdv + a.eps);
        }
        __syncthreads();
        float4 *s4 = (float4 *)xs;
#pragma unroll
        for (int k = 0; k < K; k++) {
            const uint32_t i = t + (uint32_t)k * NT;
            if (i < n4) {
                const float4 xv = st.v[k];
                const float r = rh[(4 * i) / a.gdv];
                s4[xs4_at<CH>(i)] = make_float4(xv.x * r, xv.y * r, xv.z * r, xv.w * r);
            }
        }
        __syncthreads();
        return 1.0f;
    }
    const float4 *x4 = (const float4 *)a.x, *w4 = (const float4 *)a.nw;
    float4 *s4 = (float4 *)xs;
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < K; k++) {
        const uint32_t i = t + (uint32_t)k * NT;
        if (i < n4) {
            float4 v = st.v[k];
            if (PRO == SGK_PRO_RMS) {
                const float4 g = st.g[k];
                ss = fmaf(v.x, v.x, ss); ss = fmaf(v.y, v.y, ss);
                ss = fmaf(v.z, v.z, ss); ss = fmaf(v.w, v.w, ss);
                v.x *= g.x; v.y *= g.y; v.z *= g.z; v.w *= g.w;
            }
            s4[xs4_at<CH>(i)] = v;
        }
    }
    for (uint32_t i = t + (uint32_t)K * NT; i < n4; i += NT) {   // rows wider than K*NT*4
        float4 v = x4[i];
        if (PRO == SGK_PRO_RMS) {
            const float4 g = w4[i];
            ss = fmaf(v.x, v.x, ss); ss = fmaf(v.y, v.y, ss);
            ss = fmaf(v.z, v.z, ss); ss = fmaf(v.w, v.w, ss);
            v.x *= g.x; v.y *= g.y; v.z *= g.z; v.w *= g.w;
        }
        s4[xs4_at<CH>(i)] = v;
    }
    for (uint32_t i = 4 * n4 + t; i < n; i += NT) {       // cols % 4 tail (f32 test models; never with CH)
        float v = a.x[i];
        if (PRO == SGK_PRO_RMS) { ss = fmaf(v, v, ss); v *= a.nw[i]; }
        xs[i] = v;
    }
    if (PRO == SGK_PRO_RMS) {
        ss = wave_sum(ss);
        if ((t & 63) == 0) red[t >> 6] = ss;
    }
    __syncthreads();
    if (PRO != SGK_PRO_RMS) return 1.0f;
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < NT / 64; i += 2) tot += red[i] + red[i + 1];
    return 1.0f / sqrtf(tot / (float)n + a.eps);
}

// float4s per thread a TPB-thread workgroup's stage_issue keeps in flight:
// enough for rows of 8192 columns, the widest the row-group GEMV takes.
constexpr int XK = 8192 / 4 / TPB;
static_assert(SGK_GATED_MAX_HEADS <= TPB, "gated prologue: one thread per head's factor");

template <int PRO>
__device__ __forceinline__ float stage_x(const sgk_gemv &a, float *xs) {
    xstage<PRO, TPB, XK> st;
    stage_issue<PRO, TPB, XK>(a, st);
    return stage_finish<PRO, TPB, XK>(a, st, xs);
}

template <int EPI>
__device__ __forceinline__ void gemv_store(const sgk_gemv &a, uint32_t row, float v) {
    if (EPI == SGK_EPI_ADD) a.y[row] += v;
    else a.y[row] = v;
}

// Dot product of 16 int8 weights with 16 staged floats.
__device__ __forceinline__ float dot16(const uint4 q, const float4 x0, const float4 x1,
                                       const float4 x2, const float4 x3) {
    float s0, s1;
    s0 = (float)(int8_t)(q.x) * x0.x;
    s1 = (float)(int8_t)(q.x >> 8) * x0.y;
    s0 = fmaf((float)(int8_t)(q.x >> 16), x0.z, s0);
    s1 = fmaf((float)((int32_t)q.x >> 24), x0.w, s1);
    s0 = fmaf((float)(int8_t)(q.y), x1.x, s0);
    s1 = fmaf((float)(int8_t)(q.y >> 8), x1.y, s1);
    s0 = fmaf((float)(int8_t)(q.y >> 16), x1.z, s0);
    s1 = fmaf((float)((int32_t)q.y >> 24), x1.w, s1);
    s0 = fmaf((float)(int8_t)(q.z), x2.x, s0);
    s1 = fmaf((float)(int8_t)(q.z >> 8), x2.y, s1);
    s0 = fmaf((float)(int8_t)(q.z >> 16), x2.z, s0);
    s1 = fmaf((float)((int32_t)q.z >> 24), x2.w, s1);
    s0 = fmaf((float)(int8_t)(q.w), x3.x, s0);
    s1 = fmaf((float)(int8_t)(q.w >> 8), x3.y, s1);
    s0 = fmaf((float)(int8_t)(q.w >> 16), x3.z, s0);
    s1 = fmaf((float)((int32_t)q.w >> 24), x3.w, s1);
    return s0 + s1;
}

// ---------------------------------------------------------------------------
// Q8_0 GEMV, rows up to 8192 columns. Persistent 256-thread workgroups, as
// many as are resident at once (never more, so none waits for a slot), walk
// row groups with a grid stride; the grid is sized so every wave gets the same
// number of row groups. One wave owns R consecutive output rows at a time;
// lane l streams 16-byte chunks l, l+64, ... of each row (a chunk is half a
// Q8_0 block: 16 int8 and the block's f16 scale). The first row group's first
// chunks are requested before the prologue runs, so HBM is already busy while
// the input vector is staged.
// ---------------------------------------------------------------------------

template <int R>
struct gemv_chunk {
    uint4 q[R];
    uint16_t d[R];
};

template <int R>
__device__ __forceinline__ void gemv_load(gemv_chunk<R> &ch, const int8_t *qs, const uint16_t *d,
                                          uint32_t r0, uint32_t rows, uint32_t cols, uint32_t c) {
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint32_t rr = min(r0 + r, rows - 1);
        ch.q[r] = ldnt((const uint4 *)(qs + (size_t)rr * cols) + c);
        ch.d[r] = __builtin_nontemporal_load(d + (size_t)rr * (cols >> 5) + (c >> 1));   // read once per token, as the weights
    }
}

template <int R, bool CH>
__device__ __forceinline__ void gemv_fma(float *acc, const gemv_chunk<R> &ch, const float *xs, uint32_t c) {
    const float4 *xa = CH ? (const float4 *)xs + (c >> 6) * XS_CH_BLK + (c & 63) : (const float4 *)xs + 4 * c;
    const float4 a0 = xa[0], a1 = xa[CH ? 65 : 1], a2 = xa[CH ? 130 : 2], a3 = xa[CH ? 195 : 3];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = fmaf(h2f(ch.d[r]), dot16(ch.q[r], a0, a1, a2, a3), acc[r]);
}

// The end of a row group: each lane's partial sums of the R rows summed over
// the wave, scaled by post, and stored by the epilogue.
template <int R, int EPI>
__device__ __forceinline__ void gemv_finish(const sgk_gemv &a, float *acc, uint32_t r0, uint32_t lane, float post) {
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = wave_sum(acc[r]) * post;
    if (EPI == SGK_EPI_SWIGLU) {
        // rows come in (gate, up) pairs: y[i] = silu(gate_i) * up_i
#pragma unroll
        for (int p = 0; p < R / 2; p++)
            if (lane == (uint32_t)p && r0 + 2 * p + 1 < a.rows)
                a.y[(r0 >> 1) + p] = silu(acc[2 * p]) * acc[2 * p + 1];
    } else {
#pragma unroll
        for (int r = 0; r < R; r++)
            if (lane == (uint32_t)r && r0 + r < a.rows) gemv_store<EPI>(a, r0 + r, acc[r]);
    }
}

// One row group of R rows: every chunk of the rows, two chunks per step, the
// first chunk optionally already loaded (pre). post scales each row sum. CH:
// x staged in the chunked layout (xs4_at<true>), else linear.
template <int R, int EPI, bool PRE, bool CH>
__device__ __forceinline__ void gemv_group(const sgk_gemv &a, const float *xs, uint32_t g, uint32_t lane,
                                           const gemv_chunk<R> *pre, float post) {
    const uint32_t cols = a.cols, nch = cols >> 4, r0 = g * R;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    uint32_t c = lane;
    if (PRE) {
        if (c < nch) gemv_fma<R, CH>(acc, *pre, xs, c);
        c += 64;
    }
    for (; c + 64 < nch; c += 128) {
        gemv_chunk<R> ca, cb;
        gemv_load<R>(ca, a.qs, a.d, r0, a.rows, cols, c);
        gemv_load<R>(cb, a.qs, a.d, r0, a.rows, cols, c + 64);
        gemv_fma<R, CH>(acc, ca, xs, c);
        gemv_fma<R, CH>(acc, cb, xs, c + 64);
    }
    if (c < nch) {
        gemv_chunk<R> ca;
        gemv_load<R>(ca, a.qs, a.d, r0, a.rows, cols, c);
        gemv_fma<R, CH>(acc, ca, xs, c);
    }
    gemv_finish<R, EPI>(a, acc, r0, lane, post);
}

template <int R, int PRO, int EPI>
__global__ void __launch_bounds__(TPB) k_gemv_q8(sgk_gemv a) {
    extern __shared__ float xs[];
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t nch = a.cols >> 4;
    const uint32_t ngroups = (a.rows + R - 1) / R, gstride = gridDim.x * (TPB / 64);
    uint32_t g = blockIdx.x * (TPB / 64) + wave;
    const bool have = g < ngroups;
    xstage<PRO, TPB, XK> st;
    stage_issue<PRO, TPB, XK>(a, st);
    gemv_chunk<R> pre;
    if (have && lane < nch) gemv_load<R>(pre, a.qs, a.d, g * R, a.rows, a.cols, lane);
    const float post = stage_finish<PRO, TPB, XK, GEMV_CH(PRO)>(a, st, xs);
    if (!have) return;
    gemv_group<R, EPI, true, GEMV_CH(PRO)>(a, xs, g, lane, &pre, post);
    for (g += gstride; g < ngroups; g += gstride) gemv_group<R, EPI, false, GEMV_CH(PRO)>(a, xs, g, lane, nullptr, post);
}

// ---------------------------------------------------------------------------
// Q8_0 GEMV with a two-step load ring (the default behind the RMSNorm and
// gated prologues). The same row groups, lanes, chunks and summation order as
// k_gemv_q8 (so the same bits), but a wave walks its whole sequence of steps
// (row group g, chunks 128s + lane and 128s + 64 + lane) with two step
// buffers: while one step's FMAs run, the next step's chunks are already in
// flight, and a buffer is refilled two steps ahead as soon as its FMAs are
// done. k_gemv_q8 requests a step and waits for all of it, so its FMAs and
// the row-group ends ran with nothing of the wave in flight. Both buffers
// are requested before the input vector is staged.
// The wave index is read as a uniform value, so the step walk is scalar
// control flow with one exit; the compiler then tracks which loads are in
// flight exactly (a per-lane loop, or a second exit, made it wait for the
// other buffer too). The loads are unconditional buffer loads: a step past
// the wave's last one, a chunk past the row's end and a row past the matrix
// take an offset past the descriptor's range, which reads zeros without a
// memory request (clamped addresses instead re-read up to two steps per
// wave, 17 MB per gate/up launch).
// ---------------------------------------------------------------------------
#define RING_OOB 0x80000000u
struct ring_src {
    __amdgpu_buffer_rsrc_t q, d;
};

// A step's two chunks of the group's R rows; for the residual-add epilogue
// also y[r0 + lane] (lanes < R), read with the step's chunks so that the
// group's end does not wait on a load of its own (a read there would wait
// for every request in flight, the other buffer's too).
template <int R>
struct gemv_step {
    gemv_chunk<R> x, y;
    float yr;
};

template <int R>
__device__ __forceinline__ void ring_chunk(const sgk_gemv &a, const ring_src &rs, gemv_chunk<R> &ch, uint32_t r0,
                                           bool live, uint32_t c) {
#pragma unroll
    for (int r = 0; r < R; r++) {
        const bool ok = live && r0 + r < a.rows && c < (a.cols >> 4);
        const uint32_t qo = ok ? (r0 + r) * a.cols + 16 * c : RING_OOB;
        const uint32_t dof = ok ? ((r0 + r) * (a.cols >> 5) + (c >> 1)) * 2 : RING_OOB;
        const v4u v = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rs.q, (int)qo, 0, 2));   // nt
        ch.q[r] = make_uint4(v.x, v.y, v.z, v.w);
        ch.d[r] = __builtin_amdgcn_raw_buffer_load_b16(rs.d, (int)dof, 0, 2);   // nt (as the scales of k_gemv_q8)
    }
}

template <int R, int EPI>
__device__ __forceinline__ void ring_load(const sgk_gemv &a, const ring_src &rs, gemv_step<R> &b, uint32_t g,
                                          uint32_t s, uint32_t ngroups, uint32_t lane) {
    const bool live = g < ngroups;
    const uint32_t r0 = g * R;
    ring_chunk<R>(a, rs, b.x, r0, live, 128 * s + lane);
    ring_chunk<R>(a, rs, b.y, r0, live, 128 * s + 64 + lane);
    if (EPI == SGK_EPI_ADD) b.yr = a.y[min(r0 + min(lane, (uint32_t)R - 1), a.rows - 1)];
}

template <int R, int EPI, bool CH>
__device__ __forceinline__ void ring_fma(const sgk_gemv &a, const float *xs, const gemv_step<R> &b, float *acc,
                                         uint32_t g, uint32_t s, uint32_t spg, uint32_t lane, float post) {
    const uint32_t nch = a.cols >> 4, c = 128 * s + lane;
    if (c < nch) gemv_fma<R, CH>(acc, b.x, xs, c);
    if (c + 64 < nch) gemv_fma<R, CH>(acc, b.y, xs, c + 64);
    if (s == spg - 1) {
        if (EPI == SGK_EPI_ADD) {                   // y += row sum, y as read with this step
            const uint32_t r0 = g * R;
#pragma unroll
            for (int r = 0; r < R; r++) {
                acc[r] = wave_sum(acc[r]) * post;
                if (lane == (uint32_t)r && r0 + r < a.rows) a.y[r0 + r] = b.yr + acc[r];
            }
        } else {
            gemv_finish<R, EPI>(a, acc, g * R, lane, post);
        }
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = 0.0f;
    }
}

template <int R, int PRO, int EPI>
__global__ void __launch_bounds__(TPB) k_gemv_ring(sgk_gemv a) {
    extern __shared__ float xs[];
    constexpr bool CH = GEMV_CH(PRO);
    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nch = a.cols >> 4, spg = (nch + 127) / 128;
    // Rounds of one row group per wave over consecutive groups, a
    // workgroup's waves on adjacent groups: all waves stream one compact
    // window of rows at a time. Measured over a 27B token against this
    // order: contiguous ranges per wave 6% slower, and a round's groups
    // dealt wave-major (wave j of workgroup b at j * blocks + b, which spreads
    // a partial last round over the CUs) 3% slower.
    const uint32_t ngroups = (a.rows + R - 1) / R, gstride = gridDim.x * (TPB / 64);
    uint32_t g = blockIdx.x * (TPB / 64) + wave, s = 0;
    uint32_t gb = g, sb = s;                        // buffer b's step: one after buffer a's
    if (++sb == spg) { sb = 0; gb += gstride; }
    ring_src rs;
    rs.q = __builtin_amdgcn_make_buffer_rsrc((void *)a.qs, (short)0, (int)(a.rows * a.cols), 0x00020000);
    rs.d = __builtin_amdgcn_make_buffer_rsrc((void *)a.d, (short)0, (int)(a.rows * (a.cols >> 5) * 2), 0x00020000);
    xstage<PRO, TPB, XK> st;
    stage_issue<PRO, TPB, XK>(a, st);
    gemv_step<R> ba, bb;
    ring_load<R, EPI>(a, rs, ba, g, s, ngroups, lane);
    __builtin_amdgcn_sched_barrier(0);              // keep a's requests ahead of b's
    ring_load<R, EPI>(a, rs, bb, gb, sb, ngroups, lane);
    __builtin_amdgcn_sched_barrier(0);
    const float post = stage_finish<PRO, TPB, XK, CH>(a, st, xs);
    if (g >= ngroups) return;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    while (true) {
        ring_fma<R, EPI, CH>(a, xs, ba, acc, g, s, spg, lane, post);
        g = gb; s = sb;                             // a's next step: one after b's
        if (++s == spg) { s = 0; g += gstride; }
        ring_load<R, EPI>(a, rs, ba, g, s, ngroups, lane);
        if (gb < ngroups) ring_fma<R, EPI, CH>(a, xs, bb, acc, gb, sb, spg, lane, post);
        gb = g; sb = s;                             // b's next step: one after a's
        if (++sb == spg) { sb = 0; gb += gstride; }
        ring_load<R, EPI>(a, rs, bb, gb, sb, ngroups, lane);
        if (g >= ngroups) break;
    }
}

// f32-weight GEMV (small test models only): one wave per row pair.
template <int PRO, int EPI>
__global__ void __launch_bounds__(TPB) k_gemv_f32(sgk_gemv a) {
    extern __shared__ float xs[];
    const float post = stage_x<PRO>(a, xs);
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t ngroups = (a.rows + 1) / 2;
    for (uint32_t g = blockIdx.x * (TPB / 64) + wave; g < ngroups; g += gridDim.x * (TPB / 64)) {
        const uint32_t r0 = 2 * g, r1 = min(r0 + 1, a.rows - 1);
        const float *w0 = a.wf + (size_t)r0 * a.cols, *w1 = a.wf + (size_t)r1 * a.cols;
        float s0 = 0.0f, s1 = 0.0f;
        for (uint32_t c = lane; c < a.cols; c += 64) {
            s0 = fmaf(w0[c], xs[c], s0);
            s1 = fmaf(w1[c], xs[c], s1);
        }
        s0 = wave_sum(s0) * post;
        s1 = wave_sum(s1) * post;
        if (lane == 0) {
            if (EPI == SGK_EPI_SWIGLU) {
                if (r0 + 1 < a.rows) a.y[g] = silu(s0) * s1;
            } else {
                gemv_store<EPI>(a, r0, s0);
                if (r0 + 1 < a.rows) gemv_store<EPI>(a, r0 + 1, s1);
            }
        }
    }
}


// Workgroups of `kern` (tpb threads, lds bytes of dynamic LDS) that fit on one
// CU at once: the wave slots its VGPR count leaves per SIMD, and the LDS.
template <typename K>
static uint32_t resident_per_cu(K kern, uint32_t tpb, size_t lds) {
    hipFuncAttributes at;
    int vg = 128, shm = 0;
    if (hipFuncGetAttributes(&at, (const void *)kern) == hipSuccess) {
        vg = at.numRegs > 0 ? at.numRegs : 128;
        shm = (int)at.sharedSizeBytes;
    }
    int waves_simd = 512 / ((vg + 7) & ~7);
    waves_simd = waves_simd > 8 ? 8 : waves_simd;
    const int by_waves = 4 * waves_simd / (int)(tpb / 64);
    const size_t per_wg = ((lds + (size_t)shm + 511) & ~(size_t)511);
    const int by_lds = per_wg ? (int)(163840 / per_wg) : 64;
    int api = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&api, (const void *)kern, (int)tpb, lds) != hipSuccess) api = 64;
    int n = by_waves < by_lds ? by_waves : by_lds;
    n = api < n ? api : n;
    return n < 1 ? 1u : (uint32_t)n;
}

static int device_cus() {
    static int cus = 0;
    if (!cus && hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0) != hipSuccess) cus = 256;
    return cus;
}

// The prefill GEMM's form, read at every launch: the wide warp-specialised
// kernel (k_gemm_q8_wide, 128 x 256 tiles, one workgroup per CU) unless
// SURGE_GEMM_WS is "0" (k_gemm_q8_mfma: 128 x 128 tiles, 256 threads, two
// per CU) or SURGE_GEMM_WIDE is "0" (k_gemm_q8_ws: 128 x 128 tiles, 512
// threads, two per CU). All three give the same bits.
enum { GEMM_PLAIN, GEMM_WS, GEMM_WIDE };
static int gemm_kind() {
    const char *e = getenv("SURGE_GEMM_WS");
    if (e && e[0] == '0' && !e[1]) return GEMM_PLAIN;
    e = getenv("SURGE_GEMM_WIDE");
    if (e && e[0] == '0' && !e[1]) return GEMM_WS;
    return GEMM_WIDE;
}
// Workgroups of the prefill GEMM resident at once: one per CU for the wide
// form, two for the others (their LDS). SURGE_GEMM_SLOTS (decimal, >= 1)
// overrides it, for tests that exercise the round split on small shapes.
static uint32_t gemm_slots(int kind) {
    const char *e = getenv("SURGE_GEMM_SLOTS");
    if (e && *e) {
        char *end = NULL;
        const unsigned long v = strtoul(e, &end, 10);
        if (end && !*end && v >= 1 && v <= 65536) return (uint32_t)v;
    }
    return (kind == GEMM_WIDE ? 1u : 2u) * (uint32_t)device_cus();
}

static hipError_t allow_lds(const void *kern, size_t lds) {
    if (lds <= 65536) return hipSuccess;
    if (lds > 163840) return hipErrorInvalidValue;
    return hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
}



// Row groups the busiest CU carries when `blocks` workgroups of TPB/64 waves
// split `groups` row groups (wave i of the grid-stride order takes
// ceil or floor of groups/waves) and workgroup b runs on CU b mod cus.
static uint32_t gemv_cu_load(uint32_t groups, uint32_t blocks, uint32_t cus) {
    const uint32_t wpb = TPB / 64, waves = blocks * wpb, q = groups / waves, r = groups % waves;
    uint32_t worst = 0;
    for (uint32_t c = 0; c < cus && c < blocks; c++) {
        uint32_t load = 0;
        for (uint32_t b = c; b < blocks; b += cus)
            for (uint32_t w = 0; w < wpb; w++) load += q + (b * wpb + w < r ? 1u : 0u);
        worst = load > worst ? load : worst;
    }
    return worst;
}

// Grid for the row-group GEMV: resident workgroups only. Candidates are the
// wave-balanced count (every wave gets ceil(groups / waves) groups, as few
// waves as that allows) and every whole number of workgroups per CU up to
// residency; the one whose busiest CU carries the fewest row groups wins, ties
// going to the count nearest three workgroups per CU (measured best on
// MI355X for these kernels: enough waves to hide latency, few prologues).
static uint32_t gemv_grid(uint32_t groups, uint32_t per) {
    const uint32_t cus = (uint32_t)device_cus(), wpb = TPB / 64;
    const uint32_t max_waves = cus * per * wpb;
    const uint32_t k = (groups + max_waves - 1) / max_waves;
    const uint32_t waves = (groups + k - 1) / k;
    uint32_t best = (waves + wpb - 1) / wpb, best_load = gemv_cu_load(groups, best, cus);
    for (uint32_t m = 1; m <= per; m++) {
        const uint32_t b = cus * m, load = gemv_cu_load(groups, b, cus);
        const uint32_t d_new = b > 3 * cus ? b - 3 * cus : 3 * cus - b;
        const uint32_t d_old = best > 3 * cus ? best - 3 * cus : 3 * cus - best;
        if (load < best_load || (load == best_load && d_new < d_old)) { best = b; best_load = load; }
    }
    return best;
}

// Launch k_gemv_q8<R,...>: resident workgroups only, sized so every wave gets
// ceil(groups / waves) row groups and no wave gets one fewer than another by
// more than one (the caller may fix the count with tune_blocks).
template <int R, int PRO, int EPI>
static hipError_t launch_q8(const sgk_gemv &a, size_t lds, hipStream_t s) {
    auto kern = k_gemv_q8<R, PRO, EPI>;
    hipError_t e = allow_lds((const void *)kern, lds);
    if (e != hipSuccess) return e;
    static size_t seen_lds[8];                      // residency per LDS size, per instantiation
    static uint32_t seen_per[8];
    static int nseen = 0;
    uint32_t per = 0;
    for (int i = 0; i < nseen; i++)
        if (seen_lds[i] == lds) per = seen_per[i];
    if (!per) {
        per = resident_per_cu(kern, TPB, lds);
        if (nseen < 8) { seen_lds[nseen] = lds; seen_per[nseen] = per; nseen++; }
    }
    const uint32_t groups = (a.rows + R - 1) / R;
    uint32_t blocks = a.tune_blocks;
    if (!blocks) {                                  // per (groups) of this instantiation
        static uint32_t seen_g[16], seen_b[16];
        static int ng = 0;
        for (int i = 0; i < ng && !blocks; i++)
            if (seen_g[i] == groups) blocks = seen_b[i];
        if (!blocks) {
            blocks = gemv_grid(groups, per);
            if (ng < 16) { seen_g[ng] = groups; seen_b[ng] = blocks; ng++; }
        }
    }
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(TPB), lds, s, a);
    return hipGetLastError();
}

// Launch k_gemv_ring<2,...>: two workgroups per CU (8 waves, each with two
// steps in flight), fewer if there are fewer row groups than waves. Measured
// on MI355X over the 27B shapes (one workgroup per CU, 1.5, 2, 2.5 and 3):
// two per CU was fastest for every shape it takes; three, with the ring, put
// more in flight than the memory system serves faster.
template <int PRO, int EPI>
static hipError_t launch_ring(const sgk_gemv &a, size_t lds, hipStream_t s) {
    auto kern = k_gemv_ring<2, PRO, EPI>;
    hipError_t e = allow_lds((const void *)kern, lds);
    if (e != hipSuccess) return e;
    static size_t seen_lds[8];
    static uint32_t seen_per[8];
    static int nseen = 0;
    uint32_t per = 0;
    for (int i = 0; i < nseen; i++)
        if (seen_lds[i] == lds) per = seen_per[i];
    if (!per) {
        per = resident_per_cu(kern, TPB, lds);
        if (nseen < 8) { seen_lds[nseen] = lds; seen_per[nseen] = per; nseen++; }
    }
    const uint32_t groups = (a.rows + 1) / 2, wpb = TPB / 64;
    uint32_t blocks = (uint32_t)device_cus() * (per < 2 ? per : 2u);
    if ((groups + wpb - 1) / wpb < blocks) blocks = (groups + wpb - 1) / wpb;
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(TPB), lds, s, a);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Balanced Q8_0 GEMV (the default for Q8_0 matrices whose width is a multiple
// of 1024). One BT-thread workgroup per CU. Workgroup b owns the row groups
// [b*G/NB, (b+1)*G/NB) of 2 rows; their steps (group, 1024-column block j),
// group-major, are dealt to its waves in equal contiguous ranges, so every
// wave of the chip has the same number of 2 KB steps to within one (the
// grid-stride kernel above gives whole row groups to waves, up to 12% apart).
// A wave streams a step as k_gemv_q8<2> streams a chunk pair (lane l: chunk
// l + 64 j of both rows, f32 FMA per chunk) and keeps BP steps in flight in
// a register ring indexed statically; all BP of the first steps are
// requested (after x) before x is staged, so HBM streams while x arrives. Each wave
// writes one wave-reduced partial per row group it touched into LDS (the
// other waves' slots of that group are 0); the workgroup then adds a group's
// slots in wave order (adding zeros is exact: a group one wave did whole
// keeps k_gemv_q8's bits) and applies the prologue's factor and the
// epilogue. EPI_ADD may update y in place: a workgroup reads its rows of y
// (into registers, one row per thread) before it writes them.
// ---------------------------------------------------------------------------
#define BT 768
#define BW (BT / 64)
// Steps in flight per wave: 3 (72 KB per CU). Over a 27B decode token, 2 and
// 3 ran alike and 0.4-0.7% faster than 4; 6 was 2% slower.
#define BP 3
constexpr int BXK_NONE = (SGK_BAL_MAX_COLS + 4 * BT - 1) / (4 * BT);
constexpr int BXK_RMS = (SGK_BAL_MAX_RMS_COLS + 4 * BT - 1) / (4 * BT);

__host__ __device__ __forceinline__ uint32_t bal_lds_floats(uint32_t rows, uint32_t cols, uint32_t nb) {
    const uint32_t G = (rows + 1) / 2, ng = (G + nb - 1) / nb;
    return xs_ch_floats(cols) + ng * (BW * 2 + 2);
}

template <int PRO, int EPI, bool IL>
__global__ void __launch_bounds__(BT) k_gemv_bal(sgk_gemv a) {
    extern __shared__ float lds[];
    const uint32_t lane = threadIdx.x & 63, t = threadIdx.x;
    const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nsteps = a.cols >> 10, G = (a.rows + 1) / 2, nb = gridDim.x, b = blockIdx.x;
    // IL: the workgroup's k-th group is b + k*nb (all workgroups stream one
    // compact window at a time); else the contiguous range from g0
    const uint32_t g0 = IL ? b : (uint32_t)((uint64_t)b * G / nb);
    const uint32_t ng = IL ? (b < G ? (G - b + nb - 1) / nb : 0) : (uint32_t)((uint64_t)(b + 1) * G / nb) - g0;
    const uint32_t gs = IL ? nb : 1;
    if (!ng) return;
    const uint32_t T = ng * nsteps, s0 = w * T / BW, ns = (w + 1) * T / BW - s0;
    float *xs = lds, *part = lds + xs_ch_floats(a.cols), *res = part + ng * BW * 2;
    // The ring's loads are range-checked buffer loads (as k_gemv_ring's): a
    // step past the wave's range reads zeros without a memory request, so
    // every slot is refilled unconditionally and the walk below is one loop
    // with one exit, whose waits the compiler counts exactly (a steady loop
    // plus peeled tails made it copy the ring into other registers at the
    // loop's entry, which waited for all BP steps).
    ring_src rs;
    rs.q = __builtin_amdgcn_make_buffer_rsrc((void *)a.qs, (short)0, (int)(a.rows * a.cols), 0x00020000);
    rs.d = __builtin_amdgcn_make_buffer_rsrc((void *)a.d, (short)0, (int)(a.rows * (a.cols >> 5) * 2), 0x00020000);
    gemv_chunk<2> ring[BP];
    auto issue = [&](gemv_chunk<2> &ch, uint32_t k, uint32_t j, bool live) {
        ring_chunk<2>(a, rs, ch, (g0 + k * gs) * 2, live, lane + 64 * j);
    };
    auto next = [&](uint32_t &k, uint32_t &j) { if (++j == nsteps) { j = 0; k++; } };
    // x is requested first and the ring after it: the loads return in order,
    // so x requested behind the ring's BP steps (72 KB per CU) waited for all
    // of them. For EPI_ADD thread t < 2 * ng holds y of the workgroup's row t
    // in a register, requested with the ring (the launcher keeps 2 * ng <=
    // BT): a read into LDS here made the staging wait for every request in
    // flight.
    constexpr int K = PRO == SGK_PRO_RMS ? BXK_RMS : BXK_NONE;
    xstage<PRO, BT, K> st;
    stage_issue<PRO, BT, K>(a, st);
    uint32_t ki = s0 / nsteps, ji = s0 % nsteps;
#pragma unroll
    for (int u = 0; u < BP; u++) {          // the first steps, in slot order
        issue(ring[u], ki, ji, (uint32_t)u < ns);
        next(ki, ji);
        __builtin_amdgcn_sched_barrier(0);
    }
    float yv = 0.0f;
    if (EPI == SGK_EPI_ADD) {
        const uint32_t i = min(t, 2 * ng - 1), row = (g0 + (i >> 1) * gs) * 2 + (i & 1);
        yv = a.y[min(row, a.rows - 1)];
    }
    for (uint32_t i = t; i < ng * BW * 2; i += BT) part[i] = 0.0f;
    const float post = stage_finish<PRO, BT, K, true>(a, st, xs);
    float acc[2] = {0.0f, 0.0f};
    uint32_t kc = s0 / nsteps, jc = s0 % nsteps;
    auto consume = [&](int u, uint32_t i) {
        gemv_fma<2, true>(acc, ring[u], xs, lane + 64 * jc);
        if (jc == nsteps - 1 || i == ns - 1) {
            acc[0] = wave_sum(acc[0]);
            acc[1] = wave_sum(acc[1]);
            if (lane < 2) part[(kc * BW + w) * 2 + lane] = lane == 0 ? acc[0] : acc[1];
            acc[0] = acc[1] = 0.0f;
        }
        next(kc, jc);
    };
    for (uint32_t i = 0; i < ns; i += BP) {
#pragma unroll
        for (int u = 0; u < BP; u++) {
            if (i + u < ns) consume(u, i + u);
            issue(ring[u], ki, ji, i + u + BP < ns);
            next(ki, ji);
        }
    }
    if (EPI == SGK_EPI_ADD && t < ng * 2) res[t] = yv;
    __syncthreads();
    for (uint32_t i = t; i < ng * 2; i += BT) {
        const uint32_t k = i >> 1, r = i & 1, row = (g0 + k * gs) * 2 + r;
        float v = 0.0f;
#pragma unroll
        for (uint32_t ww = 0; ww < BW; ww++) v += part[(k * BW + ww) * 2 + r];
        v *= post;
        if (EPI == SGK_EPI_SWIGLU) {
            const float u = __shfl_down(v, 1);
            if (r == 0 && row + 1 < a.rows) a.y[row >> 1] = silu(v) * u;
        } else if (row < a.rows) {
            a.y[row] = EPI == SGK_EPI_ADD ? res[i] + v : v;
        }
    }
}

// Which kernel takes a Q8_0 GEMV of `cols` columns (multiples of 1024 only)
// and prologue `pro`: 0 k_gemv_q8 or k_gemv_ring, 1 k_gemv_bal contiguous,
// 2 k_gemv_bal interleaved. By default the interleaved balanced kernel takes
// the GEMVs without a prologue longer than 4096 columns: the 27B down
// projection (17408 columns, 18.5 us against 20.2 for the row-front kernel
// it replaced, back-to-back over the layers) and the attention output
// projections of 6144 columns (27B decode 187.2-187.8 -> 187.6-187.9 tok/s,
// 2B 1251 -> 1263 tok/s with its 6144-column down projection, same boxes,
// alternating, same tokens). Contiguous ranges are slower than interleaved
// ones everywhere. SURGE_GEMV=q8|bal|bali forces one.
static int gemv_bal_on(uint32_t cols, int pro) {
    const char *e = getenv("SURGE_GEMV");
    if (e && e[0] == 'q' && e[1] == '8' && !e[2]) return 0;
    if (e && e[0] == 'b' && e[1] == 'a' && e[2] == 'l' && e[3] == 'i' && !e[4]) return 2;
    if (e && e[0] == 'b' && e[1] == 'a' && e[2] == 'l' && !e[3]) return 1;
    return pro == SGK_PRO_NONE && cols > 4096 ? 2 : 0;
}
// Whether a Q8_0 GEMV with a prologue (RMSNorm or gated) that k_gemv_bal
// does not take runs the ring form k_gemv_ring (the default) or the
// row-group form k_gemv_q8 (SURGE_GEMV=q8, or the tune_r / tune_blocks
// measurement overrides). Without a prologue k_gemv_q8 stays. The ring there
// ran the 2B shape's output and down projections (4-13 MB) 4% faster over a
// token, but it is not built: with those instantiations in the code object
// the 27B decode ran 0.5% slower on the same kernels (also with them
// present and never launched), a code-layout effect on the headline shape.
// The ring also loses to k_gemv_bal on the 17408-column down projection
// (20.3-21.7 against 18.7-19.4 us).
static int gemv_ring_on() {
    const char *e = getenv("SURGE_GEMV");
    return !(e && e[0] == 'q' && e[1] == '8' && !e[2]);
}

template <int PRO, int EPI>
static hipError_t launch_bal(const sgk_gemv &a, hipStream_t s) {
    auto kern = gemv_bal_on(a.cols, PRO) == 2 ? k_gemv_bal<PRO, EPI, true> : k_gemv_bal<PRO, EPI, false>;
    const uint32_t nb = (uint32_t)device_cus();
    const size_t lds = (size_t)bal_lds_floats(a.rows, a.cols, nb) * 4;
    hipError_t e = allow_lds((const void *)kern, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, dim3(nb), dim3(BT), lds, s, a);
    return hipGetLastError();
}

template <int PRO, int EPI>
static hipError_t gemv_dispatch(const sgk_gemv *a, hipStream_t s) {
    if (((uintptr_t)a->x & 15) || (PRO == SGK_PRO_RMS && ((uintptr_t)a->nw & 15))) return hipErrorInvalidValue;
    if (PRO == SGK_PRO_GATED && (!a->gss || !a->gdv || a->gdv % 4 || a->cols % a->gdv ||
                                 a->cols / a->gdv > SGK_GATED_MAX_HEADS || a->cols > (uint32_t)XK * TPB * 4))
        return hipErrorInvalidValue;
    if (!a->qs) {
        const size_t lds = (size_t)a->cols * 4;
        hipError_t e = allow_lds((const void *)k_gemv_f32<PRO, EPI>, lds);
        if (e != hipSuccess) return e;
        const uint32_t groups = (a->rows + 1) / 2;
        hipLaunchKernelGGL((k_gemv_f32<PRO, EPI>), dim3(min((groups + 3) / 4, 4096u)), dim3(TPB), lds, s, *a);
        return hipGetLastError();
    }
    if (PRO != SGK_PRO_GATED && gemv_bal_on(a->cols, PRO) && !a->tune_r && !a->tune_blocks && a->cols % 1024 == 0 &&
        2 * (((a->rows + 1) / 2 + (uint32_t)device_cus() - 1) / (uint32_t)device_cus()) <= BT &&
        (uint64_t)a->rows * a->cols < RING_OOB &&
        a->cols <= (PRO == SGK_PRO_RMS ? SGK_BAL_MAX_RMS_COLS : SGK_BAL_MAX_COLS) &&
        bal_lds_floats(a->rows, a->cols, (uint32_t)device_cus()) * 4 <= 160 * 1024)
        return launch_bal<PRO == SGK_PRO_RMS ? SGK_PRO_RMS : SGK_PRO_NONE, EPI>(*a, s);
    const size_t lds = GEMV_CH(PRO) ? (size_t)xs_ch_floats(a->cols) * 4 : (size_t)a->cols * 4;
    if constexpr (PRO != SGK_PRO_NONE)
        if (!a->tune_r && !a->tune_blocks && gemv_ring_on() && (uint64_t)a->rows * a->cols < RING_OOB)
            return launch_ring<PRO, EPI>(*a, lds, s);
    const int R = EPI == SGK_EPI_SWIGLU ? 2 : (a->tune_r == 1 ? 1 : a->tune_r == 4 ? 4 : 2);
    if (R == 4) return launch_q8<4, PRO, EPI>(*a, lds, s);
    if (R == 1) return launch_q8<1, PRO, (EPI == SGK_EPI_SWIGLU ? SGK_EPI_STORE : EPI)>(*a, lds, s);
    return launch_q8<2, PRO, EPI>(*a, lds, s);
}

extern "C" hipError_t sgk_gemv_launch(const sgk_gemv *a, hipStream_t s) {
#define CASE(P, E) if (a->pro == P && a->epi == E) return gemv_dispatch<P, E>(a, s)
    CASE(SGK_PRO_NONE, SGK_EPI_STORE);
    CASE(SGK_PRO_NONE, SGK_EPI_ADD);
    CASE(SGK_PRO_NONE, SGK_EPI_SWIGLU);
    CASE(SGK_PRO_RMS, SGK_EPI_STORE);
    CASE(SGK_PRO_RMS, SGK_EPI_ADD);
    CASE(SGK_PRO_RMS, SGK_EPI_SWIGLU);
    CASE(SGK_PRO_GATED, SGK_EPI_ADD);
    CASE(SGK_PRO_GATED, SGK_EPI_STORE);
#undef CASE
    return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
// Q8_0 repack: 34-byte blocks -> int8 plane + f16 scale plane
// ---------------------------------------------------------------------------

__global__ void k_repack_q8(const uint8_t *src, uint32_t rows, uint32_t cols, int8_t *qs,
                            uint16_t *d, uint16_t *dt, uint32_t ld, uint32_t row0, uint32_t step) {
    const uint32_t nbl = cols >> 5;
    const uint64_t b = (uint64_t)blockIdx.x * TPB + threadIdx.x;
    if (b >= (uint64_t)rows * nbl) return;
    const uint32_t r = (uint32_t)(b / nbl), j = (uint32_t)(b % nbl);
    const uint8_t *p = src + b * 34;
    const uint64_t dr = (uint64_t)row0 + (uint64_t)r * step;
    const uint16_t dv = (uint16_t)(p[0] | (p[1] << 8));
    d[dr * nbl + j] = dv;
    if (dt) dt[(uint64_t)j * ld + dr] = dv;
    uint32_t *o = (uint32_t *)(qs + dr * cols + (uint64_t)j * 32);
#pragma unroll
    for (int k = 0; k < 8; k++)
        o[k] = (uint32_t)p[2 + 4 * k] | ((uint32_t)p[3 + 4 * k] << 8) |
               ((uint32_t)p[4 + 4 * k] << 16) | ((uint32_t)p[5 + 4 * k] << 24);
}

extern "C" hipError_t sgk_repack_q8(const uint8_t *src, uint32_t rows, uint32_t cols,
                                    int8_t *qs, uint16_t *d, uint16_t *dt, uint32_t ld, uint32_t row0,
                                    uint32_t row_step, hipStream_t s) {
    const uint64_t n = (uint64_t)rows * (cols >> 5);
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(k_repack_q8, dim3((unsigned)((n + TPB - 1) / TPB)), dim3(TPB), 0, s, src,
                       rows, cols, qs, d, dt, ld, row0, row_step);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Embedding gather (ref.c:826-854): d * q in f32, one multiply.
// ---------------------------------------------------------------------------

__global__ void k_embed(const int8_t *qs, const uint16_t *d, const float *wf, uint32_t hidden,
                        const sgk_step *step, int32_t token, float *x) {
    const uint32_t i = blockIdx.x * TPB + threadIdx.x;
    if (i >= hidden) return;
    const uint64_t t = (uint64_t)(uint32_t)(step ? step->token : token);
    if (qs) x[i] = h2f(d[t * (hidden >> 5) + (i >> 5)]) * (float)qs[t * hidden + i];
    else x[i] = wf[t * hidden + i];
}

extern "C" hipError_t sgk_embed(const int8_t *qs, const uint16_t *d, const float *wf,
                                uint32_t hidden, const sgk_step *step, int32_t token, float *x,
                                hipStream_t s) {
    hipLaunchKernelGGL(k_embed, dim3((hidden + TPB - 1) / TPB), dim3(TPB), 0, s, qs, d, wf,
                       hidden, step, token, x);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Elementwise ops (ref.c:172-188; kernels.metal:316-335, 694-714)
// ---------------------------------------------------------------------------

__global__ void k_elementwise(int op, const float *a, const float *b, void *out, uint32_t n,
                              float scale) {
    const uint32_t i = blockIdx.x * TPB + threadIdx.x;
    if (i >= n) return;
    float *o = (float *)out;
    switch (op) {
    case SGK_EW_SWIGLU: o[i] = silu(a[i]) * b[i]; break;
    case SGK_EW_SILU: o[i] = silu(a[i]); break;
    case SGK_EW_GATE_SIGMOID: o[i] = a[i] * sigm(b[i]); break;
    case SGK_EW_ADD: o[i] = a[i] + b[i]; break;
    case SGK_EW_SCALE: o[i] = a[i] * scale; break;
    case SGK_EW_TO_F16: ((uint16_t *)out)[i] = f2h(a[i]); break;
    }
}

extern "C" hipError_t sgk_elementwise(int op, const float *a, const float *b, void *out,
                                      uint32_t n, float scale, hipStream_t s) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(k_elementwise, dim3((n + TPB - 1) / TPB), dim3(TPB), 0, s, op, a, b, out,
                       n, scale);
    return hipGetLastError();
}

__global__ void k_fill(float *p, float v, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * TPB + threadIdx.x; i < n; i += (uint64_t)gridDim.x * TPB)
        p[i] = v;
}

extern "C" hipError_t sgk_fill_f32(float *p, float v, uint64_t n, hipStream_t s) {
    if (!n) return hipSuccess;
    uint64_t blocks = (n + TPB - 1) / TPB;
    hipLaunchKernelGGL(k_fill, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(TPB), 0, s, p,
                       v, n);
    return hipGetLastError();
}

// Seeded fill of n values, f16 (bits of f16) or f32: a hash of (seed, index)
// mapped to a sum of two uniforms in [-scale, scale] (a triangular spread).
__global__ void k_fill_hash(void *p, uint64_t n, int f16, uint32_t seed, float scale) {
    for (uint64_t i = (uint64_t)blockIdx.x * TPB + threadIdx.x; i < n; i += (uint64_t)gridDim.x * TPB) {
        uint64_t h = (i + 1) * 0x9E3779B97F4A7C15ull ^ ((uint64_t)seed << 32 | seed);
        h ^= h >> 31; h *= 0xBF58476D1CE4E5B9ull; h ^= h >> 29; h *= 0x94D049BB133111EBull; h ^= h >> 32;
        const float u0 = (float)(uint32_t)(h & 0xFFFFu) / 65535.0f, u1 = (float)(uint32_t)((h >> 16) & 0xFFFFu) / 65535.0f;
        const float v = (u0 + u1 - 1.0f) * scale;
        if (f16) ((uint16_t *)p)[i] = f2h(v);
        else ((float *)p)[i] = v;
    }
}

extern "C" hipError_t sgk_fill_hash(void *p, uint64_t n, int f16, uint32_t seed, float scale, hipStream_t s) {
    if (!n) return hipSuccess;
    uint64_t blocks = (n + TPB - 1) / TPB;
    hipLaunchKernelGGL(k_fill_hash, dim3((unsigned)(blocks < 8192 ? blocks : 8192)), dim3(TPB), 0, s, p, n, f16,
                       seed, scale);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// RMSNorm over strided slices; RoPE over strided slices; softmax.
// ---------------------------------------------------------------------------

__global__ void __launch_bounds__(TPB) k_rmsnorm_heads(const float *x, const float *w, float *out,
                                                       uint32_t n, uint32_t stride, float eps) {
    __shared__ float red[4];
    const float *xh = x + (size_t)blockIdx.x * stride;
    float *oh = out + (size_t)blockIdx.x * stride;
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < n; i += TPB) { float v = xh[i]; ss = fmaf(v, v, ss); }
    ss = block_sum(ss, red);
    const float r = 1.0f / sqrtf(ss / (float)n + eps);
    for (uint32_t i = threadIdx.x; i < n; i += TPB) {
        float v = xh[i] * r;
        oh[i] = w ? v * w[i] : v;
    }
}

extern "C" hipError_t sgk_rmsnorm_heads(const float *x, const float *w, float *out, uint32_t n,
                                        uint32_t heads, uint32_t stride, float eps,
                                        hipStream_t s) {
    if (!heads || !n) return hipSuccess;
    hipLaunchKernelGGL(k_rmsnorm_heads, dim3(heads), dim3(TPB), 0, s, x, w, out, n,
                       stride ? stride : n, eps);
    return hipGetLastError();
}

__global__ void k_rope_heads(const float *x, const float *cs, float *out, uint32_t head_dim,
                             uint32_t rope_dim, uint32_t stride) {
    // head_dim <= TPB (checked by the launcher): one element per thread.
    const float *xh = x + (size_t)blockIdx.x * stride;
    float *oh = out + (size_t)blockIdx.x * stride;
    const uint32_t half = rope_dim >> 1, i = threadIdx.x;
    float v = 0.0f;
    if (i < half) v = xh[i] * cs[i] - xh[i + half] * cs[half + i];
    else if (i < rope_dim) v = xh[i - half] * cs[i] + xh[i] * cs[i - half];
    else if (i < head_dim) v = xh[i];
    __syncthreads();   // every read of the slice precedes any in-place write
    if (i < head_dim) oh[i] = v;
}

extern "C" hipError_t sgk_rope_heads(const float *x, const float *cs, float *out,
                                     uint32_t head_dim, uint32_t rope_dim, uint32_t heads,
                                     uint32_t stride, hipStream_t s) {
    if (!heads || head_dim > TPB) return heads ? hipErrorInvalidValue : hipSuccess;
    hipLaunchKernelGGL(k_rope_heads, dim3(heads), dim3(TPB), 0, s, x, cs, out, head_dim, rope_dim,
                       stride ? stride : head_dim);
    return hipGetLastError();
}

// softmax over n with the reference's NaN / +-inf conventions (ref.c:190-235)
__global__ void __launch_bounds__(TPB) k_softmax(const float *x, float *out, uint32_t n) {
    __shared__ float red[4];
    __shared__ float bc[2];
    float mx = -INFINITY;
    for (uint32_t i = threadIdx.x; i < n; i += TPB) mx = fmaxf(mx, x[i]);
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    if (threadIdx.x == 0) bc[0] = isnan(x[0]) ? x[0] : fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    mx = bc[0];
    if (isnan(mx)) { for (uint32_t i = threadIdx.x; i < n; i += TPB) out[i] = mx; return; }
    if (isinf(mx)) {
        float hits = 0.0f;
        for (uint32_t i = threadIdx.x; i < n; i += TPB) hits += (x[i] == mx) ? 1.0f : 0.0f;
        hits = block_sum(hits, red);
        const float u = 1.0f / (mx < 0.0f ? (float)n : hits);
        for (uint32_t i = threadIdx.x; i < n; i += TPB) out[i] = (mx < 0.0f || x[i] == mx) ? u : 0.0f;
        return;
    }
    float sum = 0.0f;
    for (uint32_t i = threadIdx.x; i < n; i += TPB) sum += expf(x[i] - mx);
    sum = block_sum(sum, red);
    for (uint32_t i = threadIdx.x; i < n; i += TPB) out[i] = expf(x[i] - mx) / sum;
}

extern "C" hipError_t sgk_softmax(const float *x, float *out, uint32_t n, hipStream_t s) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(k_softmax, dim3(1), dim3(TPB), 0, s, x, out, n);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Decode attention for one or many tokens. Token z of a launch (gridDim.z)
// reads its descriptor steps[z] (position; it attends over pos+1 keys), its
// query/gate row at q + z*q_tok, and owns its own m/s/acc slice. A decode step
// is the one-token case; a prefill chunk runs the same kernels over its tokens.
// ---------------------------------------------------------------------------

// Split count as the kernels see it: the decode policy (kernels.h), or the
// prefill policy (at most SGK_PREFILL_SPLITS splits of >= 1024 keys, so a
// chunk's partial scratch stays bounded).
__device__ __forceinline__ uint32_t dev_splits(uint32_t seq, int prefill, uint32_t cap) {
    if (!prefill) return dev_n_splits(seq, cap);
    uint32_t n = seq / 1024u;
    n = n < 1 ? 1 : n;
    return n > SGK_PREFILL_SPLITS ? SGK_PREFILL_SPLITS : n;
}

// Element offset of position pos of kv head kh in a K/V cache (the launchers
// resolve 0 strides to the reference layout).
__device__ __forceinline__ size_t kv_at(const sgk_attn &a, uint32_t pos, uint32_t kh) {
    return (size_t)pos * a.kv_ps + (size_t)kh * a.kv_hs;
}
static inline sgk_attn kv_resolved(const sgk_attn *a) {
    sgk_attn b = *a;
    if (!b.kv_ps) { b.kv_ps = b.n_kv * b.hd; b.kv_hs = b.hd; }
    return b;
}

// q_norm/k_norm + RoPE + f16 KV store. Workgroup (head, token): query heads
// first, then kv heads.
__global__ void __launch_bounds__(TPB) k_attn_prep(sgk_attn a, const float *qn, const float *kn,
                                                   const float *cs_table, float eps) {
    __shared__ float red[4];
    __shared__ float buf[TPB];
    const uint32_t z = blockIdx.y, pos = a.steps[z].pos, t = threadIdx.x, b = blockIdx.x, hd = a.hd;
    const float *cs = cs_table + (size_t)pos * a.rope_dim;
    const bool isq = b < a.n_heads;
    const uint32_t kh = b - a.n_heads;
    float *row = (float *)a.q + (size_t)z * a.q_tok;
    float *x = isq ? row + (size_t)b * a.q_stride : row + (size_t)a.n_heads * a.q_stride + (size_t)kh * hd;
    const float *w = isq ? qn : kn;
    const float v = t < hd ? x[t] : 0.0f;
    const float ss = block_sum(v * v, red);
    const float r = 1.0f / sqrtf(ss / (float)hd + eps);
    const float xn = t < hd ? (v * r) * w[t] : 0.0f;
    buf[t] = xn;
    __syncthreads();
    const uint32_t half = a.rope_dim >> 1;
    float o = xn;
    if (t < half) o = buf[t] * cs[t] - buf[t + half] * cs[half + t];
    else if (t < a.rope_dim) o = buf[t - half] * cs[t] + buf[t] * cs[t - half];
    if (t >= hd) return;
    if (isq) {
        x[t] = o;
    } else {
        const size_t at = kv_at(a, pos, kh) + t;
        const float *vraw = row + (size_t)a.n_heads * a.q_stride + (size_t)a.n_kv * hd + (size_t)kh * hd;
        ((uint16_t *)a.kc)[at] = f2h(o);
        ((uint16_t *)a.vc)[at] = f2h(vraw[t]);
    }
}

extern "C" hipError_t sgk_attn_prep(const sgk_attn *a, const float *qn, const float *kn,
                                    const float *cs_table, float eps, hipStream_t s) {
    if (a->hd > TPB || !a->ntok) return a->ntok ? hipErrorInvalidValue : hipSuccess;
    hipLaunchKernelGGL(k_attn_prep, dim3(a->n_heads + a->n_kv, a->ntok), dim3(TPB), 0, s, kv_resolved(a), qn, kn,
                       cs_table, eps);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Split-K GQA decode attention partial.
//
// Workgroup (split i, kv head hk, token z) owns keys [i*seq/n, (i+1)*seq/n) and
// all G = n_heads/n_kv query heads of the group, so every K/V byte is read
// once per token. Keys are processed in tiles of 32: scores (8 lanes per key,
// HD/8 dims per lane, q from LDS), tile max and exp per head, then P*V with
// one output dim per lane. Across tiles the running max/sum/acc are rescaled
// (online softmax); a split of at most 32 keys is exactly the reference's
// two-pass form. Output: m, s and the UNNORMALISED acc, as ref.c's
// attn_partial.
// ---------------------------------------------------------------------------

#define GMAX 8

// The query heads a partial workgroup serves: the whole GQA group of kv head
// blockIdx.y, or (per-head form, grid y = n_heads) query head blockIdx.y
// alone, reading its group's kv head. In the per-head form every head of the
// split that holds the position stores the new K/V row (the same bytes), so
// each workgroup reads back a row it has written itself.
struct attn_group { uint32_t G, hk, h0; };
__device__ __forceinline__ attn_group attn_group_of(const sgk_attn &a) {
    const uint32_t gf = a.n_heads / a.n_kv;
    if (a.per_head) return {1u, blockIdx.y / gf, blockIdx.y};
    return {gf, blockIdx.y, blockIdx.y * gf};
}

// Query / key prep shared by k_attn_prep and the fused decode partial:
// RMSNorm (w) then half-split RoPE over the first rope_dim dims, element d
// of a row x whose raw values and 1/rms factor are given (ref.c:1207-1235,
// 561-606). cs is the position's cos|sin row.
__device__ __forceinline__ float prep_elem(const float *x, float r, const float *w, const float *cs,
                                           uint32_t d, uint32_t rope_dim) {
    const uint32_t half = rope_dim >> 1;
    if (d < half) return ((x[d] * r) * w[d]) * cs[d] - ((x[d + half] * r) * w[d + half]) * cs[half + d];
    if (d < rope_dim) return ((x[d - half] * r) * w[d - half]) * cs[d] + ((x[d] * r) * w[d]) * cs[d - half];
    return (x[d] * r) * w[d];
}

// ---------------------------------------------------------------------------
// Split-K GQA attention partial (tiled).
//
// Workgroup (split i, kv head hk, token z) owns keys [i*seq/n, (i+1)*seq/n)
// and all G = n_heads/n_kv query heads of its group, so every K/V byte is
// read once per token. Keys go in tiles of TK = 256*DPT/HD (64 at head_dim
// 256). Every K and V load of a tile is issued unconditionally, indices
// clamped into the split (keys past its end score -inf and their V is
// zeroed), so a tile costs one memory round trip; the next tile's K is
// requested once the scores are formed and its V once P*V is done.
//   scores: TPK = HD/DPT lanes per key, DPT dims per lane, q from LDS;
//   softmax: one wave per head over the tile, running max/sum rescaled
//            across tiles (online form);
//   P*V:    lane = (key group kg, 8-dim chunk vc), KGV key groups folded at
//           the end in a fixed order (xor shuffles, then waves in order).
// Output: m, s and the UNNORMALISED acc of each (head, split), as ref.c's
// attn_partial (ref.c:416-455). Empty splits give m=-inf, s=0, acc=0.
//
// With a.fuse_prep (decode, one token): the workgroup first forms the
// q_norm+RoPE'd queries of its heads in LDS from the raw projection rows,
// and the split holding the new position also stores that token's
// k_norm+RoPE'd K and raw V as f16 at the position before reading any key
// (one writer per (position, kv head)).
// ---------------------------------------------------------------------------

template <int HD, int DPTMAX = 64>
struct attn_geom {
    static constexpr int DPT = HD < DPTMAX ? HD : DPTMAX;   // score dims per lane
    static constexpr int TPK = HD / DPT;            // lanes per key
    static constexpr int TK = TPB / TPK;            // keys per tile
    static constexpr int KU = DPT / 8;              // K uint4 per lane
    static constexpr int VC = HD / 8;               // 8-dim chunks of a V row
    static constexpr int KGV = TPB / VC;            // key groups in P*V
    static constexpr int VU = TK / KGV;             // V uint4 per lane
    static constexpr int QP = DPT + 4;              // padded q chunk (LDS banks)
    static constexpr int QROW = TPK * QP;
};

__device__ __forceinline__ void h8(const uint4 r, float *f) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
        f[2 * e] = h2f((uint16_t)(w[e] & 0xFFFF));
        f[2 * e + 1] = h2f((uint16_t)(w[e] >> 16));
    }
}

template <int HD, int DPTMAX>
__global__ void __launch_bounds__(TPB) k_attn_partial(sgk_attn a) {
    using Gm = attn_geom<HD, DPTMAX>;
    constexpr int DPT = Gm::DPT, TPK = Gm::TPK, TK = Gm::TK, KU = Gm::KU, VC = Gm::VC, KGV = Gm::KGV,
                  VU = Gm::VU, QP = Gm::QP, QROW = Gm::QROW;
    __shared__ float qsh[GMAX * QROW];
    __shared__ float sc[GMAX][TK];
    __shared__ float mrun[GMAX], srun[GMAX], alpha[GMAX], rn[GMAX + 1];
    __shared__ __align__(16) float red[TPB / 64][GMAX * HD];   // end fold; raw rows during prep

    const attn_group gr = attn_group_of(a);
    const uint32_t G = gr.G, n_kv = a.n_kv, z = blockIdx.z;
    const uint32_t i = blockIdx.x, hk = gr.hk, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint32_t h0 = gr.h0;
    const float *q = a.q + (size_t)z * a.q_tok;
    const bool fp = a.fuse_prep != 0;

    // 1. Loads that need no position go first, so their round trip overlaps
    //    the position's: the group's q rows and, for the fused prep, both
    //    norm weights and the raw k and v rows (unused outside the split that
    //    holds the position). Every load is unconditional at a clamped index
    //    (pointers the call does not use are swapped for q), so no branch
    //    makes a load wait early.
    constexpr int QPT = (GMAX * HD + TPB - 1) / TPB;   // q values per thread
    float qv[QPT];
#pragma unroll
    for (int k = 0; k < QPT; k++) {
        const uint32_t e = min(t + k * TPB, G * HD - 1);
        qv[k] = q[(size_t)(h0 + e / HD) * a.q_stride + e % HD];
    }
    const uint32_t td = min(t, (uint32_t)HD - 1);
    const float *krow = fp ? q + (size_t)a.n_heads * a.q_stride + (size_t)hk * HD : q;
    const float *vrow = fp ? krow + (size_t)n_kv * HD : q;
    const float qn0 = (fp ? a.qn : q)[td], kn0 = (fp ? a.kn : q)[td];
    const float kr0 = krow[td], vr0 = vrow[td];

    const uint32_t pos = a.steps ? a.steps[z].pos : 0;
    const uint32_t seq = a.steps ? pos + 1 : a.seq;
    const uint32_t ns = a.steps ? dev_splits(seq, a.prefill, a.split_cap) : a.n_splits;
    if (i >= ns) return;
    const uint32_t t0 = (uint32_t)((uint64_t)i * seq / ns);
    const uint32_t t1 = (uint32_t)((uint64_t)(i + 1) * seq / ns);
    const uint16_t *kc = a.kc, *vc = a.vc;
    const size_t zoff = (size_t)z * a.n_heads * a.max_splits;
    const uint32_t kj = t / TPK, kp = t % TPK;      // score mapping
    const uint32_t vcc = t % VC, kg = t / VC;       // P*V mapping

    // K/V tile loads are unconditional: keys past the split clamp to its last
    // key (a whole tile past the end re-reads one row), so no branch joins
    // paths with and without loads in flight, which would make the waits
    // before later uses count as if nothing were queued behind them.
    uint4 kr[KU], vr[VU];
    const uint32_t klast = t1 ? t1 - 1 : 0;
    auto load_k = [&](uint32_t ts) {
        const uint32_t key = min(ts + kj, klast);
        const uint4 *p = (const uint4 *)(kc + kv_at(a, key, hk) + kp * DPT);
#pragma unroll
        for (int u = 0; u < KU; u++) kr[u] = p[u];
    };
    auto load_v = [&](uint32_t ts) {
#pragma unroll
        for (int u = 0; u < VU; u++) {
            const uint32_t key = min(ts + kg + u * KGV, klast);
            vr[u] = ((const uint4 *)(vc + kv_at(a, key, hk)))[vcc];
        }
    };
    // 2. The position's cos|sin entry, then the first tile's K and V; all of
    //    it overlaps the prep's first steps.
    const float cs0 = (fp ? a.cs + (size_t)pos * a.rope_dim : q)[min(td, a.rope_dim ? a.rope_dim - 1 : 0u)];
    __builtin_amdgcn_sched_barrier(0);              // keep it ahead of the tile in the load queue
    load_k(t0);
    load_v(t0);
    if (fp) {
        __shared__ float cs_s[HD], qn_s[HD], kn_s[HD];
        __shared__ __align__(16) uint16_t knew[HD], vnew[HD];
        float *raw = &red[0][0];                 // [G][HD] q, then k past the q slots
        const bool kv_writer = i == ns - 1;
        // LDS stores are unconditional (duplicates store equal values; q
        // slots past the group are never read); each waits only for its own
        // data, not the tile behind it.
        constexpr int KOFF = QPT * TPB;                   // raw k row, past every q slot
        static_assert(KOFF + HD <= (TPB / 64) * GMAX * HD, "raw q|k rows exceed the fold buffer");
#pragma unroll
        for (int k = 0; k < QPT; k++) raw[t + k * TPB] = qv[k];
        qn_s[td] = qn0;
        raw[KOFF + td] = kr0;
        kn_s[td] = kn0;
        __syncthreads();
        cs_s[td] = td < a.rope_dim ? cs0 : 0.0f;        // read after the next barrier
        for (uint32_t h = wave; h <= (uint32_t)G; h += TPB / 64) {
            if (h == (uint32_t)G && !kv_writer) break;
            const float *x = h < (uint32_t)G ? raw + h * HD : raw + KOFF;
            float ss = 0.0f;
            for (uint32_t d = lane; d < HD; d += 64) ss = fmaf(x[d], x[d], ss);
            ss = wave_sum(ss);
            if (lane == 0) rn[h] = 1.0f / sqrtf(ss / (float)HD + a.eps);
        }
        __syncthreads();
        for (uint32_t e = t; e < G * HD; e += TPB) {
            const uint32_t h = e / HD, d = e % HD;
            qsh[h * QROW + (d / DPT) * QP + d % DPT] = prep_elem(raw + h * HD, rn[h], qn_s, cs_s, d, a.rope_dim);
        }
        if (kv_writer) {
            const size_t at = kv_at(a, pos, hk);
            for (uint32_t d = t; d < HD; d += TPB) {
                const uint16_t kh = f2h(prep_elem(raw + KOFF, rn[G], kn_s, cs_s, d, a.rope_dim));
                const uint16_t vh = f2h(vr0);
                ((uint16_t *)a.kc)[at + d] = kh;
                ((uint16_t *)a.vc)[at + d] = vh;
                knew[d] = kh;
                vnew[d] = vh;
            }
        }
        __syncthreads();
        // The first tile was requested before the new row was stored: if it
        // holds the position, take that key's K and V from LDS. Later tiles
        // are loaded after the store and the barrier above, which makes the
        // stored row visible to the whole workgroup.
        if (kv_writer && t0 < t1 && pos - t0 < (uint32_t)TK) {
            if (t0 + kj == pos) {
#pragma unroll
                for (int u = 0; u < KU; u++) kr[u] = ((const uint4 *)(knew + kp * DPT))[u];
            }
#pragma unroll
            for (int u = 0; u < VU; u++)
                if (t0 + kg + u * KGV == pos) vr[u] = ((const uint4 *)vnew)[vcc];
        }
    } else {
#pragma unroll
        for (int k = 0; k < QPT; k++) {
            const uint32_t e = t + k * TPB, h = e / HD, d = e % HD;
            if (e < G * HD) qsh[h * QROW + (d / DPT) * QP + d % DPT] = qv[k];
        }
    }
    if (t < (uint32_t)G) { mrun[t] = -INFINITY; srun[t] = 0.0f; }
    __syncthreads();

    float acc[GMAX][8];
#pragma unroll
    for (int h = 0; h < GMAX; h++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[h][e] = 0.0f;

    for (uint32_t ts = t0; ts < t1; ts += TK) {
        const uint32_t nk = min((uint32_t)TK, t1 - ts);
        // scores
        float part[GMAX];
#pragma unroll
        for (int h = 0; h < GMAX; h++) part[h] = 0.0f;
#pragma unroll
        for (int u = 0; u < KU; u++) {
            float kf[8];
            h8(kr[u], kf);
#pragma unroll
            for (int h = 0; h < GMAX; h++) {
                if (h < (int)G) {
                    const float4 *qa = (const float4 *)(qsh + h * QROW + kp * QP + u * 8);
                    const float4 x0 = qa[0], x1 = qa[1];
                    float s = part[h];
                    s = fmaf(x0.x, kf[0], s); s = fmaf(x0.y, kf[1], s); s = fmaf(x0.z, kf[2], s);
                    s = fmaf(x0.w, kf[3], s); s = fmaf(x1.x, kf[4], s); s = fmaf(x1.y, kf[5], s);
                    s = fmaf(x1.z, kf[6], s); s = fmaf(x1.w, kf[7], s);
                    part[h] = s;
                }
            }
        }
        load_k(ts + TK);                             // past the split: one row, unused
#pragma unroll
        for (int h = 0; h < GMAX; h++) {
            if (TPK >= 2) part[h] += lane_xor1(part[h]);
            if (TPK >= 4) part[h] += lane_xor2(part[h]);
            if (TPK >= 8) part[h] += lane_xor<4>(part[h]);
            if (TPK >= 16) part[h] += lane_xor8(part[h]);
        }
        if (kp == 0) {
#pragma unroll
            for (int h = 0; h < GMAX; h++)
                if (h < (int)G) sc[h][kj] = (kj < nk) ? part[h] * a.scale : -INFINITY;
        }
        __syncthreads();
        // softmax: one wave per head over the tile
        for (uint32_t h = wave; h < (uint32_t)G; h += TPB / 64) {
            constexpr int NV = TK >= 64 ? TK / 64 : 1;   // keys per lane
            float v[NV];
            float tm = -INFINITY;
#pragma unroll
            for (int r = 0; r < NV; r++) {
                const uint32_t j = lane + 64 * r;
                v[r] = j < (uint32_t)TK ? sc[h][j] : -INFINITY;
                tm = fmaxf(tm, v[r]);
            }
            tm = wave_max(tm);
            const float mold = mrun[h];
            const float mnew = fmaxf(mold, tm);
            float ps = 0.0f;
#pragma unroll
            for (int r = 0; r < NV; r++) {
                const uint32_t j = lane + 64 * r;
                const float p = (j < nk) ? expf(v[r] - mnew) : 0.0f;
                if (j < (uint32_t)TK) sc[h][j] = p;
                ps += p;
            }
            ps = wave_sum(ps);
            if (lane == 0) {
                const float al = (mold == -INFINITY) ? 0.0f : expf(mold - mnew);
                alpha[h] = al;
                mrun[h] = mnew;
                srun[h] = srun[h] * al + ps;
            }
        }
        __syncthreads();
        // P*V
#pragma unroll
        for (int h = 0; h < GMAX; h++) {
            if (h < (int)G) {
                const float al = alpha[h];
#pragma unroll
                for (int e = 0; e < 8; e++) acc[h][e] *= al;
            }
        }
#pragma unroll
        for (int u = 0; u < VU; u++) {
            const uint32_t key = kg + u * KGV;
            float vf[8];
            h8(vr[u], vf);
            if (key >= nk) {
#pragma unroll
                for (int e = 0; e < 8; e++) vf[e] = 0.0f;
            }
#pragma unroll
            for (int h = 0; h < GMAX; h++) {
                if (h < (int)G) {
                    const float p = sc[h][key];
#pragma unroll
                    for (int e = 0; e < 8; e++) acc[h][e] = fmaf(p, vf[e], acc[h][e]);
                }
            }
        }
        load_v(ts + TK);
        __syncthreads();
    }

    // Fold the key groups: inside the wave, then the four waves in order.
#pragma unroll
    for (int h = 0; h < GMAX; h++)
#pragma unroll
        for (int e = 0; e < 8; e++)
        {
            if (VC <= 2) acc[h][e] += lane_xor<2>(acc[h][e]);
            if (VC <= 4) acc[h][e] += lane_xor<4>(acc[h][e]);
            if (VC <= 8) acc[h][e] += lane_xor<8>(acc[h][e]);
            if (VC <= 16) acc[h][e] += lane_xor<16>(acc[h][e]);
            acc[h][e] += lane_xor<32>(acc[h][e]);
        }
    if (lane < (uint32_t)VC) {
#pragma unroll
        for (int h = 0; h < GMAX; h++) {
            if (h >= (int)G) break;
            float4 *dst = (float4 *)&red[wave][h * HD + vcc * 8];
            dst[0] = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
            dst[1] = make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
        }
    }
    __syncthreads();
    for (uint32_t e = t; e < G * HD; e += TPB) {
        const uint32_t h = e / HD, d = e % HD;
        const float v = (red[0][e] + red[1][e]) + (red[2][e] + red[3][e]);
        a.acc[(zoff + (size_t)(h0 + h) * ns + i) * HD + d] = v;
    }
    if (t < (uint32_t)G) {
        const size_t o = zoff + (size_t)(h0 + t) * ns + i;
        a.m[o] = mrun[t];
        a.s[o] = srun[t];
    }
}

// Shared by the MFMA attention kernels (decode partial and prefill pass).
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

#define FA_TQ 64    // tokens per workgroup (4 waves x 16)
#define FA_TK 64    // keys per tile
// LDS row pitches of the flash tiles: an MFMA fragment read (lane: row li,
// 16-byte chunk lg) is free of bank conflicts when the pitch is an odd
// multiple of 32 bytes (measured with SQ_LDS_BANK_CONFLICT: 8 LDS cycles per
// read at 9 or 33 16-byte slots, 4 at 10 or 34), hence +16 elements
#define FA_PLD (FA_TK + 16)

// x[0..7] -> f16 hi and lo fragments
__device__ __forceinline__ void fa_split8(const float *x, f16x8 &hi, f16x8 &lo) {
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const _Float16 h = (_Float16)x[e];
        hi[e] = h;
        lo[e] = (_Float16)(x[e] - (float)h);
    }
}

// K rows for the score MFMA's A operand: lane (li, lg) takes key `key`, dims
// 8*lg.. of each 32 (16 B per load, one per 32-dim block). K and V are read
// once per token, so their loads are non-temporal, as the weights' are: at
// 262000 keys, 122.2 -> 127.4 tok/s; at 4k no change.
template <int HD>
__device__ __forceinline__ void mf_load_k(v4u (&kr)[HD / 32], const uint16_t *kh, uint32_t key, uint32_t ps,
                                          uint32_t lg) {
    const v4u *p = (const v4u *)(kh + (size_t)key * ps + lg * 8);
#pragma unroll
    for (int kb = 0; kb < HD / 32; kb++) kr[kb] = __builtin_nontemporal_load(p + kb * 4);
}
// ---------------------------------------------------------------------------
// Decode split-K partial with one independent key stream per wave (head_dim
// 128 or 256, fused prep). Workgroup (split, kv head), the prep and the output
// partials are those of k_attn_partial; in each 64-key round wave w takes keys
// 16w..16w+15 and keeps its own running max, sum and output for the group's
// heads, so the key loop has no barrier and no LDS traffic:
//  - scores S^T = K Q^T on v_mfma_f32_16x16x32_f16: A = 16 keys straight
//    from the f16 cache (lane li = key, 8 dims per 32), B = the group's q
//    (column li = head li, f16 hi + lo); lane (li, lg) gets head li's scores
//    of keys 4lg..4lg+3;
//  - online softmax per head over the 4 lanes that share li (two cross-row
//    steps); the output is kept transposed (O^T), so its rescale is in-lane;
//  - O^T += V^T P^T on v_mfma_f32_16x16x16_f16: B = p in the score layout
//    (f16 hi + lo), A = V^T built in registers: lane (li, lg) loads keys
//    4lg..4lg+3 at dims 8li.. (and 8(li+16).. at head_dim 256) and packs one
//    dim of its 4 keys per operand with v_perm;
//  - the 4 waves' (max, sum, output) merge through LDS once, at the end.
// ---------------------------------------------------------------------------
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));

// keys key0..key0+3 (clamped at klast), dims 8li..8li+7 (+128 per q)
template <int HD>
__device__ __forceinline__ void wv_load_v(v4u (&vr)[4][HD / 128], const uint16_t *vh, uint32_t key0, uint32_t klast,
                                          uint32_t ps, uint32_t li) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint16_t *row = vh + (size_t)min(key0 + j, klast) * ps;
#pragma unroll
        for (int q = 0; q < HD / 128; q++) vr[j][q] = __builtin_nontemporal_load((const v4u *)(row + (li + 16 * q) * 8));
    }
}

// RKB = 0: q_norm + RoPE of the group's heads through LDS (any rope_dim), as in
// k_attn_partial. RKB = 1 or 2 (rope_dim = 64*RKB): each lane preps its own
// q fragment in registers. The 4 lanes that share li hold all of head li's
// dims (8 per 32), so the sum of squares is two cross-row steps, and a
// rotated dim's partner (d +- rope_dim/2) sits in the same lane, RKB k-blocks
// away: no LDS and no barrier, except in the split that stores the new K.
// RKB = WV_RAW: no prep and no store; q is taken as given (the per-op
// one-shots), seq and n_splits come from the call when there are no step
// descriptors, and an empty split writes m = -inf, s = 0, acc = 0 without
// touching the cache.
#define WV_RAW 3
template <int HD, int RKB>
__global__ void __launch_bounds__(TPB) __attribute__((amdgpu_waves_per_eu(2, 2))) k_attn_partial_wv(sgk_attn a) {
    static_assert(HD == 128 || HD == 256, "wave-stream decode partial takes head_dim 128 or 256");
    static_assert(RKB == WV_RAW || (RKB >= 0 && RKB <= 2 && 2 * RKB <= HD / 32),
                  "register prep takes rope_dim 64 or 128");
    constexpr bool RAW = RKB == WV_RAW;
    constexpr int RR = RAW ? 0 : RKB;                 // rotated k-blocks of the register prep
    constexpr bool REGQ = RAW || RKB > 0;             // q fragments straight from the rows
    // the first keys' K is requested before the prep, except where the
    // register prep's values leave no room for it (head_dim 256, rope 128)
    constexpr bool EARLY_K = !(HD == 256 && RKB == 2);
    constexpr int NKB = HD / 32, NQ = HD / 128, NO = HD / 16;   // score k-blocks; V chunks per lane; O^T tiles
    constexpr int QPT = (GMAX * HD + TPB - 1) / TPB, KOFF = QPT * TPB;
    constexpr int OWS = HD + 4;                                  // merge row stride (floats)
    constexpr int BIG = (4 * GMAX * OWS > KOFF + HD) ? 4 * GMAX * OWS : KOFF + HD;
    __shared__ __align__(16) float qsh[GMAX * HD];
    __shared__ __align__(16) float big[BIG];                     // prep: raw q|k rows; end: the waves' outputs
    __shared__ float mw[4][GMAX], lw[4][GMAX], rn[GMAX + 1];
    __shared__ __align__(16) float cs_s[HD], qn_s[HD], kn_s[HD];
    __shared__ __align__(16) uint16_t knew[HD], vnew[HD];
    float *raw = big;

    const attn_group gr = attn_group_of(a);
    const uint32_t G = gr.G, n_kv = a.n_kv, z = blockIdx.z;
    const uint32_t i = blockIdx.x, hk = gr.hk, t = threadIdx.x, lane = t & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t li = lane & 15, lg = lane >> 4, h0 = gr.h0;
    const float *q = a.q + (size_t)z * a.q_tok;

    // 1. position-independent loads first (as in k_attn_partial)
    float qv[REGQ ? 1 : QPT];
    f32x4 qx[NKB][2];                 // register prep: head min(li, G-1)'s dims 32kb + 8lg..
    if constexpr (!REGQ) {
#pragma unroll
        for (int k = 0; k < QPT; k++) {
            const uint32_t e = min(t + k * TPB, G * HD - 1);
            qv[k] = q[(size_t)(h0 + e / HD) * a.q_stride + e % HD];
        }
    } else {
        const float *qrow = q + (size_t)(h0 + min(li, G - 1)) * a.q_stride + lg * 8;
#pragma unroll
        for (int kb = 0; kb < NKB; kb++)
#pragma unroll
            for (int c = 0; c < 2; c++) qx[kb][c] = *(const f32x4 *)(qrow + kb * 32 + c * 4);
    }
    const uint32_t td = min(t, (uint32_t)HD - 1);
    float qn0 = 0.0f, kn0 = 0.0f, kr0 = 0.0f, vr0 = 0.0f;
    if constexpr (!RAW) {
        const float *krow = q + (size_t)a.n_heads * a.q_stride + (size_t)hk * HD;
        const float *vrow = krow + (size_t)n_kv * HD;
        qn0 = a.qn[td];
        kn0 = a.kn[td];
        kr0 = krow[td];
        vr0 = vrow[td];
    }

    const uint32_t pos = a.steps ? a.steps[z].pos : 0;
    const uint32_t seq = (RAW && !a.steps) ? a.seq : pos + 1;
    const uint32_t ns = (RAW && !a.steps) ? a.n_splits : dev_splits(seq, a.prefill, a.split_cap);
    if (i >= ns) return;
    const uint32_t t0 = (uint32_t)((uint64_t)i * seq / ns), t1 = (uint32_t)((uint64_t)(i + 1) * seq / ns);
    const uint32_t klast = t1 ? t1 - 1 : 0;
    const size_t zoff = (size_t)z * a.n_heads * a.max_splits;
    if (RAW && t1 == t0) {            // an empty split (more splits than keys, or no keys)
        for (uint32_t e = t; e < G * HD; e += TPB)
            a.acc[(zoff + (size_t)(h0 + e / HD) * ns + i) * HD + e % HD] = 0.0f;
        if (t < G) {
            a.m[zoff + (size_t)(h0 + t) * ns + i] = -INFINITY;
            a.s[zoff + (size_t)(h0 + t) * ns + i] = 0.0f;
        }
        return;
    }

    // 2. the position's cos|sin entry, then this wave's first 16 keys of K
    //    and V
    float cs0 = 0.0f;
    if constexpr (!RAW) cs0 = a.cs[(size_t)pos * a.rope_dim + min(td, a.rope_dim - 1)];
    __builtin_amdgcn_sched_barrier(0);
    v4u kr[NKB], vr[4][NQ];
    const uint16_t *kch = a.kc + (size_t)hk * a.kv_hs, *vch = a.vc + (size_t)hk * a.kv_hs;
    const uint32_t base0 = t0 + wave * 16;
    if constexpr (EARLY_K) mf_load_k<HD>(kr, kch, min(base0 + li, klast), a.kv_ps, lg);
    if constexpr (EARLY_K) wv_load_v<HD>(vr, vch, base0 + 4 * lg, klast, a.kv_ps, li);
    // register prep: the q_norm weights and the cos|sin entry go to LDS (the
    // lanes read their dims' values there, which keeps them out of registers
    // while K and V are in flight)
    if constexpr (!RAW && RKB > 0) {
        qn_s[td] = qn0;
        cs_s[td] = td < a.rope_dim ? cs0 : 0.0f;
        __syncthreads();
    }

    // 3. prep: q_norm + RoPE of the group's heads; the split holding the
    //    position stores that token's K (k_norm + RoPE) and raw V as f16
    const bool kv_writer = !RAW && i == ns - 1;
    if (!RAW && (RKB == 0 || kv_writer)) {
        if constexpr (RKB == 0) {
#pragma unroll
            for (int k = 0; k < QPT; k++) raw[t + k * TPB] = qv[k];
            qn_s[td] = qn0;
            cs_s[td] = td < a.rope_dim ? cs0 : 0.0f;
        }
        raw[KOFF + td] = kr0;
        kn_s[td] = kn0;
        __syncthreads();
        for (uint32_t h = RKB ? G + wave : wave; h <= G; h += TPB / 64) {
            if (h == G && !kv_writer) break;
            const float *x = h < G ? raw + h * HD : raw + KOFF;
            float ss = 0.0f;
            for (uint32_t d = lane; d < HD; d += 64) ss = fmaf(x[d], x[d], ss);
            ss = wave_sum(ss);
            if (lane == 0) rn[h] = 1.0f / sqrtf(ss / (float)HD + a.eps);
        }
        __syncthreads();
        if constexpr (RKB == 0) {
            for (uint32_t e = t; e < G * HD; e += TPB) {
                const uint32_t h = e / HD, d = e % HD;
                qsh[e] = prep_elem(raw + h * HD, rn[h], qn_s, cs_s, d, a.rope_dim);
            }
        }
        if (kv_writer) {
            const size_t at = kv_at(a, pos, hk);
            for (uint32_t d = t; d < HD; d += TPB) {
                const uint16_t kh = f2h(prep_elem(raw + KOFF, rn[G], kn_s, cs_s, d, a.rope_dim));
                const uint16_t vh = f2h(vr0);
                ((uint16_t *)a.kc)[at + d] = kh;
                ((uint16_t *)a.vc)[at + d] = vh;
                knew[d] = kh;
                vnew[d] = vh;
            }
        }
        __syncthreads();
    }
    // the first keys were requested before the store: take the position's row from LDS
    if (kv_writer && pos - t0 < 64u) {
        if (EARLY_K && base0 + li == pos) {
#pragma unroll
            for (int kb = 0; kb < NKB; kb++) kr[kb] = ((const v4u *)(knew + lg * 8))[kb * 4];
        }
        if constexpr (EARLY_K) {
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (base0 + 4 * lg + j == pos) {
#pragma unroll
                    for (int qq = 0; qq < NQ; qq++) vr[j][qq] = *(const v4u *)(vnew + (li + 16 * qq) * 8);
                }
        }
    }
    // q as the B operand: column li = head li (zero past the group), dims 8*lg.. of each 32
    f16x8 qh[NKB], ql[NKB];
    if constexpr (RKB == 0) {
#pragma unroll
        for (int kb = 0; kb < NKB; kb++) {
            float xv[8];
#pragma unroll
            for (int e = 0; e < 8; e++) xv[e] = li < G ? qsh[li * HD + kb * 32 + lg * 8 + e] : 0.0f;
            fa_split8(xv, qh[kb], ql[kb]);
        }
    } else if constexpr (RAW) {
#pragma unroll
        for (int kb = 0; kb < NKB; kb++) {
            float xv[8];
#pragma unroll
            for (int e = 0; e < 8; e++) xv[e] = li < G ? qx[kb][e / 4][e % 4] : 0.0f;
            fa_split8(xv, qh[kb], ql[kb]);
        }
    } else {
        // prep_elem's arithmetic on the lane's dims: x * r * w, then the half-split rotation
        float ss = 0.0f;
#pragma unroll
        for (int kb = 0; kb < NKB; kb++)
#pragma unroll
            for (int e = 0; e < 8; e++) ss = fmaf(qx[kb][e / 4][e % 4], qx[kb][e / 4][e % 4], ss);
        ss += lane_xor16(ss);
        ss += lane_xor32(ss);
        const float rq = 1.0f / sqrtf(ss / (float)HD + a.eps);
        float y[NKB][8];
#pragma unroll
        for (int kb = 0; kb < NKB; kb++)
#pragma unroll
            for (int e = 0; e < 8; e++) y[kb][e] = (qx[kb][e / 4][e % 4] * rq) * qn_s[kb * 32 + lg * 8 + e];
#pragma unroll
        for (int kb = 0; kb < RKB; kb++)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float c = cs_s[kb * 32 + lg * 8 + e], sn = cs_s[RR * 32 + kb * 32 + lg * 8 + e];
                const float lo = y[kb][e], hi = y[kb + RKB][e];
                y[kb][e] = lo * c - hi * sn;
                y[kb + RKB][e] = lo * sn + hi * c;
            }
#pragma unroll
        for (int kb = 0; kb < NKB; kb++) {
            float xv[8];
#pragma unroll
            for (int e = 0; e < 8; e++) xv[e] = li < G ? y[kb][e] : 0.0f;
            fa_split8(xv, qh[kb], ql[kb]);
        }
        // the first keys' V (and K where it waited), requested after the
        // prep, so after the new row's store and barrier in the split that
        // holds the position
        if constexpr (!EARLY_K) {
            __builtin_amdgcn_sched_barrier(0);
            mf_load_k<HD>(kr, kch, min(base0 + li, klast), a.kv_ps, lg);
            wv_load_v<HD>(vr, vch, base0 + 4 * lg, klast, a.kv_ps, li);
        }
    }

    float m_run = -INFINITY, l_run = 0.0f;
    f32x4 o[NO];
#pragma unroll
    for (int n = 0; n < NO; n++) o[n] = (f32x4){0.f, 0.f, 0.f, 0.f};
    // One 64-key round (16 keys per wave). PREF: request the next round's K
    // and V during this one; the last round requests nothing (nothing would
    // use it, and the merge below would wait for it), and it is a separate
    // instance so the loop's wait counts stay exact.
    const uint32_t nr = (t1 - t0 + 63) / 64;
    auto round = [&](uint32_t r, auto pref) {
        constexpr bool PREF = decltype(pref)::value;
        const uint32_t base = t0 + r * 64 + wave * 16;
        f32x4 sh = (f32x4){0.f, 0.f, 0.f, 0.f}, sl = sh;
#pragma unroll
        for (int kb = 0; kb < NKB; kb++) {
            const f16x8 bk = __builtin_bit_cast(f16x8, kr[kb]);
            sh = __builtin_amdgcn_mfma_f32_16x16x32_f16(bk, qh[kb], sh, 0, 0, 0);
            sl = __builtin_amdgcn_mfma_f32_16x16x32_f16(bk, ql[kb], sl, 0, 0, 0);
        }
        // the next round's K, issued here so that it is in flight during the
        // softmax and P V
        if constexpr (PREF) mf_load_k<HD>(kr, kch, min(base + 64 + li, klast), a.kv_ps, lg);
        __builtin_amdgcn_sched_barrier(0);
        float p[4], tm = -INFINITY;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float sv = (sh[e] + sl[e]) * a.scale;
            p[e] = base + 4 * lg + e < t1 ? sv : -INFINITY;
            tm = fmaxf(tm, p[e]);
        }
        tm = fmaxf(tm, lane_xor16(tm));
        tm = fmaxf(tm, lane_xor32(tm));
        const float mnew = fmaxf(m_run, tm);
        const float al = m_run == -INFINITY ? 0.0f : expf(m_run - mnew);
        float ps = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            p[e] = p[e] == -INFINITY ? 0.0f : expf(p[e] - mnew);
            ps += p[e];
        }
        ps += lane_xor16(ps);
        ps += lane_xor32(ps);
        l_run = l_run * al + ps;
        m_run = mnew;
        f16x4 phi, plo;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const _Float16 hv = (_Float16)p[e];
            phi[e] = hv;
            plo[e] = (_Float16)(p[e] - (float)hv);
        }
#pragma unroll
        for (int n = 0; n < NO; n++) o[n] *= al;
        // O^T tile m: rows = dims 8(row + 16(m/8)) + m%8, columns = heads
#pragma unroll
        for (int m = 0; m < NO; m++) {
            const int qq = m / 8, w = (m % 8) / 2;
            const uint32_t sel = (m & 1) ? 0x07060302u : 0x05040100u;
            const v2u pk = (v2u){__builtin_amdgcn_perm(vr[1][qq][w], vr[0][qq][w], sel),
                                 __builtin_amdgcn_perm(vr[3][qq][w], vr[2][qq][w], sel)};
            const f16x4 av = __builtin_bit_cast(f16x4, pk);
            o[m] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, phi, o[m], 0, 0, 0);
            o[m] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, plo, o[m], 0, 0, 0);
        }
        if constexpr (PREF) wv_load_v<HD>(vr, vch, base + 64 + 4 * lg, klast, a.kv_ps, li);
        __builtin_amdgcn_sched_barrier(0);
    };
    for (uint32_t r = 0; r + 1 < nr; r++) round(r, std::true_type{});
    if (nr) round(nr - 1, std::false_type{});
    // merge the waves: lane (li, lg) holds head li's max / sum and O^T rows
    // 4lg+e; each wave scales its rows by its weight exp(m_w - max) once, then
    // the rows are summed in wave order
    if (li < G && lg == 0) {
        mw[wave][li] = m_run;
        lw[wave][li] = l_run;
    }
    __syncthreads();
    float *ow = big;
    if (li < G) {
        const float mx = fmaxf(fmaxf(mw[0][li], mw[1][li]), fmaxf(mw[2][li], mw[3][li]));
        const float wg = m_run == -INFINITY ? 0.0f : expf(m_run - mx);
#pragma unroll
        for (int e = 0; e < 4; e++)
#pragma unroll
            for (int qq = 0; qq < NQ; qq++) {
                float *dst = ow + (wave * GMAX + li) * OWS + 8 * (4 * lg + e + 16 * qq);
                *(f32x4 *)dst = (f32x4){o[qq * 8 + 0][e], o[qq * 8 + 1][e], o[qq * 8 + 2][e], o[qq * 8 + 3][e]} * wg;
                *(f32x4 *)(dst + 4) = (f32x4){o[qq * 8 + 4][e], o[qq * 8 + 5][e], o[qq * 8 + 6][e], o[qq * 8 + 7][e]} * wg;
            }
        if (wave == 0 && lg == 0) {
            float sum = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; w++)
                if (mw[w][li] != -INFINITY) sum += expf(mw[w][li] - mx) * lw[w][li];
            const size_t oi = zoff + (size_t)(h0 + li) * ns + i;
            a.m[oi] = mx;
            a.s[oi] = sum;
        }
    }
    __syncthreads();
    for (uint32_t e = t; e < G * HD / 4; e += TPB) {
        const uint32_t h = e / (HD / 4), d = (e % (HD / 4)) * 4;
        const float *src = ow + h * OWS + d;
        const f32x4 acc = ((*(const f32x4 *)src + *(const f32x4 *)(src + GMAX * OWS)) +
                           *(const f32x4 *)(src + 2 * GMAX * OWS)) + *(const f32x4 *)(src + 3 * GMAX * OWS);
        *(f32x4 *)(a.acc + (zoff + (size_t)(h0 + h) * ns + i) * HD + d) = acc;
    }
}

// SURGE_ATTN_VALU=1 keeps the partial on the VALU kernel (for A/B
// measurement); the MFMA partial is the default for head_dim 128 and 256.
// Read at every launch (a decode state reads it when it captures its graph).
static bool getenv_mf() {
    const char *e = getenv("SURGE_ATTN_VALU");
    return !(e && e[0] == '1');
}

extern "C" hipError_t sgk_attn_partial(const sgk_attn *a, hipStream_t s) {
    if (!a->n_kv || a->n_heads % a->n_kv || a->n_heads / a->n_kv > GMAX) return hipErrorInvalidValue;
    if (a->fuse_prep && (!a->steps || a->ntok != 1 || !a->qn || !a->kn || !a->cs || a->rope_dim > a->hd))
        return hipErrorInvalidValue;
    const uint32_t gx = a->steps ? a->max_splits : a->n_splits;
    if (!gx || !a->ntok) return hipSuccess;
    dim3 grid(gx, a->per_head ? a->n_heads : a->n_kv, a->ntok);
    // q taken as given (the one-shots): the wave-stream kernel's RAW form, which
    // reads q rows as float4
    if (!a->fuse_prep && (a->hd == 128 || a->hd == 256) && ((uintptr_t)a->acc & 15) == 0 && getenv_mf() &&
        ((uintptr_t)a->q & 15) == 0 && (a->q_stride & 3) == 0 && (a->q_tok & 3) == 0) {
        const sgk_attn b = kv_resolved(a);
        if (a->hd == 256) hipLaunchKernelGGL((k_attn_partial_wv<256, WV_RAW>), grid, dim3(TPB), 0, s, b);
        else hipLaunchKernelGGL((k_attn_partial_wv<128, WV_RAW>), grid, dim3(TPB), 0, s, b);
        return hipGetLastError();
    }
    // the wave-stream kernel stores its output rows as float4
    if (a->fuse_prep && (a->hd == 128 || a->hd == 256) && ((uintptr_t)a->acc & 15) == 0 && getenv_mf()) {
        // register prep: rope_dim 64 or 128 and 16-byte aligned q rows, q_norm weights and cos|sin table
        const bool al16 = ((uintptr_t)a->q & 15) == 0 && (a->q_stride & 3) == 0 && (a->q_tok & 3) == 0 &&
                          ((uintptr_t)a->qn & 15) == 0 && ((uintptr_t)a->cs & 15) == 0;
        const int rkb = (al16 && (a->rope_dim == 64 || a->rope_dim == 128)) ? (int)(a->rope_dim / 64) : 0;
        const sgk_attn b = kv_resolved(a);
        if (a->hd == 256) {
            if (rkb == 1) hipLaunchKernelGGL((k_attn_partial_wv<256, 1>), grid, dim3(TPB), 0, s, b);
            else if (rkb == 2) hipLaunchKernelGGL((k_attn_partial_wv<256, 2>), grid, dim3(TPB), 0, s, b);
            else hipLaunchKernelGGL((k_attn_partial_wv<256, 0>), grid, dim3(TPB), 0, s, b);
        } else {
            if (rkb == 1) hipLaunchKernelGGL((k_attn_partial_wv<128, 1>), grid, dim3(TPB), 0, s, b);
            else if (rkb == 2) hipLaunchKernelGGL((k_attn_partial_wv<128, 2>), grid, dim3(TPB), 0, s, b);
            else hipLaunchKernelGGL((k_attn_partial_wv<128, 0>), grid, dim3(TPB), 0, s, b);
        }
        return hipGetLastError();
    }
#define HDCASE(H) case H: hipLaunchKernelGGL((k_attn_partial<H, 64>), grid, dim3(TPB), 0, s, kv_resolved(a)); break
    switch (a->hd) {
        HDCASE(16); HDCASE(32); HDCASE(64); HDCASE(128); HDCASE(256);
    default: return hipErrorInvalidValue;
    }
#undef HDCASE
    return hipGetLastError();
}

// LSE combine (+ optional sigmoid gate). Workgroup (head, token). NaN/inf
// conventions of ref.c:265-373: a NaN first max poisons, all-empty gives 0,
// +inf maxima combine among themselves. Loads do not wait for the merge
// weights: a lane requests its split's max and sum and its first 16 rows of
// acc before the maximum is reduced. Lane = (split group kg, 4-dim chunk),
// each group summing its splits in increasing order, the groups then added in
// order.
template <int HD>
__global__ void __launch_bounds__(TPB) k_attn_combine(sgk_attn a) {
    constexpr int C4 = HD / 4, KG = TPB / C4, PFX = 16;
    __shared__ float wts[1024];
    __shared__ float red[4];
    __shared__ float bc;
    __shared__ float4 part[KG][C4];
    const uint32_t z = blockIdx.y, h = blockIdx.x, t = threadIdx.x;
    const uint32_t ns = a.steps ? dev_splits(a.steps[z].pos + 1, a.prefill, a.split_cap) : a.n_splits;
    const size_t zoff = (size_t)z * a.n_heads * a.max_splits;
    const float *mh = a.m + zoff + (size_t)h * ns, *sh = a.s + zoff + (size_t)h * ns;
    const float4 *acc = (const float4 *)(a.acc + (zoff + (size_t)h * ns) * HD);
    float *oh = a.out + (size_t)z * a.out_tok + (size_t)h * HD;
    const float *gate = a.gate ? a.gate + (size_t)z * a.q_tok + (size_t)h * a.q_stride : NULL;
    // every load that does not depend on the merge weights goes out first:
    // this thread's first split's max and sum, and its first PFX rows of acc
    const uint32_t c = t % C4, kg = t / C4;
    const float m0 = t < ns ? mh[t] : -INFINITY, s0 = t < ns ? sh[t] : 0.0f;
    float4 v[PFX];
#pragma unroll
    for (int u = 0; u < PFX; u++) {
        const uint32_t k = kg + (uint32_t)u * KG;
        v[u] = k < ns ? acc[(size_t)k * C4 + c] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    // the output gate of this thread's four dims, last (it is needed last)
    float gv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (gate && t < (uint32_t)C4) {
#pragma unroll
        for (int e = 0; e < 4; e++) gv[e] = gate[4 * t + e];
    }
    float mx = m0;
    for (uint32_t k = t + TPB; k < ns; k += TPB) mx = fmaxf(mx, mh[k]);
    mx = wave_max(mx);
    if ((t & 63) == 0) red[t >> 6] = mx;
    __syncthreads();
    if (t == 0) bc = (ns && isnan(m0)) ? m0 : fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));   // m0 = mh[0] here
    __syncthreads();
    const float M = bc;
    if (ns == 0 || M == -INFINITY || isnan(M)) {
        const float fill = isnan(M) ? M : 0.0f;
        for (uint32_t dd = t; dd < HD; dd += TPB) oh[dd] = fill;
        return;
    }
    float sp = 0.0f;
    for (uint32_t k = t; k < ns; k += TPB) {
        const float mk = k == t ? m0 : mh[k];
        const float w = (mk == M) ? 1.0f : expf(mk - M);
        wts[k] = w;
        sp += (k == t ? s0 : sh[k]) * w;
    }
    const float S = block_sum(sp, red);   // includes the barrier that publishes wts
    float4 num = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int u = 0; u < PFX; u++) {
        const uint32_t k = kg + (uint32_t)u * KG;
        if (k < ns) {
            const float w = wts[k];
            num.x = fmaf(v[u].x, w, num.x); num.y = fmaf(v[u].y, w, num.y);
            num.z = fmaf(v[u].z, w, num.z); num.w = fmaf(v[u].w, w, num.w);
        }
    }
    uint32_t k = kg + PFX * KG;
    for (; k + 7 * KG < ns; k += 8 * KG) {
        float4 r[8];
#pragma unroll
        for (int u = 0; u < 8; u++) r[u] = acc[(size_t)(k + u * KG) * C4 + c];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const float w = wts[k + u * KG];
            num.x = fmaf(r[u].x, w, num.x); num.y = fmaf(r[u].y, w, num.y);
            num.z = fmaf(r[u].z, w, num.z); num.w = fmaf(r[u].w, w, num.w);
        }
    }
    for (; k < ns; k += KG) {
        const float4 r = acc[(size_t)k * C4 + c];
        const float w = wts[k];
        num.x = fmaf(r.x, w, num.x); num.y = fmaf(r.y, w, num.y);
        num.z = fmaf(r.z, w, num.z); num.w = fmaf(r.w, w, num.w);
    }
    part[kg][c] = num;
    __syncthreads();
    if (t >= (uint32_t)C4) return;
    float4 tot = part[0][t];
    for (int g2 = 1; g2 < KG; g2++) {
        const float4 pv = part[g2][t];
        tot.x += pv.x; tot.y += pv.y; tot.z += pv.z; tot.w += pv.w;
    }
    const float tv[4] = {tot.x, tot.y, tot.z, tot.w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const uint32_t dd = 4 * t + e;
        float o;
        if (isnan(S)) o = S;
        else o = S > 0.0f ? tv[e] / S : 0.0f;
        if (gate) o *= sigm(gv[e]);
        oh[dd] = o;
    }
}

// ---------------------------------------------------------------------------
// Prefill attention on MFMA: causal attention of a chunk of tokens (at
// consecutive positions, after k_attn_prep stored their K/V and prepped q)
// against every key up to each token's position, in one pass per (64-token
// block, query head) with an online softmax, finished in place (divide by the
// row sum, sigmoid output gate), so no partials or combine pass.
//
// Scores are computed transposed, S^T = K Q^T, on v_mfma_f32_16x16x32_f16:
// A = 16 keys straight from the staged f16 K tile, B = 16 tokens' q split
// into f16 hi + lo (q = hi + lo to ~2^-22), two MFMAs per 32 dims. Lane
// (li, lg) then holds token li's scores of keys 4lg..4lg+3 of each 16-key
// block, so a token's tile maximum and sum are in-lane plus two cross-row
// steps, and its probabilities are already the B operand of O^T += V^T P^T
// (p split into f16 hi + lo): the 8 keys of MFMA k-slots 8lg..8lg+7 are keys
// 4lg..4lg+3 of two consecutive 16-key blocks, and V is staged transposed in
// LDS with its keys in that order (an 8 x 8 transpose in registers per
// thread), so an A fragment is one 16-byte read. P never goes through LDS.
// Per 64-key tile: K and V^T staged, one wave per 16-token tile: scores
// (scaled, masked above the token's position), the running max/sum/output
// rescaled as the decode partial does per tile (ref.c:416-555 semantics; a
// fully masked tile leaves a token unchanged), then P V. MFMA 16x16x32 layout
// as in the prefill GEMM. The output is kept transposed (O^T: lane (li, lg)
// holds dims 4lg..4lg+3 of each 16-dim tile of token li), so it is stored as
// float4s.
// ---------------------------------------------------------------------------

// HW query heads per workgroup (1 or 2, heads sharing one kv head): waves
// 4 h' .. 4 h' + 3 take head HW * blockIdx.x + h', so one staged K / V^T tile
// serves HW heads.
template <int HD, int HW>
__global__ void __launch_bounds__(TPB * HW) k_attn_flash(sgk_attn a) {
    static_assert(HD % 64 == 0 && HD <= 256, "flash prefill takes head_dim 64, 128, 192 or 256");
    static_assert(FA_TK == 64, "the V^T key order pairs 16-key blocks within 32-key steps");
    constexpr int KLD = HD + 16, NKB = HD / 32, NNT = HD / 16, NSC = FA_TK / 16;
    // K staging: a key row is KC8 16-byte chunks; consecutive threads take
    // consecutive chunks of a row (contiguous LDS stores, coalesced loads),
    // KPP rows per pass, KNP passes per 64-key tile
    constexpr int KC8 = HD / 8, KPP = TPB / KC8, KNP = (FA_TK + KPP - 1) / KPP;
    constexpr int VDC = HD / 8;                  // V staging: dim chunks of 8 (threads 8*vdc + vkg)
    __shared__ __align__(16) uint16_t ks[FA_TK * KLD];
    __shared__ __align__(16) uint16_t vt[HD * FA_PLD];
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6, li = lane & 15, lg = lane >> 4, tw = wave & 3;
    const uint32_t h = blockIdx.x * HW + (wave >> 2), tb = blockIdx.y, G = a.n_heads / a.n_kv, n_kv = a.n_kv;
    const uint32_t hk = blockIdx.x * HW / G;    // the workgroup's heads share it
    const uint32_t ntok = a.ntok, z0 = tb * FA_TQ;
    const uint32_t base = a.steps[0].pos;
    const uint32_t zlast = min(z0 + FA_TQ, ntok) - 1;
    const uint32_t kend = base + zlast + 1;     // keys 0 .. kend-1 (positions are consecutive)
    const uint16_t *kc = a.kc, *vc = a.vc;
    // split sp of gridDim.z: the key tiles [sp*nt/S, (sp+1)*nt/S) of the block
    const uint32_t S = gridDim.z, sp = blockIdx.z, ntiles = (kend + FA_TK - 1) / FA_TK;
    const uint32_t kbeg = (sp * ntiles / S) * FA_TK, kstop = min(((sp + 1) * ntiles / S) * FA_TK, kend);

    // q fragments of this wave's 16 tokens (B operand: column li = token li,
    // dims 8*lg.. of each 32)
    const uint32_t zq = z0 + tw * 16 + li;      // this lane's token
    f16x8 qh[NKB], ql[NKB];
    {
        const float *qr = a.q + (size_t)min(zq, ntok - 1) * a.q_tok + (size_t)h * a.q_stride;
#pragma unroll
        for (int kb = 0; kb < NKB; kb++) {
            const float4 x0 = *(const float4 *)(qr + kb * 32 + lg * 8);
            const float4 x1 = *(const float4 *)(qr + kb * 32 + lg * 8 + 4);
            const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            fa_split8(xv, qh[kb], ql[kb]);
        }
    }
    const uint32_t rpos = base + zq;            // keys 0..rpos are visible to token zq
    const float sl2 = a.scale * 1.44269504088896340736f;   // scale * log2(e)
    float mrun = -INFINITY, srun = 0.0f;
    f32x4 o[NNT];                               // O^T tile n: dims 16n + 4lg + e of token li
#pragma unroll
    for (int n = 0; n < NNT; n++) o[n] = (f32x4){0.f, 0.f, 0.f, 0.f};

    // Staging roles (256 threads each): with two heads per workgroup waves
    // 0-3 stage K and waves 4-7 V^T, with one head every thread does both.
    // A tile's loads are requested right after the barrier that follows the
    // previous tile's stores, so they arrive while that tile is computed.
    const bool k_role = HW == 1 || t < TPB, v_role = HW == 1 || t >= TPB;
    const uint32_t tv = HW == 1 ? t : t - TPB;
    const uint32_t kk = t / KC8, kd = (t % KC8) * 8;        // K staging role: rows kk + u*KPP
    // V staging role: thread (vdc, vkg) transposes keys 8vkg..8vkg+7 of dims
    // 8vdc..8vdc+7. In a V^T row, key 32m + 16hh + 4q + e sits at column
    // 32m + 8q + 4hh + e (the P^T fragment's k-slot order), so a thread's
    // 8 keys land as two 4-key runs, 8 columns apart.
    const uint32_t vkg = tv % (FA_TK / 8), vdc = tv / (FA_TK / 8);
    const bool v_on = v_role && vdc < (uint32_t)VDC;
    const uint32_t vcol = 32 * (vkg >> 2) + 16 * (vkg & 1) + 4 * ((vkg >> 1) & 1);
    // one register array for both roles: with two heads per workgroup a wave
    // has one role (K in sr[0..KNP), V in sr[0..8)), with one head both
    constexpr int VO = HW == 2 ? 0 : KNP, NSR = HW == 2 ? (KNP > 8 ? KNP : 8) : KNP + 8;
    v4u sr[NSR];
    auto stage_load = [&](uint32_t k0) {         // keys clamped into the range
        if (k_role) {
#pragma unroll
            for (int u = 0; u < KNP; u++) {
                const uint32_t key = min(k0 + min(kk + u * KPP, (uint32_t)FA_TK - 1), kend - 1);
                sr[u] = *(const v4u *)(kc + kv_at(a, key, hk) + kd);
            }
        }
        if (v_on) {
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const uint32_t key = min(k0 + vkg * 8 + j, kend - 1);
                sr[VO + j] = *(const v4u *)(vc + kv_at(a, key, hk) + vdc * 8);
            }
        }
    };
    if (kbeg < kstop) stage_load(kbeg);
    for (uint32_t k0 = kbeg; k0 < kstop; k0 += FA_TK) {
        // stage K [key][dim] and V^T [dim][key, in k-slot order]
        if (k_role) {
#pragma unroll
            for (int u = 0; u < KNP; u++)
                if (kk + u * KPP < (uint32_t)FA_TK) *(v4u *)&ks[(kk + u * KPP) * KLD + kd] = sr[u];
        }
        if (v_on) {
#pragma unroll
            for (int dd = 0; dd < 8; dd++) {
                // half dd of keys 0..7, packed in key order: keys 0-3, then 4-7
                const uint32_t sel = (dd & 1) ? 0x07060302u : 0x05040100u;
                v2u lo2, hi2;
#pragma unroll
                for (int w = 0; w < 2; w++) {
                    lo2[w] = __builtin_amdgcn_perm(sr[VO + 2 * w + 1][dd >> 1], sr[VO + 2 * w][dd >> 1], sel);
                    hi2[w] = __builtin_amdgcn_perm(sr[VO + 2 * w + 5][dd >> 1], sr[VO + 2 * w + 4][dd >> 1], sel);
                }
                uint16_t *row = &vt[(vdc * 8 + dd) * FA_PLD + vcol];
                *(v2u *)row = lo2;
                *(v2u *)(row + 8) = hi2;
            }
        }
        __syncthreads();
        if (k0 + FA_TK < kstop) stage_load(k0 + FA_TK);
        // scores S^T: lane (li, lg) gets token li's scores of keys 16n + 4lg + e
        f32x4 sc[NSC];
#pragma unroll
        for (int n = 0; n < NSC; n++) sc[n] = (f32x4){0.f, 0.f, 0.f, 0.f};
        // K fragments (kb, n) in order i = kb * NSC + n, each requested two
        // fragments before its MFMAs (a ring of three)
        {
            auto kfrag = [&](int i) {
                return *(const f16x8 *)&ks[((i % NSC) * 16 + li) * KLD + (i / NSC) * 32 + lg * 8];
            };
            f16x8 bk[3];
            bk[0] = kfrag(0);
            bk[1] = kfrag(1);
#pragma unroll
            for (int i = 0; i < NKB * NSC; i++) {
                if (i + 2 < NKB * NSC) bk[(i + 2) % 3] = kfrag(i + 2);
                const int kb = i / NSC, n = i % NSC;
                sc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bk[i % 3], qh[kb], sc[n], 0, 0, 0);
                sc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bk[i % 3], ql[kb], sc[n], 0, 0, 0);
            }
        }
        // online softmax of token li over this tile's keys, in base 2: the
        // scores are scaled by scale * log2(e), so p = 2^(s - m) on the
        // hardware exp2 (the running max m is kept in that domain)
        float tm = -INFINITY;
#pragma unroll
        for (int n = 0; n < NSC; n++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t key = k0 + n * 16 + lg * 4 + e;
                sc[n][e] = key <= rpos ? sc[n][e] * sl2 : -INFINITY;
                tm = fmaxf(tm, sc[n][e]);
            }
        tm = fmaxf(tm, lane_xor16(tm));
        tm = fmaxf(tm, lane_xor32(tm));
        const float mnew = fmaxf(mrun, tm);
        float ps_sum = 0.0f;
#pragma unroll
        for (int n = 0; n < NSC; n++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t key = k0 + n * 16 + lg * 4 + e;
                const float pv = key <= rpos ? __builtin_amdgcn_exp2f(sc[n][e] - mnew) : 0.0f;
                sc[n][e] = pv;
                ps_sum += pv;
            }
        ps_sum += lane_xor16(ps_sum);
        ps_sum += lane_xor32(ps_sum);
        const float al = (mrun == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mrun - mnew);
        mrun = mnew;
        srun = srun * al + ps_sum;
        // most tiles at depth leave every running max of the wave unchanged
        if (__builtin_amdgcn_ballot_w64(al != 1.0f)) {
#pragma unroll
            for (int n = 0; n < NNT; n++) o[n] *= al;
        }
        // O^T += V^T P^T per 32-key step m: k-slots 8lg+e and 8lg+4+e are
        // keys 32m + 4lg + e and 32m + 16 + 4lg + e
        f16x8 ph[FA_TK / 32], pl[FA_TK / 32];
#pragma unroll
        for (int m = 0; m < FA_TK / 32; m++)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float pv = sc[2 * m + (e >> 2)][e & 3];
                const _Float16 hv = (_Float16)pv;
                ph[m][e] = hv;
                pl[m][e] = (_Float16)(pv - (float)hv);
            }
        // V^T fragments (m, n) in order i = m * NNT + n, each requested two
        // fragments ahead, as the K fragments
        {
            auto vfrag = [&](int i) {
                return *(const f16x8 *)&vt[((i % NNT) * 16 + li) * FA_PLD + (i / NNT) * 32 + lg * 8];
            };
            f16x8 av[3];
            av[0] = vfrag(0);
            av[1] = vfrag(1);
#pragma unroll
            for (int i = 0; i < (FA_TK / 32) * NNT; i++) {
                if (i + 2 < (FA_TK / 32) * NNT) av[(i + 2) % 3] = vfrag(i + 2);
                const int m = i / NNT, n = i % NNT;
                o[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i % 3], ph[m], o[n], 0, 0, 0);
                o[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i % 3], pl[m], o[n], 0, 0, 0);
            }
        }
        __syncthreads();
    }
    if (zq >= ntok) return;
    if (S > 1) {
        // partials in the decode layout [token][head][split] for k_attn_combine:
        // m the running max, s the running sum, acc the unnormalised output
        const size_t ph = ((size_t)zq * a.n_heads + h) * S + sp;
        if (lg == 0) { a.m[ph] = mrun * 0.69314718055994530942f; a.s[ph] = srun; }   // the max back in base e
        float *acc = a.acc + ph * HD;
#pragma unroll
        for (int n = 0; n < NNT; n++) *(f32x4 *)(acc + n * 16 + lg * 4) = o[n];
        return;
    }
    // finish: o / s, sigmoid gate, store (lane: token li, dims 16n + 4lg + e)
    float *out = a.out + (size_t)zq * a.out_tok + (size_t)h * HD;
    const float *gate = a.gate ? a.gate + (size_t)zq * a.q_tok + (size_t)h * a.q_stride : NULL;
#pragma unroll
    for (int n = 0; n < NNT; n++) {
        const uint32_t d0 = n * 16 + lg * 4;
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float x = isnan(srun) ? srun : (srun > 0.0f ? o[n][e] / srun : 0.0f);
            if (gate) x *= sigm(gate[d0 + e]);
            v[e] = x;
        }
        *(f32x4 *)(out + d0) = v;
    }
}

extern "C" hipError_t sgk_attn_combine(const sgk_attn *a, hipStream_t s);

// Launch the flash pass. A chunk has few (token block, head) pairs (192 for
// 512 tokens x 24 heads on 256 CUs) and each walks every key up to its
// tokens, so deep chunks split their key tiles over up to a->max_splits
// workgroups, about one per FA_SPLIT_KEYS keys of the deepest block
// (a->seq = the position after the chunk's last token, 0 = unknown: no
// split), when a->m, s, acc hold ntok x n_heads x max_splits partials. The
// splits write partials and k_attn_combine merges them in split order and
// applies the gate.
#define FA_SPLIT_KEYS 512u
extern "C" hipError_t sgk_attn_flash(const sgk_attn *a, hipStream_t s) {
    if (!a->ntok || !a->n_heads) return hipSuccess;
    if (!a->steps || !a->n_kv || a->n_heads % a->n_kv || ((uintptr_t)a->q & 15) || a->q_stride % 4 || a->q_tok % 4)
        return hipErrorInvalidValue;
    if (a->hd != 64 && a->hd != 128 && a->hd != 256) return hipErrorInvalidValue;
    // the output rows (and the split partials) are stored as float4s
    if (((uintptr_t)a->out & 15) || a->out_tok % 4 || (a->acc && ((uintptr_t)a->acc & 15))) return hipErrorInvalidValue;
    uint32_t S = 1;
    if (a->m && a->s && a->acc && a->max_splits > 1 && a->seq > FA_SPLIT_KEYS)
        S = min(a->max_splits, (a->seq + FA_SPLIT_KEYS - 1) / FA_SPLIT_KEYS);
    sgk_attn k = kv_resolved(a);
    k.max_splits = S;
    // two query heads per workgroup when their group size allows
    const uint32_t hw = (a->n_heads / a->n_kv) % 2 == 0 ? 2 : 1;
    dim3 grid(a->n_heads / hw, (a->ntok + FA_TQ - 1) / FA_TQ, S);
#define FLC(H) do { if (hw == 2) hipLaunchKernelGGL((k_attn_flash<H, 2>), grid, dim3(2 * TPB), 0, s, k);       \
                     else hipLaunchKernelGGL((k_attn_flash<H, 1>), grid, dim3(TPB), 0, s, k); } while (0)
    switch (a->hd) {
    case 64: FLC(64); break;
    case 128: FLC(128); break;
    case 256: FLC(256); break;
    }
#undef FLC
    if (S == 1) return hipGetLastError();
    sgk_attn c = k;
    c.steps = NULL;                 // every token has the same S splits
    c.n_splits = S;
    return sgk_attn_combine(&c, s);
}

extern "C" hipError_t sgk_attn_combine(const sgk_attn *a, hipStream_t s) {
    if (!a->n_heads || !a->ntok) return hipSuccess;
    if (!a->steps && a->n_splits > 1024) return hipErrorInvalidValue;
    dim3 grid(a->n_heads, a->ntok);
#define HDCASE(H) case H: hipLaunchKernelGGL(k_attn_combine<H>, grid, dim3(TPB), 0, s, *a); break
    switch (a->hd) {
        HDCASE(16); HDCASE(32); HDCASE(64); HDCASE(128); HDCASE(256);
    default: return hipErrorInvalidValue;
    }
#undef HDCASE
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Gated DeltaNet.
// ---------------------------------------------------------------------------

#define GDN_ROWS 16   // value rows per workgroup (4 per wave)

// One delta-rule row update held across a wave (ref.c:708-739): element i of
// the row lives in lane i / EPL, slot i % EPL (EPL = DK / 64, or one lane per
// element when DK < 64). s[] holds the row; returns y_j, the readout AFTER
// the write. Decode and the prefill scan share this arithmetic exactly.
template <int DK>
struct drow { static constexpr int EPL = DK >= 64 ? DK / 64 : 1; };

template <int DK>
__device__ __forceinline__ float delta_update(float *s, const float *kk, const float *qq, float vj,
                                              float beta, float decay, uint32_t lane) {
    constexpr int EPL = drow<DK>::EPL;
    const bool on = DK >= 64 || lane < (uint32_t)DK;
    float k[EPL], q[EPL];
#pragma unroll
    for (int e = 0; e < EPL; e++) {
        k[e] = on ? kk[lane * EPL + e] : 0.0f;
        q[e] = on ? qq[lane * EPL + e] : 0.0f;
    }
    float kv = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; e++) { s[e] *= decay; kv = fmaf(s[e], k[e], kv); }
    kv = wave_sum(kv);
    const float delta = (vj - kv) * beta;
    float y = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; e++) { s[e] = fmaf(k[e], delta, s[e]); y = fmaf(s[e], q[e], y); }
    return wave_sum(y);
}

template <int DK>
__device__ __forceinline__ void row_load(float *s, const float *row, uint32_t lane) {
#pragma unroll
    for (int e = 0; e < drow<DK>::EPL; e++)
        s[e] = (DK >= 64 || lane < (uint32_t)DK) ? row[lane * drow<DK>::EPL + e] : 0.0f;
}
template <int DK>
__device__ __forceinline__ void row_store(const float *s, float *row, uint32_t lane) {
    if (DK >= 64 || lane < (uint32_t)DK) {
#pragma unroll
        for (int e = 0; e < drow<DK>::EPL; e++) row[lane * drow<DK>::EPL + e] = s[e];
    }
}

template <int DK>
__device__ __forceinline__ float delta_row(float *row, const float *kk, const float *qq, float vj,
                                           float beta, float decay, uint32_t lane) {
    float sr[drow<DK>::EPL];
    row_load<DK>(sr, row, lane);
    const float y = delta_update<DK>(sr, kk, qq, vj, beta, decay, lane);
    row_store<DK>(sr, row, lane);
    return y;
}

// The per-head gates (ref.c:127-170): beta = sigmoid(b); decay by the stored form.
__device__ __forceinline__ void gdn_gates(float b, float a, float ssm_a, float dt, int neg_exp,
                                          float *beta, float *decay) {
    *beta = sigm(b);
    const float sp = softplus(a + dt);
    *decay = neg_exp ? expf(ssm_a * sp) : expf(-(expf(ssm_a) * sp));
}

// Sum over the 64 lanes of a wave of RW per-lane partials at once (one per
// state row, RW <= 16): a transposed butterfly that halves the rows a lane
// carries at each of the first log2(RW) steps (lane bits 5, 4, 3, 2 in that
// order; the bit-2 step pairs lane l with l^7, which flips bit 2 and leaves
// the pair in the same 8 lanes), then sums over the remaining lane bits.
// Returns the full sum of row rows_row<RW>(lane); lanes that agree in the top
// log2(RW) bits agree in the result. A fixed tree: reruns are bit-identical.
template <int LVL>
__device__ __forceinline__ float rows_partner(float v) {
    if (LVL == 0) return lane_xor32(v);
    if (LVL == 1) return lane_xor16(v);
    if (LVL == 2) return lane_xor8(v);
    return lane_mir8(v);
}
template <int RW, int LVL = 0>
__device__ __forceinline__ void rows_fold(float *v, uint32_t lane) {
    if constexpr (RW > 1) {
        const bool hi = lane & (32u >> LVL);
#pragma unroll
        for (int r = 0; r < RW / 2; r++) {
            const float mine = hi ? v[r + RW / 2] : v[r], other = hi ? v[r] : v[r + RW / 2];
            v[r] = mine + rows_partner<LVL>(other);
        }
        rows_fold<RW / 2, LVL + 1>(v, lane);
    } else {
        // sum over the lane bits below the ones used for rows
        float s = v[0];
        s += lane_xor1(s);
        s += lane_xor2(s);
        if (LVL <= 3) s += lane_mir8(s);
        if (LVL <= 2) s += lane_xor8(s);
        if (LVL <= 1) s += lane_xor16(s);
        if (LVL == 0) s += lane_xor32(s);
        v[0] = s;
    }
}
template <int RW>
__device__ __forceinline__ float rows_sum(float *v, uint32_t lane) {
    static_assert(RW >= 1 && RW <= 16, "rows_sum: 1..16 rows");
    rows_fold<RW>(v, lane);
    return v[0];
}
template <int RW>
__device__ __forceinline__ uint32_t rows_row(uint32_t lane) {
    constexpr int LB = RW >= 32 ? 5 : RW >= 16 ? 4 : RW >= 8 ? 3 : RW >= 4 ? 2 : RW >= 2 ? 1 : 0;
    return LB ? (lane >> (6 - LB)) & (RW - 1) : 0;
}
template <int RW>
__device__ __forceinline__ uint32_t rows_lane(uint32_t r) {   // a lane holding row r
    constexpr int LB = RW >= 32 ? 5 : RW >= 16 ? 4 : RW >= 8 ? 3 : RW >= 4 ? 2 : RW >= 2 ? 1 : 0;
    return LB ? r << (6 - LB) : 0;
}

// Gated DeltaNet decode step for one layer (reference ref.c:669-739 +
// 1273-1330, kernels.metal:520-548, 742-805, 109-134). Workgroup (value head
// h, row block jb) of GDN_NB per head: causal conv of the head's q/k channels
// and of its rows' v channels over the position-indexed ring + SiLU, q/k RMS
// (eps 1e-6, no weight) then q/dk and k/sqrt(dk), beta/decay, the rank-1
// delta update of its dv/GDN_NB state rows with their readout, all requested
// before any arithmetic. Wave w updates RW rows; each row's two dot products
// are reduced for all of them at once (rows_sum). With one block per head the
// block finishes RMSNormGated itself; with several, the head's factor needs
// every block's readouts, so it is left to the output projection's gated
// prologue: each block writes silu(z) * (y * w) of its rows and the sum of its
// rows' squared readouts, with no synchronisation between blocks.
template <int DK, int RW, int NB, int GDN_TPB>
__device__ __forceinline__ void gdn_step_body(const sgk_gdn &a, uint32_t h, uint32_t jb) {
    constexpr int GDN_NB = NB;
    constexpr int EPL = DK >= 64 ? DK / 64 : 1;
    constexpr int NW = GDN_TPB / 64;
    __shared__ float qk[2 * DK];
    __shared__ float vv[NW * RW];
    __shared__ float red[NW];
    __shared__ float ysh[SGK_GDN_MAX_DV];
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint32_t dk = DK, dv = a.dv, key_dim = a.n_k * dk, cd = a.conv_dim;
    const uint32_t rpb = (dv + GDN_NB - 1) / GDN_NB, jlo = jb * rpb, jhi = min(dv, jlo + rpb);
    const uint32_t hk = a.tiled ? h % a.n_k : h / (a.n_v / a.n_k);
    const uint32_t pos = a.step->pos, keep = a.ksize - 1;
    // The ring slot of the q/k channels is written by block 0 of the first
    // value head mapped to hk only (one writer per channel).
    const bool qk_writer = jb == 0 && (a.tiled ? h < a.n_k : (h % (a.n_v / a.n_k)) == 0);
    const bool on = DK >= 64 || lane < (uint32_t)DK;
    float *Sh = a.S + (size_t)h * dv * dk;

    // 1. requests, smallest first (loads retire in order, so the conv inputs
    //    must not queue behind the state rows): the conv input and taps, z and
    //    the gate inputs, the ring (its slots need the position), then this
    //    wave's state rows. Every load is unconditional at a clamped index and
    //    the tap loops have a fixed trip count, so nothing waits until all of
    //    them are in flight. The state rows are read and written back
    //    non-temporally (each is touched once per token): 4k decode
    //    182.6 -> 185.8 tok/s, 262000 keys 127.3 -> 128.9.
    const uint32_t nch = 2 * dk + (jhi - jlo);
    auto chan = [&](uint32_t e) -> uint32_t {
        if (e < dk) return hk * dk + e;
        if (e < 2 * dk) return key_dim + hk * dk + (e - dk);
        return 2 * key_dim + h * dv + jlo + (e - 2 * dk);
    };
    // All four ring slots are loaded (their addresses need no position), the
    // taps' slots picked once the position is in. A thread's first two
    // channels (t and t + GDN_TPB) are both requested here: the 27B's 288
    // channels per block gave 32 threads a second channel whose loads, issued
    // after the first one's arithmetic, were a memory round trip of their own
    // in front of the barrier.
    float4 cw0, rs0, cw1, rs1;
    float cx0, cx1;
    auto conv_loads = [&](float &cx, float4 &cw, float4 &rs, uint32_t c) {
        cx = a.in[c];
        cw.x = a.conv_w[(size_t)c * a.ksize];
        cw.y = a.conv_w[(size_t)c * a.ksize + min(1u, keep)];
        cw.z = a.conv_w[(size_t)c * a.ksize + min(2u, keep)];
        cw.w = a.conv_w[(size_t)c * a.ksize + min(3u, keep)];
        rs.x = a.ring[c];
        rs.y = a.ring[(size_t)cd + c];
        rs.z = a.ring[(size_t)2 * cd + c];
        rs.w = a.ring[(size_t)3 * cd + c];
    };
    const uint32_t ch0 = chan(min(t, nch - 1)), ch1 = chan(min(t + GDN_TPB, nch - 1));
    conv_loads(cx0, cw0, rs0, ch0);
    conv_loads(cx1, cw1, rs1, ch1);
    const float zraw = a.z[(size_t)h * dv + min(max(t, jlo), jhi - 1)];
    const float nwt = a.norm_w[min(t, dv - 1)];   // needed last, loaded early
    const float *bb = a.in + cd + a.n_v * dv, *aa = bb + a.n_v;
    const float gb = bb[h], ga = aa[h], gA = a.ssm_a[h], gdt = a.dt_bias[h];
    const uint32_t j0 = jlo + wave * RW;
    float sr[RW][EPL];
#pragma unroll
    for (int r = 0; r < RW; r++) {
        const uint32_t j = min(j0 + r, jhi - 1);
#pragma unroll
        for (int e = 0; e < EPL; e++) sr[r][e] = __builtin_nontemporal_load(Sh + (size_t)j * dk + (on ? lane * EPL + e : 0));
    }
    const float zj = (t >= jlo && t < jhi) ? zraw : 0.0f;
#pragma unroll
    for (int r = 0; r < RW; r++)
#pragma unroll
        for (int e = 0; e < EPL; e++) sr[r][e] = (j0 + r < jhi && on) ? sr[r][e] : 0.0f;

    // 2. conv + SiLU (the taps in order, then the current input; ref.c
    //    conv1d step); this step's input into the ring slot pos % 4.
    auto conv_out = [&](uint32_t e, uint32_t c, float cx, float4 cw, float4 rs) {
        float acc = 0.0f;
#pragma unroll
        for (uint32_t jj = 0; jj < 3; jj++) {
            const uint32_t sl = (pos + 4 - keep + jj) & 3;
            const float cr = sl == 0 ? rs.x : sl == 1 ? rs.y : sl == 2 ? rs.z : rs.w;
            const float wj = jj == 0 ? cw.x : jj == 1 ? cw.y : cw.z;
            if (jj < keep) acc = fmaf(wj, cr, acc);
        }
        const float wcur = keep == 0 ? cw.x : keep == 1 ? cw.y : keep == 2 ? cw.z : cw.w;
        acc = fmaf(wcur, cx, acc);
        const float o = silu(acc);
        if (e < nch) {
            if (e < 2 * dk) qk[e] = o; else vv[e - 2 * dk] = o;
            if (e >= 2 * dk || qk_writer) a.ring[(size_t)(pos & 3) * cd + c] = cx;
        }
    };
    // computed unconditionally (only the stores are guarded), so the second
    // channel's loads stay up front instead of sinking into a branch
    conv_out(t, ch0, cx0, cw0, rs0);
    conv_out(t + GDN_TPB, ch1, cx1, cw1, rs1);
    for (uint32_t e = t + 2 * GDN_TPB; e < nch; e += GDN_TPB) {     // wider blocks than the shapes in use
        const uint32_t c = chan(e);
        conv_loads(cx0, cw0, rs0, c);
        conv_out(e, c, cx0, cw0, rs0);
    }
    __syncthreads();
    // 3. q, k: RMS (eps 1e-6, no weight), then q / dk and k / sqrt(dk).
    if (wave < 2) {
        const float *src = qk + wave * dk;
        float ss = 0.0f;
        for (uint32_t i = lane; i < dk; i += 64) ss = fmaf(src[i], src[i], ss);
        ss = wave_sum(ss);
        if (lane == 0) red[wave] = ss;
    }
    __syncthreads();
    const float rq = 1.0f / sqrtf(red[0] / (float)dk + 1e-6f), rk = 1.0f / sqrtf(red[1] / (float)dk + 1e-6f);
    const float qsc = 1.0f / (float)dk, ksc = 1.0f / sqrtf((float)dk);
    float kq[EPL], qq[EPL];
#pragma unroll
    for (int e = 0; e < EPL; e++) {
        const uint32_t i = on ? lane * EPL + e : 0;
        qq[e] = on ? (qk[i] * rq) * qsc : 0.0f;
        kq[e] = on ? (qk[dk + i] * rk) * ksc : 0.0f;
    }
    float beta, decay;                                  // every thread, from scalar loads
    gdn_gates(gb, ga, gA, gdt, a.neg_exp, &beta, &decay);
    // 4. rank-1 update and readout of this wave's rows.
    float ss_part = 0.0f;
    if (j0 < jhi) {
        float part[RW];
#pragma unroll
        for (int r = 0; r < RW; r++) {
            float kv = 0.0f;
#pragma unroll
            for (int e = 0; e < EPL; e++) { sr[r][e] *= decay; kv = fmaf(sr[r][e], kq[e], kv); }
            part[r] = kv;
        }
        const uint32_t myrow = rows_row<RW>(lane);
        const float kvr = rows_sum<RW>(part, lane);
        const float vj = j0 + myrow < jhi ? vv[wave * RW + myrow] : 0.0f;
        const float dmine = (vj - kvr) * beta;
#pragma unroll
        for (int r = 0; r < RW; r++) {
            const float dr = lane_read(dmine, rows_lane<RW>(r));
            float y = 0.0f;
#pragma unroll
            for (int e = 0; e < EPL; e++) { sr[r][e] = fmaf(kq[e], dr, sr[r][e]); y = fmaf(sr[r][e], qq[e], y); }
            part[r] = y;
        }
        const float yr = rows_sum<RW>(part, lane);
        const bool owner = (lane & (64 / RW - 1)) == 0 && j0 + myrow < jhi;
        if (owner) ysh[j0 + myrow] = yr;
        // sum of squares of this wave's readouts, in row order
        float yy[RW];
#pragma unroll
        for (int r = 0; r < RW; r++) {
            const float yv = lane_read(yr, rows_lane<RW>(r));
            yy[r] = (j0 + r < jhi) ? yv * yv : 0.0f;
        }
#pragma unroll
        for (int r = 0; r < RW; r++) ss_part += yy[r];
#pragma unroll
        for (int r = 0; r < RW; r++) {
            const uint32_t j = j0 + r;
            if (j < jhi && on) {
#pragma unroll
                for (int e = 0; e < EPL; e++) __builtin_nontemporal_store(sr[r][e], Sh + (size_t)j * dk + lane * EPL + e);
            }
        }
    }
    if (lane == 0) red[wave] = ss_part;
    __syncthreads();
    if (NB == 1) {
        // 5. the whole head is here: RMSNormGated in place (ref.c:1322-1330),
        //    silu(z) * (y * rsqrt(mean y^2 + eps) * w).
        float tot = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; w++) tot += red[w];
        const float r = 1.0f / sqrtf(tot / (float)dv + a.eps);
        if (t < dv) {
            const float yv = ysh[t];
            a.out[(size_t)h * dv + t] = silu(zj) * ((yv * r) * nwt);
        }
        return;
    }
    // 5. this block's sum of squared readouts, and silu(z) * (y * w) of its
    //    rows: the output projection's gated prologue finishes RMSNormGated
    //    with the head's factor from the blocks' sums.
    if (t == 0) {
        float sb = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; w++) sb += red[w];
        a.ss[(size_t)h * GDN_NB + jb] = sb;
    }
    if (t >= jlo && t < jhi) a.out[(size_t)h * dv + t] = silu(zj) * (ysh[t] * nwt);
}

template <int DK, int RW, int NB, int GDN_TPB>
__global__ void __launch_bounds__(GDN_TPB) k_gdn_step(sgk_gdn a) {
    gdn_step_body<DK, RW, NB, GDN_TPB>(a, blockIdx.x, blockIdx.y);
}

extern "C" hipError_t sgk_gdn_step(const sgk_gdn *a, hipStream_t s) {
    if (a->ksize < 1 || a->ksize > 4 || !a->n_k || a->n_v % a->n_k) return hipErrorInvalidValue;
    if (!a->dv || a->dv > SGK_GDN_MAX_DV || !a->z || !a->out) return hipErrorInvalidValue;
    if (a->blocks == 1) {
        // one 512-thread workgroup per head, 16 rows per wave (dv <= 128) or
        // 32 (dv <= 256, two passes of 16 are not needed: RW = 16 covers 128)
        if (!a->norm_w || a->dv > 128) return hipErrorInvalidValue;
        const uint32_t rw = (a->dv + 7) / 8;
        dim3 grid(a->n_v, 1);
#define DKCASE1(D) case D:                                                                               \
        if (rw <= 1) hipLaunchKernelGGL((k_gdn_step<D, 1, 1, 512>), grid, dim3(512), 0, s, *a);          \
        else if (rw <= 2) hipLaunchKernelGGL((k_gdn_step<D, 2, 1, 512>), grid, dim3(512), 0, s, *a);     \
        else if (rw <= 4) hipLaunchKernelGGL((k_gdn_step<D, 4, 1, 512>), grid, dim3(512), 0, s, *a);     \
        else if (rw <= 8) hipLaunchKernelGGL((k_gdn_step<D, 8, 1, 512>), grid, dim3(512), 0, s, *a);     \
        else hipLaunchKernelGGL((k_gdn_step<D, 16, 1, 512>), grid, dim3(512), 0, s, *a);                 \
        break
        switch (a->dk) {
            DKCASE1(32); DKCASE1(64); DKCASE1(128); DKCASE1(256);
        default: return hipErrorInvalidValue;
        }
#undef DKCASE1
        return hipGetLastError();
    }
    if (!a->norm_w || !a->ss || a->dv > SGK_GDN_MAX_DV) return hipErrorInvalidValue;
    const uint32_t rpb = (a->dv + SGK_GDN_BLOCKS - 1) / SGK_GDN_BLOCKS;    // rows per block, at most 64
    dim3 grid(a->n_v, SGK_GDN_BLOCKS);
#define DKCASE(D) case D:                                                                                  \
        if (rpb <= 4) hipLaunchKernelGGL((k_gdn_step<D, 1, SGK_GDN_BLOCKS, 256>), grid, dim3(256), 0, s, *a);        \
        else if (rpb <= 8) hipLaunchKernelGGL((k_gdn_step<D, 2, SGK_GDN_BLOCKS, 256>), grid, dim3(256), 0, s, *a);   \
        else if (rpb <= 16) hipLaunchKernelGGL((k_gdn_step<D, 4, SGK_GDN_BLOCKS, 256>), grid, dim3(256), 0, s, *a);  \
        else if (rpb <= 32) hipLaunchKernelGGL((k_gdn_step<D, 8, SGK_GDN_BLOCKS, 256>), grid, dim3(256), 0, s, *a);  \
        else hipLaunchKernelGGL((k_gdn_step<D, 16, SGK_GDN_BLOCKS, 256>), grid, dim3(256), 0, s, *a);                \
        break
    switch (a->dk) {
        DKCASE(32); DKCASE(64); DKCASE(128); DKCASE(256);
    default: return hipErrorInvalidValue;
    }
#undef DKCASE
    return hipGetLastError();
}

template <int DK>
__global__ void __launch_bounds__(TPB) k_delta_multi(float *S, const float *qkv, float *out,
                                                     const float *gates, uint32_t dv, uint32_t n_v,
                                                     uint32_t n_k, uint32_t key_dim, int tiled) {
    const uint32_t h = blockIdx.x, j0 = blockIdx.y * GDN_ROWS;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t hk = (n_k && n_v >= n_k) ? (tiled ? h % n_k : h / (n_v / n_k)) : 0;
    const float *qq = qkv + (size_t)hk * DK, *kk = qkv + key_dim + (size_t)hk * DK;
    const float *v = qkv + 2 * (size_t)key_dim + (size_t)h * dv;
    const float beta = gates[h], decay = gates[n_v + h];
    float *Sh = S + (size_t)h * dv * DK;
    for (uint32_t r = wave; r < GDN_ROWS && j0 + r < dv; r += TPB / 64) {
        const uint32_t j = j0 + r;
        const float y = delta_row<DK>(Sh + (size_t)j * DK, kk, qq, v[j], beta, decay, lane);
        if (lane == 0) out[(size_t)h * dv + j] = y;
    }
}

extern "C" hipError_t sgk_delta_multi(float *S, const float *qkv, float *out, const float *gates,
                                      uint32_t dk, uint32_t dv, uint32_t n_v, uint32_t n_k,
                                      uint32_t key_dim, int tiled, hipStream_t s) {
    dim3 grid(n_v, (dv + GDN_ROWS - 1) / GDN_ROWS);
    if (!n_v || !dv) return hipSuccess;
    switch (dk) {
    case 32: hipLaunchKernelGGL(k_delta_multi<32>, grid, dim3(TPB), 0, s, S, qkv, out, gates, dv, n_v, n_k, key_dim, tiled); break;
    case 64: hipLaunchKernelGGL(k_delta_multi<64>, grid, dim3(TPB), 0, s, S, qkv, out, gates, dv, n_v, n_k, key_dim, tiled); break;
    case 128: hipLaunchKernelGGL(k_delta_multi<128>, grid, dim3(TPB), 0, s, S, qkv, out, gates, dv, n_v, n_k, key_dim, tiled); break;
    case 256: hipLaunchKernelGGL(k_delta_multi<256>, grid, dim3(TPB), 0, s, S, qkv, out, gates, dv, n_v, n_k, key_dim, tiled); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Single-token causal conv: state oldest-first [ksize-1][channels] (ref.c:669-706).
__global__ void k_conv1d_step(const float *x, const float *w, float *y, float *state,
                              uint32_t channels, uint32_t ksize) {
    const uint32_t c = blockIdx.x * TPB + threadIdx.x;
    if (c >= channels) return;
    const uint32_t keep = ksize - 1;
    const float *wc = w + (size_t)c * ksize;
    const float cur = x[c];
    float acc = 0.0f;
    for (uint32_t j = 0; j < keep; j++) acc = fmaf(wc[j], state[(size_t)j * channels + c], acc);
    acc = fmaf(wc[keep], cur, acc);
    for (uint32_t j = 0; j + 1 < keep; j++) state[(size_t)j * channels + c] = state[(size_t)(j + 1) * channels + c];
    if (keep) state[(size_t)(keep - 1) * channels + c] = cur;
    y[c] = acc;
}

extern "C" hipError_t sgk_conv1d_step(const float *x, const float *w, float *y, float *state,
                                      uint32_t channels, uint32_t ksize, hipStream_t s) {
    if (!channels || !ksize) return hipSuccess;
    hipLaunchKernelGGL(k_conv1d_step, dim3((channels + TPB - 1) / TPB), dim3(TPB), 0, s, x, w, y,
                       state, channels, ksize);
    return hipGetLastError();
}

__global__ void __launch_bounds__(TPB) k_rmsnorm_gated(const float *y, const float *z,
                                                       const float *w, float *out, uint32_t dv,
                                                       float eps) {
    __shared__ float red[4];
    const size_t o = (size_t)blockIdx.x * dv;
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < dv; i += TPB) { float v = y[o + i]; ss = fmaf(v, v, ss); }
    ss = block_sum(ss, red);
    const float r = 1.0f / sqrtf(ss / (float)dv + eps);
    for (uint32_t i = threadIdx.x; i < dv; i += TPB) out[o + i] = silu(z[o + i]) * ((y[o + i] * r) * w[i]);
}

extern "C" hipError_t sgk_rmsnorm_gated(const float *y, const float *z, const float *w,
                                        float *out, uint32_t dv, uint32_t heads, float eps,
                                        hipStream_t s) {
    if (!heads || !dv) return hipSuccess;
    hipLaunchKernelGGL(k_rmsnorm_gated, dim3(heads), dim3(TPB), 0, s, y, z, w, out, dv, eps);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Gated DeltaNet over a prefill chunk: the same arithmetic as the decode step,
// scanned over the chunk's tokens in order (state threaded through).
// ---------------------------------------------------------------------------

// Causal conv + SiLU over a chunk at consecutive positions pos0 .. pos0+ntok-1
// (the ring holds the inputs of the positions before pos0 by slot p % 4, as
// in decode). Thread (channel, block of CC_TOK tokens): the taps of token z
// are the chunk's own inputs for positions inside the chunk, else the ring
// slots; each output is the taps in order, then the current input (the
// decode step's arithmetic). The ring is only read here: k_conv_ring writes
// the chunk's last inputs into it afterwards.
// With hw = 1 or 2 the q and k heads (channels below qk_end, hw waves of
// dk = 64 hw channels each, so no head crosses a workgroup) also get k_qk_norm_chunk's
// RMS and scale before they are written: each wave sums its squares with
// wave_sum, and a head's waves are added in block_sum's order (the same
// per-lane values in the same lanes, so the same bits as the separate pass).
#define CC_TOK 16
__global__ void __launch_bounds__(TPB) k_conv_chunk(const float *in, uint32_t in_stride, const float *conv_w,
                                                    const float *ring, float *out, const sgk_step *steps,
                                                    uint32_t ntok, uint32_t cd, uint32_t ksize, uint32_t qk_end,
                                                    uint32_t hw) {
    __shared__ float red[4][CC_TOK];
    const uint32_t ch = blockIdx.x * TPB + threadIdx.x, z0 = blockIdx.y * CC_TOK;
    const bool live = ch < cd;
    const uint32_t keep = ksize - 1, pos0 = steps[0].pos;
    float o[CC_TOK];
    if (live) {
        float w[4], x[CC_TOK + 3];
#pragma unroll
        for (uint32_t j = 0; j < 4; j++) w[j] = conv_w[(size_t)ch * ksize + min(j, keep)];
        // x[3 + i] = input of token z0 + i; x[0..2] = the three before z0
#pragma unroll
        for (int i = 0; i < CC_TOK + 3; i++) {
            const int z = (int)z0 + i - 3;
            const uint32_t zc = (uint32_t)min(max(z, 0), (int)ntok - 1);
            const float vi = in[(size_t)zc * in_stride + ch];
            const float vr = ring[(size_t)((pos0 + 4 + (uint32_t)min(z, 0)) & 3) * cd + ch];
            x[i] = z < 0 ? vr : vi;
        }
#pragma unroll
        for (int i = 0; i < CC_TOK; i++) {
            float acc = 0.0f;
#pragma unroll
            for (uint32_t jj = 0; jj < 3; jj++)
                if (jj < keep) acc = fmaf(w[jj], x[3 + i - keep + jj], acc);
            const float wcur = keep == 0 ? w[0] : keep == 1 ? w[1] : keep == 2 ? w[2] : w[3];
            acc = fmaf(wcur, x[3 + i], acc);
            o[i] = z0 + i < ntok ? silu(acc) : 0.0f;
        }
    } else {
#pragma unroll
        for (int i = 0; i < CC_TOK; i++) o[i] = 0.0f;
    }
    if (hw && blockIdx.x * TPB < qk_end) {
        const uint32_t w = threadIdx.x >> 6;
        float ss[CC_TOK];
#pragma unroll
        for (int i = 0; i < CC_TOK; i++) ss[i] = wave_sum(fmaf(o[i], o[i], 0.0f));
        if (hw > 1) {
            if ((threadIdx.x & 63) == 0)
#pragma unroll
                for (int i = 0; i < CC_TOK; i++) red[w][i] = ss[i];
            __syncthreads();
            // block_sum's (r0 + r1) + (r2 + r3) with the other head's waves at zero
            const uint32_t w0 = w & 2;
#pragma unroll
            for (int i = 0; i < CC_TOK; i++) ss[i] = red[w0][i] + red[w0 + 1][i];
        }
        if (ch < qk_end) {
            const float dk = (float)(64 * hw);
            const float sc = ch < qk_end / 2 ? 1.0f / dk : 1.0f / sqrtf(dk);
#pragma unroll
            for (int i = 0; i < CC_TOK; i++) {
                const float r = 1.0f / sqrtf(ss[i] / dk + 1e-6f);
                o[i] = (o[i] * r) * sc;
            }
        }
    }
    if (live)
#pragma unroll
        for (int i = 0; i < CC_TOK; i++)
            if (z0 + i < ntok) out[(size_t)(z0 + i) * cd + ch] = o[i];
}

// The ring after a chunk: slot p % 4 = input of position p for the chunk's
// last min(ntok, 4) positions (older slots keep their values).
__global__ void k_conv_ring(const float *in, uint32_t in_stride, float *ring, const sgk_step *steps,
                            uint32_t ntok, uint32_t cd) {
    const uint32_t ch = blockIdx.x * TPB + threadIdx.x;
    if (ch >= cd) return;
    const uint32_t pos0 = steps[0].pos;
    for (uint32_t z = ntok > 4 ? ntok - 4 : 0; z < ntok; z++)
        ring[(size_t)((pos0 + z) & 3) * cd + ch] = in[(size_t)z * in_stride + ch];
}

// q and k of every key head of every token: RMS (eps 1e-6, no weight), then
// q / dk and k / sqrt(dk), in place. Workgroup (head slice, token).
__global__ void __launch_bounds__(TPB) k_qk_norm_chunk(float *conv_out, uint32_t cd, uint32_t n_k, uint32_t dk) {
    __shared__ float red[4];
    const uint32_t b = blockIdx.x, z = blockIdx.y, t = threadIdx.x;
    const bool isq = b < n_k;
    float *x = conv_out + (size_t)z * cd + (isq ? (size_t)b * dk : (size_t)n_k * dk + (size_t)(b - n_k) * dk);
    float v = 0.0f;
    for (uint32_t i = t; i < dk; i += TPB) v = fmaf(x[i], x[i], v);
    const float ss = block_sum(v, red);
    const float r = 1.0f / sqrtf(ss / (float)dk + 1e-6f);
    const float sc = isq ? 1.0f / (float)dk : 1.0f / sqrtf((float)dk);
    for (uint32_t i = t; i < dk; i += TPB) x[i] = (x[i] * r) * sc;
}

// Delta-rule scan: workgroup (value head, 16-row block) keeps its rows of S in
// registers for the whole chunk and walks the tokens in order, writing each
// token's readout y (the decode step's arithmetic; a wave's rows are reduced
// together as in k_gdn_step).
// The tokens' inputs are staged in LDS in blocks of DCT tokens (k | q of the
// key head, the block's 16 v values, beta and decay), double-buffered: the
// next block's global loads are in flight while the current block is walked,
// so a token step reads only LDS.
template <int DK, int ROWS>
struct dcg {
    static constexpr int DCT = 16;                        // tokens per staged block
    static constexpr int TPT = TPB / DCT;                 // threads per token (k|q)
    static constexpr int NV4 = 2 * DK / TPT / 4;          // k|q float4s per thread
    static constexpr int VTT = ROWS / 4;                  // threads per token (v, 4 rows each)
    static_assert(TPB / VTT >= DCT, "v staging covers a block");
};
template <int DK, int ROWS>
using dcregs = f32x4[dcg<DK, ROWS>::NV4 + 1];     // one thread's staged loads of a block

template <int DK, int ROWS>
__device__ __forceinline__ void dc_load(dcregs<DK, ROWS> &r, const sgk_gdn &a, const float *conv_out,
                                        uint32_t z0, uint32_t ntok, uint32_t hk, uint32_t h, uint32_t j0) {
    using C = dcg<DK, ROWS>;
    const uint32_t t = threadIdx.x, zt = t / C::TPT, part = t % C::TPT, key_dim = a.n_k * DK;
    const float *cz = conv_out + (size_t)min(z0 + zt, ntok - 1) * a.conv_dim;
#pragma unroll
    for (int u = 0; u < C::NV4; u++) {
        // float4 u*TPT + part of the token's k|q: consecutive threads take
        // consecutive float4s (coalesced loads, LDS stores free of bank conflicts)
        const uint32_t e = (u * C::TPT + part) * 4;          // 0 .. 2*DK-1: k, then q
        const float *src = e < DK ? cz + key_dim + (size_t)hk * DK + e : cz + (size_t)hk * DK + (e - DK);
        r[u] = *(const f32x4 *)src;
    }
    // v: token t/VTT, rows j0 + 4*(t%VTT) .. +3
    const uint32_t vz = t / C::VTT, vr = j0 + (t % C::VTT) * 4;
    const float *vp = conv_out + (size_t)min(z0 + vz, ntok - 1) * a.conv_dim + 2 * key_dim + (size_t)h * a.dv + vr;
    r[C::NV4] = (vz < (uint32_t)C::DCT && vr < a.dv) ? *(const f32x4 *)vp : (f32x4){0.f, 0.f, 0.f, 0.f};
}

template <int DK, int ROWS>
__device__ __forceinline__ void dc_store(const dcregs<DK, ROWS> &r, float *kq, float *vs, float *gs,
                                         const sgk_gdn &a, const float *gates, uint32_t in_stride, uint32_t z0,
                                         uint32_t ntok, uint32_t h) {
    using C = dcg<DK, ROWS>;
    const uint32_t t = threadIdx.x, zt = t / C::TPT, part = t % C::TPT;
#pragma unroll
    for (int u = 0; u < C::NV4; u++) *(f32x4 *)&kq[zt * 2 * DK + (u * C::TPT + part) * 4] = r[u];
    const uint32_t vz = t / C::VTT;
    if (vz < (uint32_t)C::DCT) *(f32x4 *)&vs[vz * ROWS + (t % C::VTT) * 4] = r[C::NV4];
    if (t < (uint32_t)C::DCT) {
        const uint32_t z = min(z0 + t, ntok - 1), cd = a.conv_dim, vd = a.n_v * a.dv;
        float beta, decay;
        if (gates) {
            beta = gates[(size_t)z * 2 * a.n_v + h];
            decay = gates[(size_t)z * 2 * a.n_v + a.n_v + h];
        } else {
            const float *iz = a.in + (size_t)z * in_stride;
            gdn_gates(iz[cd + vd + h], iz[cd + vd + a.n_v + h], a.ssm_a[h], a.dt_bias[h], a.neg_exp, &beta, &decay);
        }
        gs[2 * t] = beta;
        gs[2 * t + 1] = decay;
    }
}

template <int DK, int ROWS>
__global__ void __launch_bounds__(TPB) k_delta_chunk(sgk_gdn a, const float *conv_out, uint32_t in_stride,
                                                     uint32_t ntok, const float *gates) {
    using C = dcg<DK, ROWS>;
    constexpr int EPL = drow<DK>::EPL, RPW = ROWS / (TPB / 64);
    __shared__ __align__(16) float kq[2][C::DCT * 2 * DK];
    __shared__ __align__(16) float vs[2][C::DCT * ROWS];
    __shared__ float gs[2][2 * C::DCT];
    const uint32_t h = blockIdx.x, j0 = blockIdx.y * ROWS, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t dv = a.dv, vd = a.n_v * dv;
    const uint32_t hk = a.tiled ? h % a.n_k : h / (a.n_v / a.n_k);
    float *Sh = a.S + (size_t)h * dv * DK;
    const bool on = DK >= 64 || lane < (uint32_t)DK;
    float sr[RPW][EPL];
#pragma unroll
    for (int u = 0; u < RPW; u++) {
        const uint32_t j = j0 + wave + u * (TPB / 64);
#pragma unroll
        for (int e = 0; e < EPL; e++) sr[u][e] = 0.0f;
        if (j < dv) row_load<DK>(sr[u], Sh + (size_t)j * DK, lane);
    }
    f32x4 r[C::NV4 + 1];
    dc_load<DK, ROWS>(r, a, conv_out, 0, ntok, hk, h, j0);
    dc_store<DK, ROWS>(r, kq[0], vs[0], gs[0], a, gates, in_stride, 0, ntok, h);
    __syncthreads();
    for (uint32_t z0 = 0; z0 < ntok; z0 += C::DCT) {
        const uint32_t buf = (z0 / C::DCT) & 1;
        dc_load<DK, ROWS>(r, a, conv_out, z0 + C::DCT, ntok, hk, h, j0);    // past the end: clamped, unused
        const uint32_t zn = min((uint32_t)C::DCT, ntok - z0);
        for (uint32_t zz = 0; zz < zn; zz++) {
            // delta_update for the wave's RPW rows at once: both dot products
            // of all rows reduced together (rows_sum), the deltas broadcast
            const float beta = gs[buf][2 * zz], decay = gs[buf][2 * zz + 1];
            const float *kz = &kq[buf][zz * 2 * DK];
            float k[EPL], q[EPL], part[RPW];
#pragma unroll
            for (int e = 0; e < EPL; e++) {
                k[e] = on ? kz[lane * EPL + e] : 0.0f;
                q[e] = on ? kz[DK + lane * EPL + e] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < RPW; u++) {
                float kv = 0.0f;
#pragma unroll
                for (int e = 0; e < EPL; e++) { sr[u][e] *= decay; kv = fmaf(sr[u][e], k[e], kv); }
                part[u] = kv;
            }
            const uint32_t myrow = rows_row<RPW>(lane), jr = wave + myrow * (TPB / 64);
            const float kvr = rows_sum<RPW>(part, lane);
            const float dmine = (vs[buf][zz * ROWS + jr] - kvr) * beta;
#pragma unroll
            for (int u = 0; u < RPW; u++) {
                const float dr = lane_read(dmine, rows_lane<RPW>(u));
                float y = 0.0f;
#pragma unroll
                for (int e = 0; e < EPL; e++) { sr[u][e] = fmaf(k[e], dr, sr[u][e]); y = fmaf(sr[u][e], q[e], y); }
                part[u] = y;
            }
            const float yr = rows_sum<RPW>(part, lane);
            if ((lane & (64 / RPW - 1)) == 0 && j0 + jr < dv) a.y[(size_t)(z0 + zz) * vd + (size_t)h * dv + j0 + jr] = yr;
        }
        dc_store<DK, ROWS>(r, kq[buf ^ 1], vs[buf ^ 1], gs[buf ^ 1], a, gates, in_stride, z0 + C::DCT, ntok, h);
        __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < RPW; u++) {
        const uint32_t j = j0 + wave + u * (TPB / 64);
        if (j < dv) row_store<DK>(sr[u], Sh + (size_t)j * DK, lane);
    }
}

// silu(z) * rmsnorm(y, w) per (value head, token), one wave each, with the
// GEMV gated prologue's arithmetic.
__global__ void k_rmsnorm_gated_rows(const float *y, const float *zsrc, uint32_t z_stride, const float *w,
                                     float *out, uint32_t dv, uint32_t n_v, float eps) {
    const uint32_t lane = threadIdx.x & 63, h = blockIdx.x * (TPB / 64) + (threadIdx.x >> 6), z = blockIdx.y;
    if (h >= n_v) return;
    const float *yh = y + (size_t)z * n_v * dv + (size_t)h * dv;
    const float *zh = zsrc + (size_t)z * z_stride + (size_t)h * dv;
    float *oh = out + (size_t)z * n_v * dv + (size_t)h * dv;
    float ss = 0.0f;
    for (uint32_t j = lane; j < dv; j += 64) ss = fmaf(yh[j], yh[j], ss);
    ss = wave_sum(ss);
    const float r = 1.0f / sqrtf(ss / (float)dv + eps);
    for (uint32_t j = lane; j < dv; j += 64) oh[j] = silu(zh[j]) * ((yh[j] * r) * w[j]);
}

__global__ void k_embed_rows(const int8_t *qs, const uint16_t *d, const float *wf, uint32_t hidden,
                             const sgk_step *steps, float *X) {
    const uint32_t i = blockIdx.x * TPB + threadIdx.x, z = blockIdx.y;
    if (i >= hidden) return;
    const uint64_t t = (uint64_t)(uint32_t)steps[z].token;
    float *x = X + (size_t)z * hidden;
    if (qs) x[i] = h2f(d[t * (hidden >> 5) + (i >> 5)]) * (float)qs[t * hidden + i];
    else x[i] = wf[t * hidden + i];
}

// ---------------------------------------------------------------------------
// Chunked delta rule on the matrix cores: blocks of DM_T = 16 tokens in fp32
// MFMA (v_mfma_f32_16x16x4_f32). With d_t the decay, R_tw = d_{w+1}...d_t
// (R_tt = 1), g_t = d_0...d_t, G = K K^T and H = Q K^T over the block's tokens:
//   T_tw = beta_t R_tw G_tw (w < t),  W' = (I + T)^-1 diag(beta)
//   M_tw = R_tw H_tw (w <= t),        rho_w = R_{15,w}
//   Delta = W' (V - g * (K S^T))      (rows: tokens t, columns: value rows j)
//   Y     = g * (Q S^T) + M Delta
//   S'    = g_15 S + (rho * Delta)^T K
// which is the token loop of ref.c:708-739 (s = decay S; kv = s k; delta =
// (v - kv) beta; S = s + delta k^T; y = S q) unrolled over the block exactly
// in real arithmetic (in fp32 it differs by reassociation), with the decay
// products taken as plain products.
// k_dm_prep computes W', M, g and rho of every (head, block) in parallel, one
// wave each; k_dm_scan walks a head's blocks in order for 16 value rows, with
// the state held in MFMA accumulator layout across the workgroup's 4 waves
// (wave w: key columns [w DK/4, (w+1) DK/4)). Padded tokens of a partial
// block have k = q = v = 0, beta = 0 and decay 1: their Delta rows are zero
// and they leave the state as it is.
// Operand layout of the 16x16x4 f32 MFMA (lane l; r = l % 16, s = l / 16):
//   A[i][k] in lane i + 16 k, B[k][j] in lane j + 16 k,
//   D[i][j] in lane j + 16 (i / 4), element i % 4.
// A product whose right operand X is held in D layout (rows t = 4 s + e in
// lane group s, element e) feeds X's element c as B at reduction step c, the
// reduction index taken as w = 4 s + c; the left operand L then comes as one
// float4 per lane: row r, columns 4 s .. 4 s + 3.
// ---------------------------------------------------------------------------
#define DM_T 16
#define DM_WS (2 * DM_T * DM_T + 2 * DM_T)      // W', M, g, rho per (head, block)
#define DM_KP(D) ((D) + 4)                      // k, q row pitch in LDS
#define DM_SP 20                                // pitch of W', M and V^T in LDS

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <int DK>
__global__ void __launch_bounds__(TPB) k_dm_prep(sgk_gdn a, const float *qkv, uint32_t in_stride, uint32_t ntok,
                                                 const float *gates, float *ws) {
    __shared__ __align__(16) float Tl[TPB / 64][DM_T][DM_T];
    __shared__ float dl[TPB / 64][DM_T], bl[TPB / 64][DM_T];
    const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6, r = lane & 15, s = lane >> 4;
    const uint32_t nblk = (ntok + DM_T - 1) / DM_T, c = blockIdx.x * (TPB / 64) + wv, h = blockIdx.y;
    const bool live = c < nblk;                 // a wave past the last block computes block nblk-1, stores nothing
    const uint32_t cb = live ? c : nblk - 1, z0 = cb * DM_T, n = min((uint32_t)DM_T, ntok - z0);
    const uint32_t hk = a.tiled ? h % a.n_k : h / (a.n_v / a.n_k), key_dim = a.n_k * DK;
    if (s == 0) {                               // decay and beta of token r (1 and 0 past the end)
        float beta = 0.0f, decay = 1.0f;
        if (r < n) {
            const uint32_t z = z0 + r;
            if (gates) {
                beta = gates[(size_t)z * 2 * a.n_v + h];
                decay = gates[(size_t)z * 2 * a.n_v + a.n_v + h];
            } else {
                const float *iz = a.in + (size_t)z * in_stride;
                const uint32_t cd = a.conv_dim, vd = a.n_v * a.dv;
                gdn_gates(iz[cd + vd + h], iz[cd + vd + a.n_v + h], a.ssm_a[h], a.dt_bias[h], a.neg_exp, &beta, &decay);
            }
        }
        dl[wv][r] = decay;
        bl[wv][r] = beta;
    }
    // G = K K^T, H = Q K^T: token r's float4 at key columns 16 u + 4 s is
    // reduction step (u, e) for both operands
    // (four accumulators each, summed at the end: short dependency chains)
    f32x4 Gp[4], Hp[4];
#pragma unroll
    for (int e = 0; e < 4; e++) Gp[e] = Hp[e] = (f32x4){0.f, 0.f, 0.f, 0.f};
    const float *qr = qkv + (size_t)(z0 + min(r, n - 1)) * a.conv_dim + (size_t)hk * DK;
#pragma unroll
    for (int u = 0; u < DK / 16; u++) {
        f32x4 kv = *(const f32x4 *)(qr + key_dim + 16 * u + 4 * s), qv = *(const f32x4 *)(qr + 16 * u + 4 * s);
        if (r >= n) kv = qv = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            Gp[e] = mfma4(kv[e], kv[e], Gp[e]);
            Hp[e] = mfma4(qv[e], kv[e], Hp[e]);
        }
    }
    const f32x4 G = (Gp[0] + Gp[1]) + (Gp[2] + Gp[3]), H = (Hp[0] + Hp[1]) + (Hp[2] + Hp[3]);
    __syncthreads();
    float d[DM_T];
#pragma unroll
    for (int u = 0; u < DM_T; u++) d[u] = dl[wv][u];
    // D layout: column w = r of rows t = 4 s + e
    f32x4 M;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const uint32_t t = 4 * s + e;
        float R = 1.0f;
#pragma unroll
        for (int u = 1; u < DM_T; u++) R = ((uint32_t)u > r && (uint32_t)u <= t) ? R * d[u] : R;
        Tl[wv][t][r] = r < t ? bl[wv][t] * R * G[e] : 0.0f;
        M[e] = r <= t ? R * H[e] : 0.0f;
    }
    __syncthreads();
    // column r of W = (I + T)^-1 by forward substitution: W_t = e_t - sum_{w<t} T_tw W_w
    float Wc[DM_T];
#pragma unroll
    for (int t = 0; t < DM_T; t++) {
        float acc = (uint32_t)t == r ? 1.0f : 0.0f;
#pragma unroll
        for (int u = 0; u < t; u++) acc = fmaf(-Tl[wv][t][u], Wc[u], acc);
        Wc[t] = acc;
    }
    if (!live) return;
    float *o = ws + ((size_t)h * nblk + cb) * DM_WS;
    if (s == 0) {
        const float br = bl[wv][r];
#pragma unroll
        for (int t = 0; t < DM_T; t++) o[t * DM_T + r] = Wc[t] * br;
    }
#pragma unroll
    for (int e = 0; e < 4; e++) o[DM_T * DM_T + (4 * s + e) * DM_T + r] = M[e];
    if (s == 1) {
        float g = 1.0f, rho = 1.0f;
#pragma unroll
        for (int u = 0; u < DM_T; u++) {
            g = (uint32_t)u <= r ? g * d[u] : g;
            rho = (uint32_t)u > r ? rho * d[u] : rho;
        }
        o[2 * DM_T * DM_T + r] = g;
        o[2 * DM_T * DM_T + DM_T + r] = rho;
    }
}

template <int DK>
struct dm_stage {                       // one block's inputs in LDS
    float kq[2][DM_T][DM_KP(DK)];       // k rows, q rows
    float wm[2][DM_T][DM_SP];           // W', M
    float vt[DM_T][DM_SP];              // V^T: [value row][token]
    float gr[2][DM_T];                  // g, rho
};
#define DM_TPB (2 * TPB)                // four MFMA waves and four staging waves
#define DM_NKQ(D) ((D) / 32)            // float4 of k|q per staging lane (16 tokens x D/2 over 256 lanes)
template <int DK>
using dmregs = f32x4[DM_NKQ(DK) + 2];   // a staging lane's share of a block: k|q, then workspace and v

// A staging lane's byte offsets (lane 0..255), the same for every block:
// k|q (row lane / (DK/2), float4 lane % (DK/2); the further rows added per
// load), its float4 of the (head, block) workspace record (lanes below 136)
// and its float4 of v (lanes 136..199: token (lane - 136) / 4, value rows
// j0 + 4 ((lane - 136) % 4) ..). Lanes with no share of a record get an
// offset past the end, and their load returns zeros.
struct dm_src {
    uint32_t kq, ws, v;
};
#define DM_OOB 0x80000000u

template <int DK>
__device__ __forceinline__ dm_src dm_offsets(const sgk_gdn &a, uint32_t hk, uint32_t h, uint32_t j0, uint32_t lane) {
    const uint32_t key_dim = a.n_k * DK, cd4 = a.conv_dim * 4, part = lane % (DK / 2), g = lane - DM_WS / 4;
    dm_src o;
    o.kq = (lane / (DK / 2)) * cd4 + 4 * (part < DK / 4 ? key_dim + hk * DK + 4 * part : hk * DK + 4 * (part - DK / 4));
    o.ws = lane < DM_WS / 4 ? 16 * lane : DM_OOB;
    o.v = lane >= DM_WS / 4 && g < 4 * DM_T ? (g / 4) * cd4 + 4 * (2 * key_dim + h * a.dv + j0 + 4 * (g % 4)) : DM_OOB;
    return o;
}

__device__ __forceinline__ f32x4 dm_ld(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, 0, 0));
}

// Block z0's loads: buffer loads against one descriptor over the block's
// token rows (a row past ntok lies past num_records and reads as zeros: the
// whole offset is in the VGPR operand, which the range check covers) and one
// over its workspace record; one add per load.
template <int DK>
__device__ __forceinline__ void dm_load(dmregs<DK> &x, const sgk_gdn &a, const float *qkv, const float *wsb,
                                        uint32_t z0, uint32_t ntok, const dm_src &o) {
    constexpr uint32_t RPU = 512 / DK;          // token rows per k|q load
    const uint32_t cd4 = a.conv_dim * 4;
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc((void *)(qkv + (size_t)z0 * a.conv_dim), (short)0,
                                                                        (int)(min(ntok - z0, (uint32_t)DM_T) * cd4), 0x00020000);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void *)wsb, (short)0, DM_WS * 4, 0x00020000);
#pragma unroll
    for (int u = 0; u < DM_NKQ(DK); u++) x[u] = dm_ld(rq, o.kq + u * RPU * cd4);
    x[DM_NKQ(DK)] = dm_ld(rw, o.ws);
    x[DM_NKQ(DK) + 1] = dm_ld(rq, o.v);
}

template <int DK>
__device__ __forceinline__ void dm_store(const dmregs<DK> &x, dm_stage<DK> &b, uint32_t lane) {
    constexpr uint32_t RPU = 512 / DK;
    const uint32_t part = lane % (DK / 2), half = part < DK / 4 ? 0 : 1, col = 4 * (part % (DK / 4));
#pragma unroll
    for (int u = 0; u < DM_NKQ(DK); u++) *(f32x4 *)&b.kq[half][u * RPU + lane / (DK / 2)][col] = x[u];
    const f32x4 w = x[DM_NKQ(DK)], v = x[DM_NKQ(DK) + 1];
    if (lane < DM_T * DM_T / 2) {               // W' then M, four float4 per row
        *(f32x4 *)&b.wm[lane / (DM_T * DM_T / 4)][(lane / 4) % DM_T][4 * (lane % 4)] = w;
    } else if (lane < DM_WS / 4) {              // g, rho
        const uint32_t g = lane - DM_T * DM_T / 2;
        *(f32x4 *)&b.gr[g / 4][4 * (g % 4)] = w;
    } else if (lane < DM_WS / 4 + 4 * DM_T) {   // v, transposed
        const uint32_t g = lane - DM_WS / 4, z = g / 4, j = 4 * (g % 4);
        b.vt[j][z] = v[0]; b.vt[j + 1][z] = v[1]; b.vt[j + 2][z] = v[2]; b.vt[j + 3][z] = v[3];
    }
}

// Workgroup: (head, 16 value rows). Waves 0-3 hold the state and do the
// products; waves 4-7 stage the blocks from global memory, so the MFMA waves
// issue no loads and never wait on the memory counter in the loop. One
// barrier per block with two stage buffers and two partial-sum buffers:
// block c is read from sb[c % 2] only before barrier c (the operands of the
// steps after the barrier go to registers first), the staging waves store
// block c + 1 into sb[(c + 1) % 2] between barriers c - 1 and c, and the MFMA
// waves their partial sums into red[c % 2] before barrier c, read after it.
// 58 KB of LDS: two workgroups share a CU (measured on gfx950: at this
// size 4- and 8-wave workgroups fit two per CU, 5- and 6-wave ones only one).
template <int DK>
__global__ void __launch_bounds__(DM_TPB) k_dm_scan(sgk_gdn a, const float *qkv, uint32_t ntok, const float *ws) {
    constexpr int MT = DK / 64;                 // 16-column key tiles per MFMA wave
    __shared__ __align__(16) dm_stage<DK> sb[2];
    __shared__ __align__(16) f32x4 red[2][4][2][64];
    const uint32_t h = blockIdx.x, j0 = blockIdx.y * DM_T, lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint32_t r = lane & 15, s = lane >> 4, dv = a.dv, vd = a.n_v * dv, nblk = (ntok + DM_T - 1) / DM_T;
    const uint32_t hk = a.tiled ? h % a.n_k : h / (a.n_v / a.n_k);
    const float *wsh = ws + (size_t)h * nblk * DM_WS;
    if (wv >= 4) {
        const uint32_t sl = threadIdx.x - TPB;  // staging lane 0..255
        const dm_src o = dm_offsets<DK>(a, hk, h, j0, sl);
        dmregs<DK> x;
        dm_load<DK>(x, a, qkv, wsh, 0, ntok, o);
        dm_store<DK>(x, sb[0], sl);
        if (nblk > 1) dm_load<DK>(x, a, qkv, wsh + DM_WS, DM_T, ntok, o);
        __syncthreads();
        for (uint32_t c = 0; c < nblk; c++) {
            if (c + 1 < nblk) dm_store<DK>(x, sb[(c + 1) & 1], sl);
            __syncthreads();
            if (c + 2 < nblk) dm_load<DK>(x, a, qkv, wsh + (size_t)(c + 2) * DM_WS, (c + 2) * DM_T, ntok, o);
        }
        return;
    }
    float *Sr = a.S + ((size_t)h * dv + j0 + r) * DK;       // this lane's state row j0 + r
    // tile m: key columns 16 (MT wv + m) + 4 s + e of row r (D layout, the key dim as rows)
    f32x4 S[MT];
#pragma unroll
    for (int m = 0; m < MT; m++) S[m] = *(const f32x4 *)(Sr + 16 * (MT * wv + m) + 4 * s);
    __syncthreads();
    for (uint32_t c = 0; c < nblk; c++) {
        const dm_stage<DK> &b = sb[c & 1];
        // this wave's key columns of K S^T and Q S^T (rows t, columns j), one
        // accumulator per tile
        f32x4 pa[MT], pb[MT];
#pragma unroll
        for (int m = 0; m < MT; m++) {
            const uint32_t col = 16 * (MT * wv + m) + 4 * s;
            const f32x4 kv = *(const f32x4 *)&b.kq[0][r][col], qv = *(const f32x4 *)&b.kq[1][r][col];
            pa[m] = pb[m] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                pa[m] = mfma4(kv[e], S[m][e], pa[m]);
                pb[m] = mfma4(qv[e], S[m][e], pb[m]);
            }
        }
        // the block's operands of the steps after the barrier
        f32x4 kt[MT];                           // k rows 4 s + e at key column 16 (MT wv + m) + r
#pragma unroll
        for (int m = 0; m < MT; m++)
#pragma unroll
            for (int e = 0; e < 4; e++) kt[m][e] = b.kq[0][4 * s + e][16 * (MT * wv + m) + r];
        const f32x4 g4 = *(const f32x4 *)&b.gr[0][4 * s], rho4 = *(const f32x4 *)&b.gr[1][4 * s];
        const f32x4 v4 = *(const f32x4 *)&b.vt[r][4 * s], w4 = *(const f32x4 *)&b.wm[0][r][4 * s];
        const f32x4 m4 = *(const f32x4 *)&b.wm[1][r][4 * s];
        const float g15 = b.gr[0][DM_T - 1];
#pragma unroll
        for (int m = 1; m < MT; m++) { pa[0] += pa[m]; pb[0] += pb[m]; }
        red[c & 1][wv][0][lane] = pa[0];
        red[c & 1][wv][1][lane] = pb[0];
        __syncthreads();
        f32x4 A = red[c & 1][0][0][lane];
#pragma unroll
        for (int u = 1; u < 4; u++) A += red[c & 1][u][0][lane];
        f32x4 rhs, D = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 4; e++) rhs[e] = fmaf(-g4[e], A[e], v4[e]);
#pragma unroll
        for (int e = 0; e < 4; e++) D = mfma4(w4[e], rhs[e], D);            // Delta = W' rhs
        // S' = g_15 S + (rho Delta)^T K, each tile with the key dim as rows
        f32x4 Dr;
#pragma unroll
        for (int e = 0; e < 4; e++) Dr[e] = rho4[e] * D[e];
#pragma unroll
        for (int m = 0; m < MT; m++) {
            f32x4 acc = g15 * S[m];
#pragma unroll
            for (int e = 0; e < 4; e++) acc = mfma4(kt[m][e], Dr[e], acc);
            S[m] = acc;
        }
        if (wv == (c & 3)) {                                                // Y = g (Q S^T) + M Delta, waves in turn
            const uint32_t z0 = c * DM_T, n = min((uint32_t)DM_T, ntok - z0);
            f32x4 B = red[c & 1][0][1][lane];
#pragma unroll
            for (int u = 1; u < 4; u++) B += red[c & 1][u][1][lane];
            f32x4 Y;
#pragma unroll
            for (int e = 0; e < 4; e++) Y[e] = g4[e] * B[e];
#pragma unroll
            for (int e = 0; e < 4; e++) Y = mfma4(m4[e], D[e], Y);
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (4 * s + e < n) a.y[(size_t)(z0 + 4 * s + e) * vd + (size_t)h * dv + j0 + r] = Y[e];
        }
    }
#pragma unroll
    for (int m = 0; m < MT; m++) *(f32x4 *)(Sr + 16 * (MT * wv + m) + 4 * s) = S[m];
}

// SURGE_DELTA_SCAN (read per launch) selects the prefill scan: "mfma" (the
// default) the 16-token chunked form on the matrix cores, "seq" the
// sequential token loop. The chunked form needs the workspace, dk 64 or 128
// and dv a multiple of 16; other shapes run the sequential loop. Per
// 512-token call of the 27B layer (48 heads, dk = dv = 128): mfma 51 + 11 us
// (scan + prep), seq 199 us.
enum { SCAN_SEQ, SCAN_MFMA };
// SURGE_DELTA_SCAN: unset, empty or "mfma" (default), or "seq"; any other
// value is refused by the host before a scan launches
// (sgk_delta_scan_env_ok), so an A/B never measures a form it did not name.
static int scan_mode() {
    const char *e = getenv("SURGE_DELTA_SCAN");
    return e && !strcmp(e, "seq") ? SCAN_SEQ : SCAN_MFMA;
}

extern "C" int sgk_delta_scan_env_ok(void) {
    const char *e = getenv("SURGE_DELTA_SCAN");
    return !e || !*e || !strcmp(e, "mfma") || !strcmp(e, "seq");
}

extern "C" uint64_t sgk_delta_ws_floats(uint32_t n_v, uint32_t ntok) {
    return (uint64_t)n_v * ((ntok + DM_T - 1) / DM_T) * DM_WS;
}

extern "C" hipError_t sgk_gdn_chunk(const sgk_gdn *a, float *conv_out, uint32_t in_stride, uint32_t ntok,
                                    float *ws, hipStream_t s) {
    if (!ntok) return hipSuccess;
    if (a->ksize < 1 || a->ksize > 4 || !a->n_k || a->n_v % a->n_k) return hipErrorInvalidValue;
    // q/k norm inside the conv when a head is one or two whole waves; else its own pass
    const uint32_t hw = a->dk == 64 ? 1 : a->dk == 128 ? 2 : 0;
    const uint32_t qk_end = 2 * a->n_k * a->dk;
    if (qk_end > a->conv_dim) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_conv_chunk, dim3((a->conv_dim + TPB - 1) / TPB, (ntok + CC_TOK - 1) / CC_TOK), dim3(TPB), 0, s,
                       a->in, in_stride, a->conv_w, a->ring, conv_out, a->step, ntok, a->conv_dim, a->ksize,
                       hw ? qk_end : 0u, hw);
    hipLaunchKernelGGL(k_conv_ring, dim3((a->conv_dim + TPB - 1) / TPB), dim3(TPB), 0, s, a->in, in_stride, a->ring,
                       a->step, ntok, a->conv_dim);
    if (!hw)
        hipLaunchKernelGGL(k_qk_norm_chunk, dim3(2 * a->n_k, ntok), dim3(TPB), 0, s, conv_out, a->conv_dim, a->n_k,
                           a->dk);
    return sgk_delta_scan(a, conv_out, in_stride, ntok, NULL, ws, s);
}

extern "C" hipError_t sgk_delta_scan(const sgk_gdn *a, const float *qkv, uint32_t in_stride, uint32_t ntok,
                                     const float *gates, float *ws, hipStream_t s) {
    if (!ntok || !a->n_v || !a->dv) return hipSuccess;
    const int mode = ws && (a->dk == 64 || a->dk == 128) ? scan_mode() : SCAN_SEQ;
    if (mode == SCAN_MFMA && a->dv % DM_T == 0) {
        // W', M, g, rho of every (head, 16-token block), then each head's
        // blocks in order per 16 value rows
        const uint32_t nblk = (ntok + DM_T - 1) / DM_T;
#define DML(D) do {                                                                                                   \
            hipLaunchKernelGGL((k_dm_prep<D>), dim3((nblk + TPB / 64 - 1) / (TPB / 64), a->n_v), dim3(TPB), 0, s, *a, qkv, \
                               in_stride, ntok, gates, ws);                                                          \
            hipLaunchKernelGGL((k_dm_scan<D>), dim3(a->n_v, a->dv / DM_T), dim3(DM_TPB), 0, s, *a, qkv, ntok, ws); } while (0)
        if (a->dk == 64) DML(64); else DML(128);
#undef DML
        return hipGetLastError();
    }
    // 8 value rows per workgroup (16-token staged blocks: 33 KB of LDS at
    // dk 128, so three workgroups share a CU and hide each other's serial
    // reduction chains); 16 rows at dk 256 (its blocks take 64 KB)
#define DSCAN(D, R) hipLaunchKernelGGL((k_delta_chunk<D, R>), dim3(a->n_v, (a->dv + (R) - 1) / (R)), dim3(TPB), 0, s, \
                                       *a, qkv, in_stride, ntok, gates)
    switch (a->dk) {
    case 32: DSCAN(32, 8); break;
    case 64: DSCAN(64, 8); break;
    case 128: DSCAN(128, 8); break;
    case 256: DSCAN(256, 16); break;
    default: return hipErrorInvalidValue;
    }
#undef DSCAN
    return hipGetLastError();
}

// Conv over a chunk with the reference's oldest-first state [ksize-1][ch]
// (in and out), no activation: the per-op hook (kernels.metal:1111-1141).
__global__ void k_conv1d_chunk_state(const float *x, const float *w, float *out, float *state, uint32_t ch,
                                     uint32_t ksize, uint32_t ntok) {
    const uint32_t c = blockIdx.x * TPB + threadIdx.x;
    if (c >= ch) return;
    const uint32_t keep = ksize - 1;
    float st[3] = {0.f, 0.f, 0.f};
    for (uint32_t j = 0; j < keep; j++) st[j] = state[(size_t)j * ch + c];
    const float *wc = w + (size_t)c * ksize;
    for (uint32_t z = 0; z < ntok; z++) {
        const float cur = x[(size_t)z * ch + c];
        float acc = 0.0f;
        for (uint32_t j = 0; j < keep; j++) acc = fmaf(wc[j], st[j], acc);
        acc = fmaf(wc[keep], cur, acc);
        for (uint32_t j = 0; j + 1 < keep; j++) st[j] = st[j + 1];
        if (keep) st[keep - 1] = cur;
        out[(size_t)z * ch + c] = acc;
    }
    for (uint32_t j = 0; j < keep; j++) state[(size_t)j * ch + c] = st[j];
}

extern "C" hipError_t sgk_conv1d_chunk(const float *x, const float *w, float *out, float *state, uint32_t ch,
                                       uint32_t ksize, uint32_t ntok, hipStream_t s) {
    if (!ch || !ntok) return hipSuccess;
    if (ksize < 1 || ksize > 4) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_conv1d_chunk_state, dim3((ch + TPB - 1) / TPB), dim3(TPB), 0, s, x, w, out, state, ch,
                       ksize, ntok);
    return hipGetLastError();
}

// beta/decay for every (token, head): gates[z] = beta[n] | decay[n]
// (kernels.metal:1154-1172); adt = ssm_a[n] | dt_bias[n].
__global__ void k_delta_gates_chunk(const float *av, const float *bv, float *gates, const float *adt, uint32_t n,
                                    int neg_exp, uint32_t ntok) {
    const uint32_t i = blockIdx.x * TPB + threadIdx.x;
    if (i >= n * ntok) return;
    const uint32_t z = i / n, h = i % n;
    float beta, decay;
    gdn_gates(bv[i], av[i], adt[h], adt[n + h], neg_exp, &beta, &decay);
    gates[(size_t)z * 2 * n + h] = beta;
    gates[(size_t)z * 2 * n + n + h] = decay;
}

extern "C" hipError_t sgk_delta_gates_chunk(const float *a, const float *b, float *gates, const float *adt,
                                            uint32_t n, int neg_exp, uint32_t ntok, hipStream_t s) {
    if (!n || !ntok) return hipSuccess;
    hipLaunchKernelGGL(k_delta_gates_chunk, dim3((n * ntok + TPB - 1) / TPB), dim3(TPB), 0, s, a, b, gates, adt,
                       n, neg_exp, ntok);
    return hipGetLastError();
}

extern "C" hipError_t sgk_rmsnorm_gated_rows(const float *y, const float *z, uint32_t z_stride, const float *w,
                                             float *out, uint32_t dv, uint32_t n_v, uint32_t ntok, float eps,
                                             hipStream_t s) {
    if (!ntok || !n_v) return hipSuccess;
    hipLaunchKernelGGL(k_rmsnorm_gated_rows, dim3((n_v + 3) / 4, ntok), dim3(TPB), 0, s, y, z, z_stride, w, out,
                       dv, n_v, eps);
    return hipGetLastError();
}

extern "C" hipError_t sgk_embed_rows(const int8_t *qs, const uint16_t *d, const float *wf, uint32_t hidden,
                                     const sgk_step *steps, uint32_t ntok, float *X, hipStream_t s) {
    if (!ntok) return hipSuccess;
    hipLaunchKernelGGL(k_embed_rows, dim3((hidden + TPB - 1) / TPB, ntok), dim3(TPB), 0, s, qs, d, wf, hidden,
                       steps, X);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Argmax (greedy.c:17-27): lowest index wins an exact tie. Two passes:
// per-workgroup winners into `part`, then one workgroup folds them.
// ---------------------------------------------------------------------------

__device__ __forceinline__ void better(float &bv, uint32_t &bi, float v, uint32_t i) {
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}

__global__ void __launch_bounds__(TPB) k_argmax(const float *v, uint32_t n, uint32_t *part,
                                                uint32_t *out, int final_pass) {
    __shared__ float sv[TPB];
    __shared__ uint32_t si[TPB];
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    if (!final_pass) {
        for (uint32_t i = blockIdx.x * TPB + threadIdx.x; i < n; i += gridDim.x * TPB) better(bv, bi, v[i], i);
    } else {
        for (uint32_t k = threadIdx.x; k < n; k += TPB) {
            const uint32_t i = part[k];
            if (i != 0xFFFFFFFFu) better(bv, bi, v[i], i);
        }
    }
    sv[threadIdx.x] = bv;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (uint32_t o = TPB / 2; o >= 1; o >>= 1) {
        if (threadIdx.x < o) {
            float b2 = sv[threadIdx.x];
            uint32_t i2 = si[threadIdx.x];
            better(b2, i2, sv[threadIdx.x + o], si[threadIdx.x + o]);
            sv[threadIdx.x] = b2;
            si[threadIdx.x] = i2;
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        // sg_argmax_f32 scans upward from v[0] with a strict '>': a NaN at
        // index 0 is never beaten (index 0), NaNs elsewhere never win, and an
        // all-NaN or all -inf vector gives 0
        const float v0 = v[0];
        if (final_pass) *out = (si[0] == 0xFFFFFFFFu || v0 != v0) ? 0u : si[0];
        else part[blockIdx.x] = si[0];
    }
}

extern "C" hipError_t sgk_argmax(const float *v, uint32_t n, uint32_t *out, uint32_t *part,
                                 hipStream_t s) {
    const uint32_t blocks = 256;
    hipLaunchKernelGGL(k_argmax, dim3(blocks), dim3(TPB), 0, s, v, n, part, out, 0);
    hipLaunchKernelGGL(k_argmax, dim3(1), dim3(TPB), 0, s, v, blocks, part, out, 1);
    return hipGetLastError();
}

__global__ void k_step_advance(sgk_step *step, uint32_t *hist) {
    const uint32_t pos = step->pos;
    hist[pos + 1] = (uint32_t)step->token;
    step->pos = pos + 1;
}

extern "C" hipError_t sgk_step_advance(sgk_step *step, uint32_t *hist, hipStream_t s) {
    hipLaunchKernelGGL(k_step_advance, dim3(1), dim3(1), 0, s, step, hist);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Prefill GEMM Y[N][M] = X[N][K] * W[M][K]^T (chunk of N tokens through one
// weight), W in the Q8 device layout, on MFMA.
//
// Precision: x is split once per GEMM into bf16 hi + lo (k_split_bf16; x =
// hi + lo to ~2^-18). An int8 weight q is exact in bf16, so a Q8_0 block
// (32 columns: one K step of v_mfma_f32_16x16x32_bf16) of a weight row costs
// two MFMAs, xh*q then xl*q into one fp32 partial started at zero, and the
// row's block scale d is applied to that partial on the VALU:
// acc = fma(d, partial, acc). Against the dequantised form (w = d*q split
// into bf16 hi + lo, three MFMAs: xh*wh + xh*wl + xl*wh) this is a third
// fewer MFMAs, a third less LDS per weight tile (q in bf16 instead of w's hi
// and lo), no dequantisation, and no dropped xl*wl term.
//
// Tiling: workgroup 256 threads = 4 waves over a 128-token x 128-row tile
// (waves 2 x 2, each 64 x 64 = 4 x 4 MFMA tiles of 16x16), K in steps of one
// Q8_0 block (32). Per step the X hi|lo tile, the W tile (q as bf16) and the
// tile rows' block scales are double-buffered in LDS: X is requested one step ahead,
// the raw weights two steps ahead (two register sets), and the next step's
// tiles are stored after the current step's MFMAs, one barrier per step.
// XCD-aware order: workgroup b runs on XCD b % 8, which owns weight tiles
// xcd, xcd+8, ...; on each XCD the token tile is the slow index. Every load
// is unconditional at a clamped index (rows past N or M are computed and
// dropped at the store).
// MFMA 16x16x32 operand layout: A[i][k] in lane i + 16*(k/8), element k%8;
// B[k][j] in lane j + 16*(k/8); D[i][j] in lane j + 16*(i/4), element i%4.
// ---------------------------------------------------------------------------

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// X [N][ldx] f32 -> bf16 hi and lo = x - hi (both round-to-nearest-even),
// laid out per Q8_0 block: the 64 bf16 of block b of token n, hi (32) then lo
// (32), at xs + (b*N + n)*64, so a K step of the GEMM reads one contiguous
// 128-byte line per token (K % 32 == 0, ldx % 4 == 0, X 16-byte aligned).
__device__ __forceinline__ size_t xs_at(uint32_t N, uint32_t n, uint32_t k) {
    return ((size_t)(k >> 5) * N + n) * 64 + (k & 31);
}
// one value of X into the split: hi = bf16(v), lo = bf16(v - hi), as k_split_bf16 rounds them
__device__ __forceinline__ void xs_put(uint16_t *xs, uint32_t N, uint32_t n, uint32_t k, float v) {
    const __bf16 hi = (__bf16)v, lo = (__bf16)(v - (float)hi);
    uint16_t *o = xs + xs_at(N, n, k);
    o[0] = __builtin_bit_cast(uint16_t, hi);
    o[32] = __builtin_bit_cast(uint16_t, lo);
}
__global__ void __launch_bounds__(TPB) k_split_bf16(const float *X, uint32_t ldx, uint32_t N, uint32_t K,
                                                    uint16_t *xs) {
    const uint32_t k4 = K >> 2;
    const size_t total = (size_t)N * k4;
    for (size_t i = (size_t)blockIdx.x * TPB + threadIdx.x; i < total; i += (size_t)gridDim.x * TPB) {
        const uint32_t n = (uint32_t)(i / k4), c = (uint32_t)(i - (size_t)n * k4) * 4;
        const float4 v = *(const float4 *)(X + (size_t)n * ldx + c);
        const bf16x2 h01 = {(__bf16)v.x, (__bf16)v.y}, h23 = {(__bf16)v.z, (__bf16)v.w};
        const bf16x2 l01 = {(__bf16)(v.x - (float)h01[0]), (__bf16)(v.y - (float)h01[1])};
        const bf16x2 l23 = {(__bf16)(v.z - (float)h23[0]), (__bf16)(v.w - (float)h23[1])};
        uint16_t *o = xs + xs_at(N, n, c);
        *(uint2 *)o = make_uint2(__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23));
        *(uint2 *)(o + 32) = make_uint2(__builtin_bit_cast(uint32_t, l01), __builtin_bit_cast(uint32_t, l23));
    }
}

// k_rmsnorm_gated_rows' arithmetic (one wave per (value head, token)) with
// its output written straight as the next product's bf16 hi | lo split, with
// k_split_bf16's rounding, at xs_at(N, z, h*dv + j) ((n_v*dv) % 32 == 0).
__global__ void k_rmsnorm_gated_split(const float *y, const float *zsrc, uint32_t z_stride, const float *w,
                                      uint16_t *xs, uint32_t N, uint32_t dv, uint32_t n_v, float eps) {
    const uint32_t lane = threadIdx.x & 63, h = blockIdx.x * (TPB / 64) + (threadIdx.x >> 6), z = blockIdx.y;
    if (h >= n_v) return;
    const float *yh = y + (size_t)z * n_v * dv + (size_t)h * dv;
    const float *zh = zsrc + (size_t)z * z_stride + (size_t)h * dv;
    float ss = 0.0f;
    for (uint32_t j = lane; j < dv; j += 64) ss = fmaf(yh[j], yh[j], ss);
    ss = wave_sum(ss);
    const float r = 1.0f / sqrtf(ss / (float)dv + eps);
    for (uint32_t j = lane; j < dv; j += 64) {
        const float v = silu(zh[j]) * ((yh[j] * r) * w[j]);
        const __bf16 hi = (__bf16)v, lo = (__bf16)(v - (float)hi);
        uint16_t *o = xs + xs_at(N, z, h * dv + j);
        o[0] = __builtin_bit_cast(uint16_t, hi);
        o[32] = __builtin_bit_cast(uint16_t, lo);
    }
}

extern "C" hipError_t sgk_rmsnorm_gated_split(const float *y, const float *z, uint32_t z_stride, const float *w,
                                              uint16_t *xs, uint32_t dv, uint32_t n_v, uint32_t ntok, float eps,
                                              hipStream_t s) {
    if (!ntok || !n_v) return hipSuccess;
    if (((uint64_t)n_v * dv) % 32 || ((uintptr_t)xs & 15)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_rmsnorm_gated_split, dim3((n_v + 3) / 4, ntok), dim3(TPB), 0, s, y, z, z_stride, w, xs, ntok,
                       dv, n_v, eps);
    return hipGetLastError();
}

// RMSNorm fused into the split: one workgroup per row n, the row's factor
// r = 1/sqrt(mean(x^2) + eps) with k_rmsnorm_heads' arithmetic (the same
// per-thread order and block_sum, then (x*r)*w), so the hi | lo it writes are
// those of the split of k_rmsnorm_heads' output.
__global__ void __launch_bounds__(TPB) k_split_bf16_rms(const float *X, uint32_t ldx, uint32_t N, uint32_t K,
                                                        const float *w, float eps, uint16_t *xs) {
    __shared__ float red[4];
    const uint32_t n = blockIdx.x, t = threadIdx.x;
    const float *xr = X + (size_t)n * ldx;
    float ss = 0.0f;
    for (uint32_t i = t; i < K; i += TPB) { const float v = xr[i]; ss = fmaf(v, v, ss); }
    ss = block_sum(ss, red);
    const float r = 1.0f / sqrtf(ss / (float)K + eps);
    // the split itself four columns at a time (K % 32 == 0, rows 16-byte aligned)
    for (uint32_t i = 4 * t; i < K; i += 4 * TPB) {
        const float4 x4 = *(const float4 *)(xr + i);
        float v[4] = {x4.x * r, x4.y * r, x4.z * r, x4.w * r};
        if (w) {
            const float4 w4 = *(const float4 *)(w + i);
            v[0] *= w4.x; v[1] *= w4.y; v[2] *= w4.z; v[3] *= w4.w;
        }
        const bf16x2 h01 = {(__bf16)v[0], (__bf16)v[1]}, h23 = {(__bf16)v[2], (__bf16)v[3]};
        const bf16x2 l01 = {(__bf16)(v[0] - (float)h01[0]), (__bf16)(v[1] - (float)h01[1])};
        const bf16x2 l23 = {(__bf16)(v[2] - (float)h23[0]), (__bf16)(v[3] - (float)h23[1])};
        uint16_t *o = xs + xs_at(N, n, i);
        *(uint2 *)o = make_uint2(__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23));
        *(uint2 *)(o + 32) = make_uint2(__builtin_bit_cast(uint32_t, l01), __builtin_bit_cast(uint32_t, l23));
    }
}

#define GM_TN 128   // tokens per workgroup tile
#define GM_TM 128   // weight rows per workgroup tile
#define GM_LD 32    // LDS row of one 32-wide step (bf16 elements, 64 bytes, unpadded)

// Element offset of 16-byte chunk c (k 8c..8c+7) of LDS tile row `row`: the
// chunk sits at c ^ ((row >> 1) & 3), which keeps both the fragment reads
// (lane: row li, chunk lg) and the staging writes (thread: 32 bytes of one
// row) free of LDS bank conflicts (measured with SQ_LDS_BANK_CONFLICT).
__device__ __forceinline__ uint32_t gm_at(uint32_t row, uint32_t c) {
    return row * GM_LD + ((c ^ ((row >> 1) & 3)) << 3);
}

// 16 int8 weights of one row -> 16 bf16, exact (|q| <= 127 has at most 7
// significant bits, so the f32 of q has a zero low half and its high half is
// the bf16); the first 8 stored at element offset o0 of wq, the last 8 at o1.
__device__ __forceinline__ void gm_stage_q16(v4u q, uint16_t *wq, uint32_t o0, uint32_t o1) {
    uint32_t o[8];
#pragma unroll
    for (int p = 0; p < 8; p++) {
        const uint32_t u = q[p >> 1] >> (16 * (p & 1));
        const float f0 = (float)(int32_t)(int8_t)(u & 0xffu), f1 = (float)(int32_t)(int8_t)((u >> 8) & 0xffu);
        // bf16 pair (element 2p low, 2p+1 high): the high halves of f0 and f1
        o[p] = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
    }
    *(v4u *)(wq + o0) = (v4u){o[0], o[1], o[2], o[3]};
    *(v4u *)(wq + o1) = (v4u){o[4], o[5], o[6], o[7]};
}

// One token tile of a K step: for each of the wave's 4 weight tiles the
// block's partial xh*q + xl*q (two MFMAs from zero), then acc += d * partial
// with the weight row's block scale (lane j holds column j of a tile, so one
// scale per lane and tile). Every kernel of the prefill GEMM calls this per
// (step, token tile) in the same order, so they give the same bits.
__device__ __forceinline__ void gm_tile_step(f32x4 (&acc)[4], const bf16x8 &ah, const bf16x8 &al,
                                             const bf16x8 (&bq)[4], const float (&dv)[4]) {
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    f32x4 p[4];
#pragma unroll
    for (int c = 0; c < 4; c++) p[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bq[c], z, 0, 0, 0);
#pragma unroll
    for (int c = 0; c < 4; c++) p[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bq[c], p[c], 0, 0, 0);
#pragma unroll
    for (int c = 0; c < 4; c++)
#pragma unroll
        for (int e = 0; e < 4; e++) acc[c][e] = fmaf(dv[c], p[c][e], acc[c][e]);
}

// The wave's weight fragments (rows wm*64 + 16c + li) and block scales of
// LDS buffer cb.
__device__ __forceinline__ void gm_wfrag(bf16x8 (&bq)[4], float (&dv)[4], const uint16_t *wq, const float *wd,
                                         uint32_t wm, uint32_t li, uint32_t lg) {
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const uint32_t row = wm * 64 + c * 16 + li;
        bq[c] = *(const bf16x8 *)&wq[gm_at(row, lg)];
        dv[c] = wd[row];
    }
}

// One K step (Q8_0 block s) of the prefill GEMM on LDS buffer cb: request the
// next block's X and, into the register set this step frees, the raw weights
// of block s+2; the MFMAs; then stage block s+1 (X from xr, q and the scale
// from the other register set wn) into buffer cb^1. Blocks at or past kend
// (the end of this workgroup's K range) only request (clamped) and stage;
// their MFMAs are skipped.
__device__ __forceinline__ void gm_step(f32x4 (&acc)[4][4], v4u (&xr)[4], v4u &wself, uint32_t &dself,
                                        const v4u &wnext, const uint32_t &dnext,
                                        uint16_t (&xt)[2][2][GM_TN * GM_LD], uint16_t (&wq)[2][GM_TM * GM_LD],
                                        float (&wd)[2][GM_TM], uint32_t cb, const v4u *xhr, size_t xb,
                                        const v4u *wrow, const uint16_t *dcol, uint32_t dm, uint32_t s, uint32_t kend,
                                        uint32_t so0, uint32_t so1, uint32_t sr, bool sd, uint32_t wn,
                                        uint32_t wm, uint32_t li, uint32_t lg) {
    const uint32_t s1 = min(s + 1, kend - 1), s2 = min(s + 2, kend - 1);
#pragma unroll
    for (int u = 0; u < 2; u++) { xr[u] = xhr[s1 * xb + u]; xr[2 + u] = xhr[s1 * xb + 4 + u]; }
    __builtin_amdgcn_sched_barrier(0);
    wself = wrow[s2 * 2];
    dself = dcol[(size_t)s2 * dm];
    if (s < kend) {
        bf16x8 bq[4];
        float dv[4];
        gm_wfrag(bq, dv, wq[cb], wd[cb], wm, li, lg);
        bf16x8 ah[4], al[4];
#pragma unroll
        for (int a = 0; a < 4; a++) {
            const uint32_t row = wn * 64 + a * 16 + li;
            ah[a] = *(const bf16x8 *)&xt[cb][0][gm_at(row, lg)];
            al[a] = *(const bf16x8 *)&xt[cb][1][gm_at(row, lg)];
        }
#pragma unroll
        for (int a = 0; a < 4; a++) gm_tile_step(acc[a], ah[a], al[a], bq, dv);
    }
    gm_stage_q16(wnext, wq[cb ^ 1], so0, so1);
    if (sd) wd[cb ^ 1][sr] = h2f((uint16_t)dnext);
    *(v4u *)&xt[cb ^ 1][0][so0] = xr[0];
    *(v4u *)&xt[cb ^ 1][0][so1] = xr[1];
    *(v4u *)&xt[cb ^ 1][1][so0] = xr[2];
    *(v4u *)&xt[cb ^ 1][1][so1] = xr[3];
    __syncthreads();
}

// Tile of linear workgroup index b: consecutive indices go to the 8 XCDs in
// turn (XCD b % 8 runs its (b / 8)-th tile). The operand every workgroup
// re-reads is X (hi and lo, 4 bytes per element: a 128-token tile of a
// 5120-wide X is 2.6 MB), so an XCD should work on one token tile at a time
// and keep it in its 4 MB L2 while the weight tiles stream past. With nb
// token tiles dividing 8 (nb = 1, 2, 4, 8), G = 8 / nb XCDs share token tile
// xcd / G and split its row tiles (mt = xcd % G, + G, ...), so each XCD only
// ever reads one token tile's X. Otherwise an XCD walks its row tiles
// (mt = xcd, xcd + 8, ...) for one token tile before the next. gm_per_xcd
// is the tiles per XCD, so the grid is 8 * gm_per_xcd; indices past an XCD's
// last tile are holes.
__host__ __device__ __forceinline__ uint32_t gm_per_xcd(uint32_t mb, uint32_t nb) {
    if (nb <= 8 && 8 % nb == 0) {
        const uint32_t G = 8 / nb;
        return (mb + G - 1) / G;
    }
    return nb * ((mb + 7) / 8);
}
__device__ __forceinline__ bool gm_tile(uint32_t b, uint32_t mb, uint32_t nb, uint32_t &mt, uint32_t &nt) {
    const uint32_t xcd = b & 7, qq = b >> 3;
    if (nb <= 8 && 8 % nb == 0) {
        const uint32_t G = 8 / nb;
        nt = xcd / G;
        mt = xcd % G + G * qq;
        return mt < mb;
    }
    const uint32_t mper = (mb + 7) / 8;
    mt = xcd + 8 * (qq % mper);
    nt = qq / mper;
    return mt < mb && nt < nb;
}

// Split-K: workgroup row blockIdx.y of gridDim.y takes the Q8_0 blocks
// [nblk*y/Y, nblk*(y+1)/Y) and writes at Y + y*ysplit (k_splitk_reduce sums
// the partials in order); one split is the whole K. The tile is that of
// index blockIdx.x + boff. EPI == SGK_EPI_TILE writes the raw sums as one
// 128x128 tile per workgroup at Y + (blockIdx.y*gridDim.x + blockIdx.x)*16384
// (k_tile_reduce finishes them).
template <int EPI>
__global__ void __launch_bounds__(TPB) __attribute__((amdgpu_waves_per_eu(2, 2)))
k_gemm_q8_mfma(const uint16_t *xs, const int8_t *qs, const uint16_t *d, float *Y, uint32_t N, uint32_t M,
               uint32_t K, uint32_t ldy, uint64_t ysplit, uint32_t boff) {
    __shared__ __align__(16) uint16_t xt[2][2][GM_TN * GM_LD];     // [buffer][hi | lo][token][k]
    __shared__ __align__(16) uint16_t wq[2][GM_TM * GM_LD];        // [buffer][row][k]: q as bf16
    __shared__ float wd[2][GM_TM];                                 // [buffer][row]: block scale
    const uint32_t nb = (N + GM_TN - 1) / GM_TN, mb = (M + GM_TM - 1) / GM_TM;
    uint32_t mt_id, nt_id;
    if (!gm_tile(blockIdx.x + boff, mb, nb, mt_id, nt_id)) return;
    const uint32_t n0 = nt_id * GM_TN, m0 = mt_id * GM_TM;
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint32_t wn = wave & 1, wm = wave >> 1;
    const uint32_t li = lane & 15, lg = lane >> 4;
    const uint32_t nblk = K >> 5;
    const uint32_t kb0 = (uint32_t)((uint64_t)nblk * blockIdx.y / gridDim.y);
    const uint32_t kb1 = (uint32_t)((uint64_t)nblk * (blockIdx.y + 1) / gridDim.y);
    Y += (size_t)blockIdx.y * ysplit;
    // staging role: row t/2 of both tiles, k 16*(t%2) .. +15 of each block
    // (LDS chunks 2*(t%2) and 2*(t%2)+1 of the row); the even thread of a row
    // stages its scale
    const uint32_t sr = t >> 1, sk = (t & 1) * 16, so0 = gm_at(sr, sk / 8), so1 = gm_at(sr, sk / 8 + 1);
    const bool sd = !(t & 1);
    // X block s of token n: hi at xhr[s * xb], lo 4 v4u later (xs_at)
    const v4u *xhr = (const v4u *)(xs + (size_t)min(n0 + sr, N - 1) * 64 + sk);
    const size_t xb = (size_t)N * 8;
    const uint32_t wrow_i = min(m0 + sr, M - 1);
    const v4u *wrow = (const v4u *)(qs + (size_t)wrow_i * K + sk);     // block s: wrow[2 s] (16 int8)
    const uint16_t *dcol = d + wrow_i;                                   // block s: dcol[s * M]

    f32x4 acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int c = 0; c < 4; c++) acc[a][c] = (f32x4){0.f, 0.f, 0.f, 0.f};
    v4u xr[4], wA, wB;
    uint32_t dA, dB;
    // prologue: block kb0 staged into buffer 0, block kb0+1's raw weights in B
#pragma unroll
    for (int u = 0; u < 2; u++) { xr[u] = xhr[kb0 * xb + u]; xr[2 + u] = xhr[kb0 * xb + 4 + u]; }
    __builtin_amdgcn_sched_barrier(0);
    wA = wrow[kb0 * 2];
    dA = dcol[(size_t)kb0 * M];
    wB = wrow[min(kb0 + 1, kb1 - 1) * 2];
    dB = dcol[(size_t)min(kb0 + 1, kb1 - 1) * M];
    gm_stage_q16(wA, wq[0], so0, so1);
    if (sd) wd[0][sr] = h2f((uint16_t)dA);
    *(v4u *)&xt[0][0][so0] = xr[0];
    *(v4u *)&xt[0][0][so1] = xr[1];
    *(v4u *)&xt[0][1][so0] = xr[2];
    *(v4u *)&xt[0][1][so1] = xr[3];
    __syncthreads();
    // step s uses buffer s%2; its register set (A for even s) is reloaded with
    // block s+2 while the other set (holding block s+1) is staged
    for (uint32_t s = kb0; s < kb1; s += 2) {
        gm_step(acc, xr, wA, dA, wB, dB, xt, wq, wd, 0, xhr, xb, wrow, dcol, M, s, kb1, so0, so1, sr, sd, wn, wm, li,
                lg);
        gm_step(acc, xr, wB, dB, wA, dA, xt, wq, wd, 1, xhr, xb, wrow, dcol, M, s + 1, kb1, so0, so1, sr, sd, wn, wm,
                li, lg);
    }
    // epilogue: lane holds D[i = 4*lg + e][j = li] of each tile
    float *Yt = Y + ((size_t)blockIdx.y * gridDim.x + blockIdx.x) * (GM_TN * GM_TM);
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t n = n0 + wn * 64 + a * 16 + lg * 4 + e;
                const uint32_t m = m0 + wm * 64 + c * 16 + li;
                const float v = acc[a][c][e];
                if (EPI == SGK_EPI_TILE) {
                    Yt[(n - n0) * GM_TM + (m - m0)] = v;
                } else if (EPI == SGK_EPI_SWIGLU) {
                    const float up = lane_xor1(v);            // column m+1 lives in lane li^1
                    if (!(li & 1) && n < N && m + 1 < M) Y[(size_t)n * ldy + (m >> 1)] = silu(v) * up;
                } else if (EPI == SGK_EPI_SWIGLU_XS) {        // Y is the next product's split
                    const float up = lane_xor1(v);
                    if (!(li & 1) && n < N && m + 1 < M) xs_put((uint16_t *)Y, N, n, m >> 1, silu(v) * up);
                } else if (n < N && m < M) {
                    if (EPI == SGK_EPI_ADD) Y[(size_t)n * ldy + m] += v;
                    else Y[(size_t)n * ldy + m] = v;
                }
            }
}

// Warp-specialised form of k_gemm_q8_mfma: 512-thread workgroups (two per
// CU) and the same 128x128 tile, fragments and per-step arithmetic
// (gm_tile_step), so the same bits. Waves 0-3 (consumers) own the
// accumulators and, in K step s, only read fragments of LDS buffer s%2 and
// issue the MFMAs and scale FMAs; waves 4-7 (producers) meanwhile convert
// block s+1's weights to bf16 and stage them, their scales and its X into
// buffer (s+1)%2. One barrier per step, so one group's MFMAs overlap
// the other's VALU and LDS work on every SIMD. A step is short, so the
// producers keep four register sets: block b's X and raw weights sit in set
// (b - kb0) % 4, both requested three steps before they are staged.
#define GW_TPB 512
#ifndef GW_NS
#define GW_NS 4      // producer register sets: blocks requested GW_NS - 1 steps ahead
#endif
struct gw_set {
    v4u x[4];        // X hi and lo of the thread's chunk in its two token rows
    v4u w;           // 16 raw int8 weights
    uint32_t d;      // block scale
};
// X staging: thread p takes 16-byte chunk p%4 of token rows p/4 and p/4 + 64,
// so a load instruction covers whole 64-byte rows (16 cache lines, not 32)
// (X block blk of the thread's first token at xhr[blk * xb], its lo 4 v4u
// later, the second token r64 v4u on; the scale of block blk at dcol[blk * dm])
__device__ __forceinline__ void gw_request_x(gw_set &st, const v4u *xhr, size_t xb, uint32_t blk, uint32_t r64) {
    const v4u *p = xhr + blk * xb;
    st.x[0] = p[0];
    st.x[1] = p[r64];
    st.x[2] = p[4];
    st.x[3] = p[r64 + 4];
}
__device__ __forceinline__ void gw_request_w(gw_set &st, const v4u *wrow, const uint16_t *dcol, uint32_t dm,
                                             uint32_t blk) {
    st.w = wrow[blk * 2];
    st.d = dcol[(size_t)blk * dm];
}
__device__ __forceinline__ void gw_stage(const gw_set &st, uint16_t (&xt)[2][GM_TN * GM_LD],
                                         uint16_t (&wq)[GM_TM * GM_LD], float (&wd)[GM_TM], uint32_t so0,
                                         uint32_t so1, uint32_t sr, bool sd, uint32_t xo0, uint32_t xo1) {
    gm_stage_q16(st.w, wq, so0, so1);
    if (sd) wd[sr] = h2f((uint16_t)st.d);
    *(v4u *)&xt[0][xo0] = st.x[0];
    *(v4u *)&xt[0][xo1] = st.x[1];
    *(v4u *)&xt[1][xo0] = st.x[2];
    *(v4u *)&xt[1][xo1] = st.x[3];
}
// Producer step s: request X and weights of block s+NS-1 into set rq (free:
// its last block was staged in step s-1), stage block s+1 (set st) into cb^1.
template <int NS>
__device__ __forceinline__ void gw_produce(gw_set &rq, const gw_set &st,
                                           uint16_t (&xt)[2][2][GM_TN * GM_LD], uint16_t (&wq)[2][GM_TM * GM_LD],
                                           float (&wd)[2][GM_TM], uint32_t cb, const v4u *xhr, size_t xb,
                                           const v4u *wrow, const uint16_t *dcol, uint32_t dm, uint32_t s,
                                           uint32_t kend, uint32_t so0, uint32_t so1, uint32_t sr, bool sd,
                                           uint32_t xo0, uint32_t xo1, uint32_t r64) {
    gw_request_x(rq, xhr, xb, min(s + NS - 1, kend - 1), r64);
    gw_request_w(rq, wrow, dcol, dm, min(s + NS - 1, kend - 1));
    __builtin_amdgcn_sched_barrier(0);
    gw_stage(st, xt[cb ^ 1], wq[cb ^ 1], wd[cb ^ 1], so0, so1, sr, sd, xo0, xo1);
    __syncthreads();
}
// Consumer step s: the fragments of buffer cb, the MFMAs and scale FMAs (none
// past kend). X fragments are read one token tile at a time (register room
// for two workgroups per CU).
__device__ __forceinline__ void gw_consume(f32x4 (&acc)[4][4], uint16_t (&xt)[2][2][GM_TN * GM_LD],
                                           uint16_t (&wq)[2][GM_TM * GM_LD], float (&wd)[2][GM_TM], uint32_t cb,
                                           uint32_t s, uint32_t kend, uint32_t wn, uint32_t wm, uint32_t li,
                                           uint32_t lg) {
    if (s < kend) {
        bf16x8 bq[4];
        float dv[4];
        gm_wfrag(bq, dv, wq[cb], wd[cb], wm, li, lg);
#pragma unroll
        for (int a = 0; a < 4; a++) {
            const uint32_t row = wn * 64 + a * 16 + li;
            const bf16x8 ah = *(const bf16x8 *)&xt[cb][0][gm_at(row, lg)];
            const bf16x8 al = *(const bf16x8 *)&xt[cb][1][gm_at(row, lg)];
            gm_tile_step(acc[a], ah, al, bq, dv);
        }
    }
    __syncthreads();
}

template <int EPI, int NS>
__global__ void __launch_bounds__(GW_TPB) __attribute__((amdgpu_waves_per_eu(4, 4)))
k_gemm_q8_ws(const uint16_t *xs, const int8_t *qs, const uint16_t *d, float *Y, uint32_t N, uint32_t M,
             uint32_t K, uint32_t ldy, uint64_t ysplit, uint32_t boff) {
    __shared__ __align__(16) uint16_t xt[2][2][GM_TN * GM_LD];     // [buffer][hi | lo][token][k]
    __shared__ __align__(16) uint16_t wq[2][GM_TM * GM_LD];        // [buffer][row][k]: q as bf16
    __shared__ float wd[2][GM_TM];                                 // [buffer][row]: block scale
    const uint32_t nb = (N + GM_TN - 1) / GM_TN, mb = (M + GM_TM - 1) / GM_TM;
    uint32_t mt_id, nt_id;
    if (!gm_tile(blockIdx.x + boff, mb, nb, mt_id, nt_id)) return;
    const uint32_t n0 = nt_id * GM_TN, m0 = mt_id * GM_TM;
    const uint32_t t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t nblk = K >> 5;
    const uint32_t kb0 = (uint32_t)((uint64_t)nblk * blockIdx.y / gridDim.y);
    const uint32_t kb1 = (uint32_t)((uint64_t)nblk * (blockIdx.y + 1) / gridDim.y);
    // Both roles pass the same barriers: one after the prologue and one per
    // step of the same loop (steps past kb1 only request, clamped, and stage).
    if (wave >= 4) {
        // producer staging roles: weight row p/2, k 16*(p%2) .. +15 of each
        // block (LDS chunks 2*(p%2), +1); X chunk p%4 of token rows p/4, p/4+64
        const uint32_t pt = t - 256, sr = pt >> 1, sk = (pt & 1) * 16;
        const uint32_t so0 = gm_at(sr, sk / 8), so1 = gm_at(sr, sk / 8 + 1);
        const bool sd = !(pt & 1);
        const uint32_t xr0 = pt >> 2, xc = pt & 3;
        const uint32_t xo0 = gm_at(xr0, xc), xo1 = gm_at(xr0 + 64, xc);
        const uint32_t xn0 = min(n0 + xr0, N - 1), xn1 = min(n0 + xr0 + 64, N - 1);
        const v4u *xhr = (const v4u *)(xs + (size_t)xn0 * 64 + xc * 8);
        const size_t xb = (size_t)N * 8;
        const uint32_t r64 = (xn1 - xn0) * 8;                              // token p/4+64, in 16-byte units
        const uint32_t wrow_i = min(m0 + sr, M - 1);
        const v4u *wrow = (const v4u *)(qs + (size_t)wrow_i * K + sk);     // block s: wrow[2 s] (16 int8)
        const uint16_t *dcol = d + wrow_i;
        // prologue: blocks kb0..kb0+NS-2 requested, block kb0 staged into
        // buffer 0; block b then sits in set (b - kb0) % NS. The loop runs
        // 2*NS steps per turn (set and buffer indices static), as does the
        // consumers', so both pass the same barriers.
        gw_set g[NS];
        const uint32_t kl = kb1 - 1;
#pragma unroll
        for (int u = 0; u < NS - 1; u++) {
            gw_request_x(g[u], xhr, xb, min(kb0 + u, kl), r64);
            gw_request_w(g[u], wrow, dcol, M, min(kb0 + u, kl));
        }
        __builtin_amdgcn_sched_barrier(0);
        gw_stage(g[0], xt[0], wq[0], wd[0], so0, so1, sr, sd, xo0, xo1);
        __syncthreads();
        for (uint32_t s = kb0; s < kb1; s += 2 * NS) {
#pragma unroll
            for (int u = 0; u < 2 * NS; u++)
                gw_produce<NS>(g[(u + NS - 1) % NS], g[(u + 1) % NS], xt, wq, wd, u & 1, xhr, xb, wrow, dcol, M,
                               s + u, kb1, so0, so1, sr, sd, xo0, xo1, r64);
        }
        return;
    }
    const uint32_t wn = wave & 1, wm = wave >> 1;
    const uint32_t li = lane & 15, lg = lane >> 4;
    Y += (size_t)blockIdx.y * ysplit;
    f32x4 acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int c = 0; c < 4; c++) acc[a][c] = (f32x4){0.f, 0.f, 0.f, 0.f};
    __syncthreads();
    for (uint32_t s = kb0; s < kb1; s += 2 * NS) {
#pragma unroll
        for (int u = 0; u < 2 * NS; u++) gw_consume(acc, xt, wq, wd, u & 1, s + u, kb1, wn, wm, li, lg);
    }
    // epilogue (consumers): lane holds D[i = 4*lg + e][j = li] of each tile
    float *Yt = Y + ((size_t)blockIdx.y * gridDim.x + blockIdx.x) * (GM_TN * GM_TM);
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t n = n0 + wn * 64 + a * 16 + lg * 4 + e;
                const uint32_t m = m0 + wm * 64 + c * 16 + li;
                const float v = acc[a][c][e];
                if (EPI == SGK_EPI_TILE) {
                    Yt[(n - n0) * GM_TM + (m - m0)] = v;
                } else if (EPI == SGK_EPI_SWIGLU) {
                    const float up = lane_xor1(v);            // column m+1 lives in lane li^1
                    if (!(li & 1) && n < N && m + 1 < M) Y[(size_t)n * ldy + (m >> 1)] = silu(v) * up;
                } else if (EPI == SGK_EPI_SWIGLU_XS) {        // Y is the next product's split
                    const float up = lane_xor1(v);
                    if (!(li & 1) && n < N && m + 1 < M) xs_put((uint16_t *)Y, N, n, m >> 1, silu(v) * up);
                } else if (n < N && m < M) {
                    if (EPI == SGK_EPI_ADD) Y[(size_t)n * ldy + m] += v;
                    else Y[(size_t)n * ldy + m] = v;
                }
            }
}

// Wide form (the default): 512-thread workgroups, one per CU, over a tile of
// 128 tokens x 256 weight rows, so each X tile staged feeds twice the MFMAs
// of the 128-row tile (X, bf16 hi and lo, is the operand every workgroup
// re-reads) and a step's LDS fragment reads per MFMA drop by a third. Waves
// 0-3 (consumers, 256 registers each) own 64 tokens x 128 rows (4 x 8 MFMA
// tiles) and run gm_tile_step's arithmetic per (step, token tile, weight
// tile), so the bits are those of the other forms; waves 4-7 (producers)
// stage block s+1 while the consumers work on block s, from NS register
// sets requested NS-1 steps ahead. Producer thread p stages X as in the
// 128-row form and all 32 weights and the scale of tile row p.
#define GX_TM 256
#ifndef GX_CW
#define GX_CW 8      // consumer waves: 8 (64 x 64 each, 768 threads) or 4 (64 x 128 each, 512 threads)
#endif
struct gx_set {
    v4u x[4];        // X hi and lo of the thread's chunk in its two token rows
    uint32_t d;      // the block scale of the thread's row
};
__device__ __forceinline__ void gx_request(gx_set &st, const v4u *xhr, size_t xb, const uint16_t *dcol, uint32_t dm,
                                           uint32_t blk, uint32_t r64) {
    const v4u *p = xhr + blk * xb;
    st.x[0] = p[0];
    st.x[1] = p[r64];
    st.x[2] = p[4];
    st.x[3] = p[r64 + 4];
    st.d = dcol[(size_t)blk * dm];
}
// The thread's row weights of 4 consecutive blocks (one 128-byte line when
// aligned), requested together: a row's blocks are K bytes apart from the
// next row's, so a request per block would touch every line four times.
__device__ __forceinline__ void gx_request_w4(v4u (&w)[8], const v4u *wrow, uint32_t blk, uint32_t kl) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t b = min(blk + j, kl);
        w[2 * j] = wrow[b * 2];
        w[2 * j + 1] = wrow[b * 2 + 1];
    }
}
__device__ __forceinline__ void gx_stage(const gx_set &st, const v4u &w0, const v4u &w1,
                                         uint16_t (&xt)[2][GM_TN * GM_LD], uint16_t (&wq)[GX_TM * GM_LD],
                                         float (&wd)[GX_TM], uint32_t row, uint32_t xo0, uint32_t xo1) {
    gm_stage_q16(w0, wq, gm_at(row, 0), gm_at(row, 1));
    gm_stage_q16(w1, wq, gm_at(row, 2), gm_at(row, 3));
    wd[row] = h2f((uint16_t)st.d);
    *(v4u *)&xt[0][xo0] = st.x[0];
    *(v4u *)&xt[0][xo1] = st.x[1];
    *(v4u *)&xt[1][xo0] = st.x[2];
    *(v4u *)&xt[1][xo1] = st.x[3];
}
template <int WT>
__device__ __forceinline__ void gx_consume(f32x4 (&acc)[4][WT], uint16_t (&xt)[2][2][GM_TN * GM_LD],
                                           uint16_t (&wq)[2][GX_TM * GM_LD], float (&wd)[2][GX_TM], uint32_t cb,
                                           uint32_t s, uint32_t kend, uint32_t wn, uint32_t wm, uint32_t li,
                                           uint32_t lg) {
    if (s < kend) {
        bf16x8 bq[WT];
        float dv[WT];
#pragma unroll
        for (int c = 0; c < WT; c++) {
            const uint32_t row = wm * (16 * WT) + c * 16 + li;
            bq[c] = *(const bf16x8 *)&wq[cb][gm_at(row, lg)];
            dv[c] = wd[cb][row];
        }
#pragma unroll
        for (int a = 0; a < 4; a++) {
            const uint32_t row = wn * 64 + a * 16 + li;
            const bf16x8 ah = *(const bf16x8 *)&xt[cb][0][gm_at(row, lg)];
            const bf16x8 al = *(const bf16x8 *)&xt[cb][1][gm_at(row, lg)];
#pragma unroll
            for (int h = 0; h < WT / 4; h++) {
                f32x4 (&ac)[4] = *reinterpret_cast<f32x4 (*)[4]>(&acc[a][4 * h]);
                const bf16x8 (&bh)[4] = *reinterpret_cast<const bf16x8 (*)[4]>(&bq[4 * h]);
                const float (&dh)[4] = *reinterpret_cast<const float (*)[4]>(&dv[4 * h]);
                gm_tile_step(ac, ah, al, bh, dh);
            }
        }
    }
    __syncthreads();
}

template <int EPI, int NS, int CW>
__global__ void __launch_bounds__((CW + 4) * 64) __attribute__((amdgpu_waves_per_eu((CW + 4) / 4, (CW + 4) / 4)))
k_gemm_q8_wide(const uint16_t *xs, const int8_t *qs, const uint16_t *d, float *Y, uint32_t N, uint32_t M,
               uint32_t K, uint32_t ldy, uint64_t ysplit, uint32_t boff) {
    __shared__ __align__(16) uint16_t xt[2][2][GM_TN * GM_LD];     // [buffer][hi | lo][token][k]
    __shared__ __align__(16) uint16_t wq[2][GX_TM * GM_LD];        // [buffer][row][k]: q as bf16
    __shared__ float wd[2][GX_TM];                                 // [buffer][row]: block scale
    const uint32_t nb = (N + GM_TN - 1) / GM_TN, mb = (M + GX_TM - 1) / GX_TM;
    uint32_t mt_id, nt_id;
    if (!gm_tile(blockIdx.x + boff, mb, nb, mt_id, nt_id)) return;
    const uint32_t n0 = nt_id * GM_TN, m0 = mt_id * GX_TM;
    const uint32_t t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t nblk = K >> 5;
    const uint32_t kb0 = (uint32_t)((uint64_t)nblk * blockIdx.y / gridDim.y);
    const uint32_t kb1 = (uint32_t)((uint64_t)nblk * (blockIdx.y + 1) / gridDim.y);
    // Both roles pass the same barriers: one after the prologue and one per
    // step, 2*NS steps per turn (steps past kb1 only request, clamped, and stage).
    constexpr int WT = 16 / CW * 2;          // weight tiles (16 rows) per consumer wave
    if (wave >= CW) {
        const uint32_t pt = t - CW * 64;
        const uint32_t xr0 = pt >> 2, xc = pt & 3;
        const uint32_t xo0 = gm_at(xr0, xc), xo1 = gm_at(xr0 + 64, xc);
        const uint32_t xn0 = min(n0 + xr0, N - 1), xn1 = min(n0 + xr0 + 64, N - 1);
        const v4u *xhr = (const v4u *)(xs + (size_t)xn0 * 64 + xc * 8);
        const size_t xb = (size_t)N * 8;
        const uint32_t r64 = (xn1 - xn0) * 8;                              // token p/4+64, in 16-byte units
        const uint32_t wrow_i = min(m0 + pt, M - 1);
        const v4u *wrow = (const v4u *)(qs + (size_t)wrow_i * K);          // block s: wrow[2 s], wrow[2 s + 1]
        const uint16_t *dcol = d + wrow_i;
        // X and the scale per block in NS sets (block b in set (b - kb0) % NS);
        // weights per 4 blocks in two batches (block b in batch ((b - kb0) / 4) % 2,
        // slot (b - kb0) % 4), the next batch requested 4 steps before its first
        // block is staged. A turn is 8 steps, so every index is static.
        static_assert(2 * NS == 8, "wide GEMM producer: a turn of 8 steps holds two weight batches");
        gx_set g[NS];
        v4u wb[2][8];
        const uint32_t kl = kb1 - 1;
        gx_request_w4(wb[0], wrow, kb0, kl);
        gx_request_w4(wb[1], wrow, kb0 + 4, kl);
#pragma unroll
        for (int u = 0; u < NS - 1; u++) gx_request(g[u], xhr, xb, dcol, M, min(kb0 + u, kl), r64);
        __builtin_amdgcn_sched_barrier(0);
        gx_stage(g[0], wb[0][0], wb[0][1], xt[0], wq[0], wd[0], pt, xo0, xo1);
        __syncthreads();
        for (uint32_t s = kb0; s < kb1; s += 2 * NS) {
#pragma unroll
            for (int u = 0; u < 2 * NS; u++) {
                // request block s+u+NS-1 into the set block s+u-1 freed, and
                // after a batch's last block is staged (steps 2 and 6) the
                // batch 8 blocks on into it; stage block s+u+1 into the buffer
                // step s+u does not read
                gx_request(g[(u + NS - 1) % NS], xhr, xb, dcol, M, min(s + u + NS - 1, kl), r64);
                if (u == 3) gx_request_w4(wb[0], wrow, s + 8, kl);
                if (u == 7) gx_request_w4(wb[1], wrow, s + 12, kl);
                __builtin_amdgcn_sched_barrier(0);
                const uint32_t nbuf = (u & 1) ^ 1, b = ((u + 1) >> 2) & 1, j = (u + 1) & 3;
                gx_stage(g[(u + 1) % NS], wb[b][2 * j], wb[b][2 * j + 1], xt[nbuf], wq[nbuf], wd[nbuf], pt, xo0, xo1);
                __syncthreads();
            }
        }
        return;
    }
    const uint32_t wn = wave & 1, wm = wave >> 1;
    const uint32_t li = lane & 15, lg = lane >> 4;
    Y += (size_t)blockIdx.y * ysplit;
    f32x4 acc[4][WT];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int c = 0; c < WT; c++) acc[a][c] = (f32x4){0.f, 0.f, 0.f, 0.f};
    __syncthreads();
    for (uint32_t s = kb0; s < kb1; s += 2 * NS) {
#pragma unroll
        for (int u = 0; u < 2 * NS; u++) gx_consume<WT>(acc, xt, wq, wd, u & 1, s + u, kb1, wn, wm, li, lg);
    }
    // epilogue (consumers): lane holds D[i = 4*lg + e][j = li] of each tile
    float *Yt = Y + ((size_t)blockIdx.y * gridDim.x + blockIdx.x) * (GM_TN * GX_TM);
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int c = 0; c < WT; c++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t n = n0 + wn * 64 + a * 16 + lg * 4 + e;
                const uint32_t m = m0 + wm * (16 * WT) + c * 16 + li;
                const float v = acc[a][c][e];
                if (EPI == SGK_EPI_TILE) {
                    Yt[(n - n0) * GX_TM + (m - m0)] = v;
                } else if (EPI == SGK_EPI_SWIGLU) {
                    const float up = lane_xor1(v);            // column m+1 lives in lane li^1
                    if (!(li & 1) && n < N && m + 1 < M) Y[(size_t)n * ldy + (m >> 1)] = silu(v) * up;
                } else if (EPI == SGK_EPI_SWIGLU_XS) {        // Y is the next product's split
                    const float up = lane_xor1(v);
                    if (!(li & 1) && n < N && m + 1 < M) xs_put((uint16_t *)Y, N, n, m >> 1, silu(v) * up);
                } else if (n < N && m < M) {
                    if (EPI == SGK_EPI_ADD) Y[(size_t)n * ldy + m] += v;
                    else Y[(size_t)n * ldy + m] = v;
                }
            }
}

// Split-K epilogue: the S partials P[s][N][M] summed in order, then the GEMM
// epilogue (store, += residual, SwiGLU on (gate, up) column pairs).
template <int EPI>
__global__ void __launch_bounds__(TPB) k_splitk_reduce(const float *P, uint32_t S, uint32_t N, uint32_t M,
                                                       float *Y, uint32_t ldy) {
    const size_t nm = (size_t)N * M, step = EPI == SGK_EPI_SWIGLU || EPI == SGK_EPI_SWIGLU_XS ? 2 : 1;
    for (size_t i = ((size_t)blockIdx.x * TPB + threadIdx.x) * step; i < nm; i += (size_t)gridDim.x * TPB * step) {
        const uint32_t n = (uint32_t)(i / M), m = (uint32_t)(i - (size_t)n * M);
        float v = P[i];
        for (uint32_t k = 1; k < S; k++) v += P[(size_t)k * nm + i];
        if (EPI == SGK_EPI_SWIGLU || EPI == SGK_EPI_SWIGLU_XS) {
            float u = P[i + 1];
            for (uint32_t k = 1; k < S; k++) u += P[(size_t)k * nm + i + 1];
            if (EPI == SGK_EPI_SWIGLU_XS) xs_put((uint16_t *)Y, N, n, m >> 1, silu(v) * u);
            else Y[(size_t)n * ldy + (m >> 1)] = silu(v) * u;
        } else if (EPI == SGK_EPI_ADD) {
            Y[(size_t)n * ldy + m] += v;
        } else {
            Y[(size_t)n * ldy + m] = v;
        }
    }
}

// The split-K epilogue with += residual fused with the next product's input
// split: workgroup n sums row n's S partials in order into Y (the arithmetic
// of k_splitk_reduce<SGK_EPI_ADD>), then writes the bf16 hi | lo split of
// RMSNorm(Y row n) with weight w (k_split_bf16_rms': the same per-thread order
// of the sum of squares, block_sum, (y * r) * w), so both outputs are those
// of the two kernels run one after the other.
template <int S>
__global__ void __launch_bounds__(TPB) k_splitk_reduce_rms(const float *P, uint32_t N, uint32_t M,
                                                           float *Y, uint32_t ldy, const float *w, float eps,
                                                           uint16_t *xs) {
    __shared__ float red[4];
    const uint32_t n = blockIdx.x, t = threadIdx.x;
    const size_t nm = (size_t)N * M;
    float *yr = Y + (size_t)n * ldy;
    float ss = 0.0f;
    // columns t, t + TPB, ... eight at a time, each with its S partials and
    // residual requested together before any is added (a runtime loop over the
    // splits waited for each split's loads in turn: 15 memory round trips per
    // 5120-column row at S = 3, now 3); the partials are added in split order
    // and the sum of squares runs over the columns in increasing order
    constexpr int U = 8;
    for (uint32_t i0 = t; i0 < M; i0 += U * TPB) {
        float v[S][U], y[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint32_t i = min(i0 + u * TPB, M - 1);
            y[u] = yr[i];
#pragma unroll
            for (int k = 0; k < S; k++) v[k][u] = P[(size_t)k * nm + (size_t)n * M + i];
        }
        __builtin_amdgcn_sched_barrier(0);          // all of them before the first add
#pragma unroll
        for (int u = 0; u < U; u++) {
            float acc = v[0][u];
#pragma unroll
            for (int k = 1; k < S; k++) acc += v[k][u];
            if (i0 + u * TPB < M) {
                y[u] += acc;
                yr[i0 + u * TPB] = y[u];
                ss = fmaf(y[u], y[u], ss);
            }
        }
    }
    ss = block_sum(ss, red);                    // its barriers also publish the row's stores to the workgroup
    const float r = 1.0f / sqrtf(ss / (float)M + eps);
    for (uint32_t i = 4 * t; i < M; i += 4 * TPB) {
        const float4 x4 = *(const float4 *)(yr + i);
        const float4 w4 = *(const float4 *)(w + i);
        const float v[4] = {(x4.x * r) * w4.x, (x4.y * r) * w4.y, (x4.z * r) * w4.z, (x4.w * r) * w4.w};
        const bf16x2 h01 = {(__bf16)v[0], (__bf16)v[1]}, h23 = {(__bf16)v[2], (__bf16)v[3]};
        const bf16x2 l01 = {(__bf16)(v[0] - (float)h01[0]), (__bf16)(v[1] - (float)h01[1])};
        const bf16x2 l23 = {(__bf16)(v[2] - (float)h23[0]), (__bf16)(v[3] - (float)h23[1])};
        uint16_t *o = xs + xs_at(N, n, i);
        *(uint2 *)o = make_uint2(__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23));
        *(uint2 *)(o + 32) = make_uint2(__builtin_bit_cast(uint32_t, l01), __builtin_bit_cast(uint32_t, l23));
    }
}

// Split-K epilogue of the tiles a SGK_EPI_TILE launch computed (tiles of
// GM_TN tokens x TM rows): workgroup (t, part) takes 1/parts of the tile of
// index t + boff, parts = GM_TN*TM / (4*TPB); each thread requests its 4
// columns of all S partial tiles (P + (s*ntile + t)*GM_TN*TM) at once, sums
// them in order, then applies the GEMM epilogue.
#define GM_TR_SMAX 16
template <int TM>
constexpr uint32_t gm_tr_parts() { return GM_TN * TM / (4 * TPB); }
template <int EPI, int TM>
__global__ void __launch_bounds__(TPB) k_tile_reduce(const float *P, uint32_t S, uint32_t ntile, uint32_t boff,
                                                     uint32_t N, uint32_t M, float *Y, uint32_t ldy) {
    static_assert(gm_tr_parts<TM>() * TPB * 4 == GM_TN * TM, "k_tile_reduce covers a tile exactly");
    const uint32_t nb = (N + GM_TN - 1) / GM_TN, mb = (M + TM - 1) / TM;
    uint32_t mt, nt;
    if (!gm_tile(blockIdx.x + boff, mb, nb, mt, nt)) return;
    const uint32_t idx = (blockIdx.y * TPB + threadIdx.x) * 4;       // 4 columns of one token row
    const uint32_t n = nt * GM_TN + idx / TM, m = mt * TM + idx % TM;
    if (n >= N || m >= M) return;
    const float4 *Pt = (const float4 *)(P + (size_t)blockIdx.x * (GM_TN * TM) + idx);
    const size_t sstride = (size_t)ntile * (GM_TN * TM) / 4;
    float4 part[GM_TR_SMAX];
#pragma unroll
    for (uint32_t k = 0; k < GM_TR_SMAX; k++) part[k] = k < S ? Pt[k * sstride] : make_float4(0.f, 0.f, 0.f, 0.f);
    float4 v = part[0];
#pragma unroll
    for (uint32_t k = 1; k < GM_TR_SMAX; k++)
        if (k < S) { v.x += part[k].x; v.y += part[k].y; v.z += part[k].z; v.w += part[k].w; }
    float *y = Y + (size_t)n * ldy;
    if (EPI == SGK_EPI_SWIGLU) {
        // (gate, up) column pairs: m is even, so m+1 and m+3 sit in this float4
        if (m + 1 < M) y[m >> 1] = silu(v.x) * v.y;
        if (m + 3 < M) y[(m >> 1) + 1] = silu(v.z) * v.w;
        return;
    }
    if (EPI == SGK_EPI_SWIGLU_XS) {             // Y is the next product's split
        if (m + 1 < M) xs_put((uint16_t *)Y, N, n, m >> 1, silu(v.x) * v.y);
        if (m + 3 < M) xs_put((uint16_t *)Y, N, n, (m >> 1) + 1, silu(v.z) * v.w);
        return;
    }
    const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
        if (m + e >= M) break;
        if (EPI == SGK_EPI_ADD) y[m + e] += vv[e];
        else y[m + e] = vv[e];
    }
}

// f32-weight GEMM for small test models (VALU, 16x16 outputs per workgroup).
template <int EPI>
__global__ void __launch_bounds__(TPB) k_gemm_f32(const float *X, const float *W, float *Y, uint32_t N,
                                                  uint32_t M, uint32_t K, uint32_t ldx, uint32_t ldy) {
    const uint32_t n = blockIdx.y * 16 + (threadIdx.x >> 4), m = blockIdx.x * 16 + (threadIdx.x & 15);
    float s = 0.f;
    if (n < N && m < M)
        for (uint32_t k = 0; k < K; k++) s = fmaf(X[(size_t)n * ldx + k], W[(size_t)m * K + k], s);
    if (EPI == SGK_EPI_SWIGLU) {
        const float up = __shfl_xor(s, 1, 64);
        if (!(m & 1) && n < N && m + 1 < M) Y[(size_t)n * ldy + (m >> 1)] = silu(s) * up;
    } else if (n < N && m < M) {
        if (EPI == SGK_EPI_ADD) Y[(size_t)n * ldy + m] += s;
        else Y[(size_t)n * ldy + m] = s;
    }
}

extern "C" hipError_t sgk_gemm(const sgk_gemm_args *a, hipStream_t s) {
    if (!a->N || !a->M || !a->K) return hipSuccess;
    if (a->epi == SGK_EPI_SWIGLU && (a->M & 1)) return hipErrorInvalidValue;
    if (a->ys && (a->epi != SGK_EPI_SWIGLU || !a->qs || (a->M / 2) % 32 || a->ys == a->xs)) return hipErrorInvalidValue;
    // the SwiGLU outputs as the next product's split: the launches below take ys for Y
    const int epi = a->ys ? SGK_EPI_SWIGLU_XS : a->epi;
    float *const Yo = a->ys ? (float *)a->ys : a->Y;
    if (a->nw && !a->qs) return hipErrorInvalidValue;      // the fused RMSNorm is part of the Q8 split
    if (a->qs) {
        if (a->K % 32 || !a->xs || !a->dt || a->ldx % 4 || ((uintptr_t)a->X & 15) || ((uintptr_t)a->xs & 15))
            return hipErrorInvalidValue;
        const uint32_t k4 = a->K / 4;
        const uint64_t total = (uint64_t)a->N * k4;
        const uint32_t sg = (uint32_t)min((total + TPB - 1) / TPB, (uint64_t)4096);
        if (a->nw && ((uintptr_t)a->nw & 15)) return hipErrorInvalidValue;
        if (a->post_done) *a->post_done = 0;
        if (a->xs_ready) {
            // the previous product's reduce wrote this split
        } else if (a->nw) {
            hipLaunchKernelGGL(k_split_bf16_rms, dim3(a->N), dim3(TPB), 0, s, a->X, a->ldx, a->N, a->K, a->nw, a->eps, a->xs);
        } else {
            hipLaunchKernelGGL(k_split_bf16, dim3(sg), dim3(TPB), 0, s, a->X, a->ldx, a->N, a->K, a->xs);
        }
        const int kind = gemm_kind();
        const uint32_t TM = kind == GEMM_WIDE ? GX_TM : GM_TM;
        const uint32_t mb = (a->M + TM - 1) / TM, nb = (a->N + GM_TN - 1) / GM_TN;
        const uint32_t grid = 8 * gm_per_xcd(mb, nb), nblk = a->K / 32, tiles = mb * nb;
        // Workgroups run in rounds of `slots` (one or two resident per CU) and
        // every tile takes the same time, so a launch costs ceil(tiles / slots)
        // rounds. Narrow weights (one partial round) split K up to 4 ways to
        // fill the round; wide ones whose last round is under half full run
        // the full rounds as they are and split the leftover tiles' K over a
        // whole round, partial tiles summed in order by k_tile_reduce. Splits
        // keep at least 8 Q8_0 blocks and fit the partials in a->part.
        const uint32_t slots = gemm_slots(kind);
        const uint32_t gtpb = kind == GEMM_PLAIN ? TPB : kind == GEMM_WIDE ? (GX_CW + 4) * 64 : GW_TPB;
#define GL(E, G, Yp, LDY, YS, BOFF)                                                                             \
        do {                                                                                                   \
            if (kind == GEMM_WIDE)                                                                              \
                hipLaunchKernelGGL((k_gemm_q8_wide<E, GW_NS, GX_CW>), G, dim3(gtpb), 0, s, a->xs, a->qs, a->dt, Yp, a->N, \
                                   a->M, a->K, LDY, YS, BOFF);                                                 \
            else if (kind == GEMM_WS)                                                                           \
                hipLaunchKernelGGL((k_gemm_q8_ws<E, GW_NS>), G, dim3(gtpb), 0, s, a->xs, a->qs, a->dt, Yp, a->N,   \
                                   a->M, a->K, LDY, YS, BOFF);                                                 \
            else                                                                                                \
                hipLaunchKernelGGL((k_gemm_q8_mfma<E>), G, dim3(gtpb), 0, s, a->xs, a->qs, a->dt, Yp, a->N, a->M,  \
                                   a->K, LDY, YS, BOFF);                                                       \
        } while (0)
        uint32_t S = 1;
        if (a->part && tiles < slots) {
            S = min(4u, slots / tiles);
            while (S > 1 && (nblk / S < 8 || (uint64_t)S * a->N * a->M > a->part_cap)) S--;
        }
        if (S > 1) {
            GL(SGK_EPI_STORE, dim3(grid, S), a->part, a->M, (uint64_t)a->N * a->M, 0u);
            if (a->epi == SGK_EPI_ADD && a->post_nw && a->post_done && a->ldy % 4 == 0 && a->M % 32 == 0 &&
                !((uintptr_t)a->Y & 15) && !((uintptr_t)a->post_nw & 15)) {
                // the residual add fused with the next product's RMSNorm and split (into this
                // product's xs, which it has finished reading)
                auto red = S == 2 ? k_splitk_reduce_rms<2> : S == 3 ? k_splitk_reduce_rms<3> : k_splitk_reduce_rms<4>;
                hipLaunchKernelGGL(red, dim3(a->N), dim3(TPB), 0, s, a->part, a->N, a->M, a->Y, a->ldy,
                                   a->post_nw, a->post_eps, a->xs);
                *a->post_done = 1;
                return hipGetLastError();
            }
            const uint32_t rg = (uint32_t)min(((uint64_t)a->N * a->M + TPB - 1) / TPB, (uint64_t)4096);
#define GR(E) hipLaunchKernelGGL((k_splitk_reduce<E>), dim3(rg), dim3(TPB), 0, s, a->part, S, a->N, a->M, Yo, a->ldy)
            if (epi == SGK_EPI_ADD) GR(SGK_EPI_ADD);
            else if (epi == SGK_EPI_SWIGLU) GR(SGK_EPI_SWIGLU);
            else if (epi == SGK_EPI_SWIGLU_XS) GR(SGK_EPI_SWIGLU_XS);
            else GR(SGK_EPI_STORE);
#undef GR
            return hipGetLastError();
        }
        uint32_t full = grid, S2 = 1;
        if (a->part && grid > slots) {
            full = grid / slots * slots;               // indices of the full rounds
            const uint32_t left = grid - full;
            if (left && left <= slots / 2) {
                S2 = min((uint32_t)GM_TR_SMAX, slots / left);
                while (S2 > 1 && (nblk / S2 < 8 || (uint64_t)S2 * left * (GM_TN * TM) > a->part_cap)) S2--;
            }
            if (S2 < 2) full = grid;
        }
        if (epi == SGK_EPI_ADD) GL(SGK_EPI_ADD, dim3(full), a->Y, a->ldy, (uint64_t)0, 0u);
        else if (epi == SGK_EPI_SWIGLU) GL(SGK_EPI_SWIGLU, dim3(full), a->Y, a->ldy, (uint64_t)0, 0u);
        else if (epi == SGK_EPI_SWIGLU_XS) GL(SGK_EPI_SWIGLU_XS, dim3(full), Yo, a->ldy, (uint64_t)0, 0u);
        else GL(SGK_EPI_STORE, dim3(full), a->Y, a->ldy, (uint64_t)0, 0u);
        if (full < grid) {
            const uint32_t left = grid - full;
            GL(SGK_EPI_TILE, dim3(left, S2), a->part, 0u, (uint64_t)0, full);
#define GT(E, TMV) hipLaunchKernelGGL((k_tile_reduce<E, TMV>), dim3(left, gm_tr_parts<TMV>()), dim3(TPB), 0, s, a->part, S2, left, full, a->N, a->M, Yo, a->ldy)
#define GT2(E) do { if (kind == GEMM_WIDE) GT(E, GX_TM); else GT(E, GM_TM); } while (0)
            if (epi == SGK_EPI_ADD) GT2(SGK_EPI_ADD);
            else if (epi == SGK_EPI_SWIGLU) GT2(SGK_EPI_SWIGLU);
            else if (epi == SGK_EPI_SWIGLU_XS) GT2(SGK_EPI_SWIGLU_XS);
            else GT2(SGK_EPI_STORE);
#undef GT2
#undef GT
        }
#undef GL
    } else {
        dim3 grid((a->M + 15) / 16, (a->N + 15) / 16);
#define GF(E) hipLaunchKernelGGL(k_gemm_f32<E>, grid, dim3(TPB), 0, s, a->X, a->wf, a->Y, a->N, a->M, a->K, a->ldx, a->ldy)
        if (a->epi == SGK_EPI_ADD) GF(SGK_EPI_ADD); else if (a->epi == SGK_EPI_SWIGLU) GF(SGK_EPI_SWIGLU); else GF(SGK_EPI_STORE);
#undef GF
    }
    return hipGetLastError();
}

extern "C" hipError_t sgk_gemm_q8(const float *X, const int8_t *qs, const uint16_t *dt, float *Y,
                                  uint32_t N, uint32_t M, uint32_t K, uint16_t *xs, float *part,
                                  uint64_t part_cap, hipStream_t s) {
    sgk_gemm_args a = {X, qs, dt, NULL, Y, N, M, K, K, M, SGK_EPI_STORE, xs, part, part_cap};
    return sgk_gemm(&a, s);
}

// ---------------------------------------------------------------------------
// Measurement kernels: a plain streaming read (16-byte non-temporal loads, a
// grid stride over the bytes, one value per workgroup written so the loads
// are not removed) and an empty kernel; the floor any decode kernel of the
// same size stands on.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(TPB) k_read(const uint4 *p, uint64_t n16, float *out) {
    // wave w of the grid reads 4 KB pieces w, w + W, ... (lane l: 16 bytes at
    // l, l + 64, l + 128, l + 192 of the piece: four loads in flight, one
    // contiguous stream per wave, as a GEMV wave streams its rows)
    uint32_t acc = 0;
    const uint64_t W = (uint64_t)gridDim.x * (TPB / 64), lane = threadIdx.x & 63;
    const uint64_t n4k = n16 / 256;
    for (uint64_t w = (uint64_t)blockIdx.x * (TPB / 64) + (threadIdx.x >> 6); w < n4k; w += W) {
        const uint4 *q = p + w * 256 + lane;
        const uint4 v0 = ldnt(q), v1 = ldnt(q + 64), v2 = ldnt(q + 128), v3 = ldnt(q + 192);
        acc ^= (v0.x ^ v0.y ^ v0.z ^ v0.w) ^ (v1.x ^ v1.y ^ v1.z ^ v1.w) ^ (v2.x ^ v2.y ^ v2.z ^ v2.w) ^
               (v3.x ^ v3.y ^ v3.z ^ v3.w);
    }
    for (uint64_t i = n4k * 256 + (uint64_t)blockIdx.x * TPB + threadIdx.x; i < n16; i += (uint64_t)gridDim.x * TPB) {
        const uint4 v = ldnt(p + i);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    __shared__ float red[TPB / 64];
    const float s = block_sum((float)(acc & 0xffu), red);
    if (threadIdx.x == 0) out[blockIdx.x] = s;
}
__global__ void k_empty() {}

extern "C" hipError_t sgk_read(const void *p, uint64_t bytes, float *out, uint32_t blocks, hipStream_t s) {
    if (!p || bytes % 16 || !blocks) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_read, dim3(blocks), dim3(TPB), 0, s, (const uint4 *)p, bytes / 16, out);
    return hipGetLastError();
}
extern "C" hipError_t sgk_empty(hipStream_t s) {
    hipLaunchKernelGGL(k_empty, dim3(1), dim3(64), 0, s);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// A device-resident workspace for callers that cannot allocate (code under
// graph capture, serving loops): the no-allocation entry points place their
// partials here instead of in memory from hipMalloc. Each GPU holds its own
// copy until the process ends; its device address is looked up once per
// device (hipGetSymbolAddress, with that device current) and kept, and only
// that address is ever handed to kernels, fills or copies. Every call on one
// GPU shares it, so calls that overlap on one GPU race.
// ---------------------------------------------------------------------------
static __device__ __align__(256) uint8_t scratch[SGK_SCRATCH_BYTES];
#define SGK_SCRATCH_DEVICES 64
static void *scratch_at[SGK_SCRATCH_DEVICES];

extern "C" hipError_t sgk_scratch_init(int dev) {
    if (dev < 0 || dev >= SGK_SCRATCH_DEVICES) return hipErrorInvalidDevice;
    if (scratch_at[dev]) return hipSuccess;
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return e;
    if (cur != dev) return hipErrorInvalidDevice;       // the caller makes `dev` current
    void *p = NULL;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    scratch_at[dev] = p;
    return hipSuccess;
}

extern "C" void *sgk_scratch_ptr(int dev) {
    return (dev >= 0 && dev < SGK_SCRATCH_DEVICES) ? scratch_at[dev] : NULL;
}

extern "C" uint32_t sgk_device_cus(void) { return (uint32_t)device_cus(); }
