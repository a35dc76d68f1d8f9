"""GPU per-op parity: each HIP kernel, called through the C ABI, against the
CPU oracle on the same seeded inputs (the reference's own per-op strategy,
reference tests/test_metal_ops.c:1-63).

Bars (stated per test): integer/byte work bit-exact; fp32 outputs within
1e-3 relative, measured both as the reference's scale-relative
max|err|/max|want| and per element with an absolute floor of 1e-3*max|want|.
The GPU accumulates in fp32 where the oracle uses double, so ~1e-6 is the
expected error; 1e-3 is the acceptance bar.
"""
import numpy as np
import pytest

import oracle_lib as O
import surge_amd as S
from oracle_lib import fp

pytestmark = pytest.mark.gpu
TOL = 1e-3


def rel_err(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = max(np.abs(want).max(), 1e-30)
    return float(np.abs(got - want).max() / scale)


def assert_close(got, want, tol=TOL):
    e = rel_err(got, want)
    assert e < tol, f"scale-relative error {e:.3e} >= {tol}"
    floor = tol * max(np.abs(want).max(), 1e-30)
    bad = np.abs(np.asarray(got, np.float64) - want) > tol * np.abs(want) + floor
    assert not bad.any(), f"{bad.sum()} elements outside rel {tol} + floor"


def q8_matrix(rng, rows, cols, sigma=0.02):
    """BASELINE GEMV config: 32 int8 uniform in [-127,127] per block and
    scale f16(|N(0, sigma)|/127) (about 30% subnormal at sigma 0.02)."""
    nb = cols // 32
    q = rng.integers(-127, 128, size=(rows, nb, 32), dtype=np.int8)
    d = (np.abs(rng.standard_normal((rows, nb))) * sigma / 127).astype(np.float16)
    raw = np.zeros((rows, nb, 34), np.uint8)
    raw[:, :, :2] = d.view(np.uint8).reshape(rows, nb, 2)
    raw[:, :, 2:] = q.view(np.uint8)
    return raw.reshape(-1)


def oracle_matvec_q8(raw, x, rows, cols):
    y = np.zeros(rows, np.float32)
    O.oracle().sg_ref_matvec_q8(raw.ctypes.data, fp(x), fp(y), rows, cols)
    return y


def gpu_matvec_q8(gpu, raw, x, rows, cols):
    w, xb, y = gpu.buf(raw), gpu.buf(x), gpu.buf(np.zeros(rows, np.float32))
    gpu.run_op("k_matvec_q8", w, xb, y, [rows, cols])
    out = y.array.copy()
    for b in (w, xb, y):
        b.free()
    return out


# ---------------------------------------------------------------- GEMV

def test_gemv_q8_scale_decode_exact_all_f16_patterns(gpu):
    """Row r has one block with scale bits r, q = (1, 0, ...), x = e_0: y[r]
    must be exactly the f16 value, subnormals included."""
    rows, cols = 65536, 32
    raw = np.zeros((rows, 34), np.uint8)
    raw[:, :2] = np.arange(rows, dtype=np.uint16).view(np.uint8).reshape(rows, 2)
    raw[:, 2] = 1
    x = np.zeros(cols, np.float32)
    x[0] = 1
    got = gpu_matvec_q8(gpu, raw.reshape(-1), x, rows, cols)
    want = np.arange(rows, dtype=np.uint16).view(np.float16).astype(np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin], want[fin])
    assert np.isnan(got[np.isnan(want)]).all()


def test_gemv_q8_baseline_config_4096(gpu):
    rng = np.random.default_rng(0)
    rows = cols = 4096
    raw = q8_matrix(rng, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    got = gpu_matvec_q8(gpu, raw, x, rows, cols)
    want = oracle_matvec_q8(raw, x, rows, cols)
    assert_close(got, want)
    assert rel_err(got, want) < 1e-5          # fp32 accumulation, expect ~1e-7
    again = gpu_matvec_q8(gpu, raw, x, rows, cols)
    assert np.array_equal(got, again)          # bit-identical reruns


@pytest.mark.parametrize("rows,cols", [(1, 32), (37, 64), (3, 17408), (5120, 6144),
                                       (16480, 5120), (40000, 2048), (7, 96)])
def test_gemv_q8_shapes(gpu, rows, cols):
    rng = np.random.default_rng(rows * 7 + cols)
    raw = q8_matrix(rng, rows, cols, sigma=1.0)
    x = rng.standard_normal(cols).astype(np.float32)
    assert_close(gpu_matvec_q8(gpu, raw, x, rows, cols), oracle_matvec_q8(raw, x, rows, cols))


def test_gemv_f32(gpu):
    rng = np.random.default_rng(3)
    rows, cols = 50, 24
    w = rng.standard_normal(rows * cols).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    want = np.zeros(rows, np.float32)
    O.oracle().sg_ref_matvec_f32(fp(w), fp(x), fp(want), rows, cols)
    wb, xb, yb = gpu.buf(w), gpu.buf(x), gpu.buf(np.zeros(rows, np.float32))
    gpu.run_op("k_matvec_f32", wb, xb, yb, [rows, cols])
    assert_close(yb.array, want)


def test_gemv_rejects_bad_shapes(gpu):
    w, x, y = gpu.buf(np.zeros(34, np.uint8)), gpu.buf(np.zeros(48, np.float32)), gpu.buf(np.zeros(1, np.float32))
    with pytest.raises(S.SurgeError):
        gpu.run_op("k_matvec_q8", w, x, y, [1, 48])     # cols % 32
    with pytest.raises(S.SurgeError):
        gpu.run_op("k_matvec_q8", w, x, y, [2, 32])     # w too small
    with pytest.raises(S.SurgeError):
        gpu.run_op("k_matvec_q8", w, x, w, [1, 32])     # out aliases input


# ---------------------------------------------------------------- attention

def f16(rng, n):
    return rng.standard_normal(n).astype(np.float16)


def run_partial_combine(gpu, q, k16, v16, nh, nkv, hd, seq, qs, ns):
    sc = 1.0 / np.sqrt(hd)
    p = [nh, nkv, hd, seq, qs, S.fbits(sc), ns]
    qb, kb, vb = gpu.buf(q), gpu.buf(k16.view(np.uint16) if seq else np.zeros(1, np.uint16)), \
        gpu.buf(v16.view(np.uint16) if seq else np.zeros(1, np.uint16))
    mb, sb = gpu.buf(np.zeros(nh * ns, np.float32)), gpu.buf(np.zeros(nh * ns, np.float32))
    ab, ob = gpu.buf(np.zeros(nh * ns * hd, np.float32)), gpu.buf(np.zeros(nh * hd, np.float32))
    gpu.attn_partial(qb, kb, vb, mb, sb, ab, p)
    gpu.attn_combine(mb, sb, ab, ob, p)
    res = (mb.array.copy(), sb.array.copy(), ab.array.copy(), ob.array.copy())
    for b in (qb, kb, vb, mb, sb, ab, ob):
        b.free()
    return res


def oracle_attn(q, k16, v16, nh, nkv, hd, seq, qs, ns):
    kc = k16.astype(np.float32) if seq else np.zeros(1, np.float32)
    vc = v16.astype(np.float32) if seq else np.zeros(1, np.float32)
    sc = np.float32(1.0 / np.sqrt(hd))
    m, s = np.zeros(nh * ns, np.float32), np.zeros(nh * ns, np.float32)
    acc = np.zeros(nh * ns * hd, np.float32)
    O.oracle().sg_ref_attn_partials(fp(q), fp(kc), fp(vc), nh, nkv, hd, seq, qs, sc, ns, fp(m), fp(s), fp(acc))
    out = np.zeros(nh * hd, np.float32)
    O.oracle().sg_ref_attn_decode_splitk(fp(q), fp(kc), fp(vc), nh, nkv, hd, seq, qs, sc, ns, fp(out))
    return m, s, acc, out


ATT_CASES = [(16, 512, 8), (16, 512, 16), (16, 512, 0), (16, 4096, 32), (16, 4096, 64), (16, 4096, 0),
             (16, 32768, 64), (16, 32768, 0), (24, 512, 0), (24, 4096, 8), (24, 4096, 0), (24, 32768, 32),
             (24, 32768, 0), (24, 131072, 0)]


@pytest.mark.parametrize("nh,seq,ns", ATT_CASES, ids=[f"{h}q-{s}-{n or 'policy'}" for h, s, n in ATT_CASES])
def test_splitk_gqa_baseline_config(gpu, nh, seq, ns):
    """BASELINE attention config: 16 q / 4 kv heads (and the 27B's 24 / 4),
    head_dim 256, f16 KV N(0,1), q N(0,1), scale 1/16, at 512 / 4096 / 32768
    keys with 8-64 splits and with the decode policy's own count (ns 0: about
    64 keys per split, at most 128, so at 32768 keys every split walks four
    64-key rounds, at 131072 sixteen), then the LSE combine. The one-shot runs the decode
    path's MFMA partial (k_attn_partial_wv) with q taken as given."""
    rng = np.random.default_rng(seq + ns + nh)
    nkv, hd = 4, 256
    ns = ns or S.lib().sg_gpu_splitk_gqa_n_splits(seq)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k16, v16 = f16(rng, seq * nkv * hd), f16(rng, seq * nkv * hd)
    gm, gs, gacc, gout = run_partial_combine(gpu, q, k16, v16, nh, nkv, hd, seq, hd, ns)
    om, os_, oacc, oout = oracle_attn(q, k16, v16, nh, nkv, hd, seq, hd, ns)
    assert np.abs(gm - om).max() <= 1e-5 * np.abs(om).max()
    assert_close(gs, os_)
    assert_close(gacc, oacc)
    assert_close(gout, oout)
    assert rel_err(gout, oout) < 1e-5


@pytest.mark.parametrize("hd,seq,ns", [(256, 4096, 64), (128, 1000, 7), (256, 70, 3)])
def test_splitk_per_head_and_gqa_partials_same_bytes(gpu, hd, seq, ns):
    """The per-head partial (one workgroup per query head) and the GQA one
    (one per kv head, all of its group) give the same bytes, as the
    reference contracts for its two kernels (surge.h:1170-1254)."""
    rng = np.random.default_rng(hd + seq)
    nh, nkv = 24, 4
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k16, v16 = f16(rng, seq * nkv * hd), f16(rng, seq * nkv * hd)
    p = [nh, nkv, hd, seq, hd, S.fbits(1.0 / np.sqrt(hd)), ns]
    outs = []
    for gqa in (True, False):
        bufs = [gpu.buf(q), gpu.buf(k16.view(np.uint16)), gpu.buf(v16.view(np.uint16)),
                gpu.buf(np.zeros(nh * ns, np.float32)), gpu.buf(np.zeros(nh * ns, np.float32)),
                gpu.buf(np.zeros(nh * ns * hd, np.float32))]
        gpu.attn_partial(*bufs, p, gqa=gqa)
        outs.append([b.array.copy() for b in bufs[3:]])
        for b in bufs:
            b.free()
    for x, y in zip(*outs):
        assert np.array_equal(x, y)


def test_splitk_valu_partial_matches_mfma(gpu, monkeypatch):
    """SURGE_ATTN_VALU=1 (the A/B switch) runs the VALU partial: against the
    oracle at the 27B shape, and against the MFMA partial's output."""
    rng = np.random.default_rng(77)
    nh, nkv, hd, seq, ns = 24, 4, 256, 3000, 47
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k16, v16 = f16(rng, seq * nkv * hd), f16(rng, seq * nkv * hd)
    mf = run_partial_combine(gpu, q, k16, v16, nh, nkv, hd, seq, hd, ns)
    monkeypatch.setenv("SURGE_ATTN_VALU", "1")
    va = run_partial_combine(gpu, q, k16, v16, nh, nkv, hd, seq, hd, ns)
    monkeypatch.delenv("SURGE_ATTN_VALU")
    om, os_, oacc, oout = oracle_attn(q, k16, v16, nh, nkv, hd, seq, hd, ns)
    assert_close(va[3], oout)
    assert_close(va[2], oacc)
    assert rel_err(va[3], mf[3]) < 1e-5


@pytest.mark.parametrize("nh,nkv,hd,seq,ns", [(4, 4, 64, 100, 3), (8, 1, 128, 77, 5), (6, 2, 32, 40, 64),
                                              (2, 2, 16, 1, 1), (24, 4, 256, 1000, 31), (4, 2, 128, 0, 4)])
def test_splitk_shapes_and_edges(gpu, nh, nkv, hd, seq, ns):
    """Per-head (G=1), wide groups, tiny head dims, more splits than keys
    (empty splits), seq 0, and a gated q_stride whose gate half is NaN."""
    rng = np.random.default_rng(nh * 1000 + seq)
    qs = 2 * hd
    q = rng.standard_normal(nh * qs).astype(np.float32).reshape(nh, qs)
    q[:, hd:] = np.nan                      # the gate half must never be read
    q = np.ascontiguousarray(q.reshape(-1))
    k16, v16 = f16(rng, seq * nkv * hd), f16(rng, seq * nkv * hd)
    gm, gs, gacc, gout = run_partial_combine(gpu, q, k16, v16, nh, nkv, hd, seq, qs, ns)
    om, os_, oacc, oout = oracle_attn(q, k16, v16, nh, nkv, hd, seq, qs, ns)
    assert np.isfinite(gout).all()
    assert np.array_equal(np.isneginf(gm), np.isneginf(om))   # same empty splits
    fin = np.isfinite(om)
    if fin.any():
        assert np.abs(gm[fin] - om[fin]).max() <= 1e-5 * max(np.abs(om[fin]).max(), 1)
    if seq:
        assert_close(gout, oout)
    else:
        assert (gout == 0).all()


def test_attn_decode_f16_single_call(gpu):
    rng = np.random.default_rng(11)
    nh, nkv, hd, seq = 16, 4, 256, 700
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k16, v16 = f16(rng, seq * nkv * hd), f16(rng, seq * nkv * hd)
    qb, kb, vb = gpu.buf(q), gpu.buf(k16.view(np.uint16)), gpu.buf(v16.view(np.uint16))
    ob = gpu.buf(np.zeros(nh * hd, np.float32))
    gpu.attn_decode_f16(qb, kb, vb, ob, [nh, nkv, hd, seq, hd, S.fbits(1 / 16)])
    want = np.zeros(nh * hd, np.float32)
    kc, vc = k16.astype(np.float32), v16.astype(np.float32)
    O.oracle().sg_ref_attn_decode(fp(q), fp(kc), fp(vc), nh, nkv, hd, seq, hd, np.float32(1 / 16), fp(want))
    assert_close(ob.array, want)


def test_combine_degenerate_cases(gpu):
    hd, ns, nh = 32, 3, 4
    rng = np.random.default_rng(1)
    acc = rng.standard_normal(nh * ns * hd).astype(np.float32)
    m = np.float32([[1.5, -np.inf, 0.5], [-np.inf] * 3, [np.nan, 1, 2], [np.inf, 3, np.inf]]).reshape(-1)
    s = np.float32([[2, 0, 3], [0, 0, 0], [1, 1, 1], [2, 1, 4]]).reshape(-1)
    mb, sb, ab = gpu.buf(m), gpu.buf(s), gpu.buf(acc)
    ob = gpu.buf(np.full(nh * hd, 7, np.float32))
    gpu.attn_combine(mb, sb, ab, ob, [nh, 1, hd, 0, hd, 0, ns])
    want = np.zeros(nh * hd, np.float32)
    for h in range(nh):
        O.oracle().sg_ref_attn_combine(fp(m[h * ns:(h + 1) * ns].copy()), fp(s[h * ns:(h + 1) * ns].copy()),
                                       fp(acc[h * ns * hd:(h + 1) * ns * hd].copy()), ns, hd,
                                       fp(want[h * hd:(h + 1) * hd]))
    got = ob.array.reshape(nh, hd)
    want = want.reshape(nh, hd)
    assert_close(got[0], want[0])
    assert (got[1] == 0).all()                       # all splits empty
    assert np.isnan(got[2]).all()                    # NaN first max propagates
    assert_close(got[3], want[3])                    # +inf ties combine among themselves


# ---------------------------------------------------------------- DeltaNet

def test_delta_multi_baseline_config(gpu):
    """BASELINE DeltaNet config: 16 heads, dk = dv = 128, S N(0, 0.1), q, k
    L2-normalised, v N(0,1), beta = sigmoid(N), decay = exp(-softplus(N)).
    Two consecutive steps thread S."""
    rng = np.random.default_rng(4)
    nv = nk = 16
    dk = dv = 128
    kd = nk * dk
    S0 = (rng.standard_normal(nv * dv * dk) * 0.1).astype(np.float32)
    Sg = gpu.buf(S0.copy())
    So = S0.copy()
    for step in range(2):
        q = rng.standard_normal((nk, dk))
        k = rng.standard_normal((nk, dk))
        q = (q / np.linalg.norm(q, axis=1, keepdims=True)).astype(np.float32)
        k = (k / np.linalg.norm(k, axis=1, keepdims=True)).astype(np.float32)
        v = rng.standard_normal(nv * dv).astype(np.float32)
        qkv = np.concatenate([q.reshape(-1), k.reshape(-1), v]).astype(np.float32)
        beta = np.array([O.oracle().sg_ref_sigmoid(float(b)) for b in rng.standard_normal(nv)], np.float32)
        decay = np.array([O.oracle().sg_ref_delta_decay_neg_a(-1.0, float(a), 0.0) for a in rng.standard_normal(nv)],
                         np.float32)
        qb, ob, gb = gpu.buf(qkv), gpu.buf(np.zeros(nv * dv, np.float32)), gpu.buf(np.concatenate([beta, decay]))
        gpu.delta_multi(Sg, qb, ob, gb, [dk, dv, nv, nk, kd, 1])
        want = np.zeros(nv * dv, np.float32)
        for h in range(nv):
            hk = h % nk
            O.oracle().sg_ref_delta_step(fp(So[h * dv * dk:]), fp(np.ascontiguousarray(q[hk])),
                                         fp(np.ascontiguousarray(k[hk])), fp(np.ascontiguousarray(v[h * dv:(h + 1) * dv])),
                                         float(beta[h]), float(decay[h]), fp(want[h * dv:]), dk, dv)
        assert_close(ob.array, want)
        assert_close(Sg.array, So)
        for b in (qb, ob, gb):
            b.free()


def test_delta_multi_tiled_group_map(gpu):
    """48 value heads over 16 key heads (the 27B shape): tiled h % n_k."""
    rng = np.random.default_rng(9)
    nv, nk, dk, dv = 48, 16, 128, 128
    kd = nk * dk
    S0 = (rng.standard_normal(nv * dv * dk) * 0.1).astype(np.float32)
    qkv = rng.standard_normal(2 * kd + nv * dv).astype(np.float32) * 0.1
    gates = np.concatenate([rng.uniform(0, 1, nv), rng.uniform(0.5, 1, nv)]).astype(np.float32)
    Sg, qb, ob, gb = gpu.buf(S0.copy()), gpu.buf(qkv), gpu.buf(np.zeros(nv * dv, np.float32)), gpu.buf(gates)
    gpu.delta_multi(Sg, qb, ob, gb, [dk, dv, nv, nk, kd, 1])
    So, want = S0.copy(), np.zeros(nv * dv, np.float32)
    for h in range(nv):
        hk = h % nk
        O.oracle().sg_ref_delta_step(fp(So[h * dv * dk:]), fp(qkv[hk * dk:]), fp(qkv[kd + hk * dk:]),
                                     fp(qkv[2 * kd + h * dv:]), float(gates[h]), float(gates[nv + h]),
                                     fp(want[h * dv:]), dk, dv)
    assert_close(ob.array, want)
    assert_close(Sg.array, So)


def test_conv1d_step_baseline_config(gpu):
    """Causal conv width 4 over 2048 channels with rolling state, 3 steps."""
    rng = np.random.default_rng(6)
    ch, ks = 2048, 4
    w = rng.standard_normal(ch * ks).astype(np.float32)
    st_o = np.zeros((ks - 1) * ch, np.float32)
    ob = gpu.buf(np.zeros(ch * ks, np.float32))    # y[ch] | state[(ks-1)*ch]
    wb = gpu.buf(w)
    for _ in range(3):
        x = rng.standard_normal(ch).astype(np.float32)
        xb = gpu.buf(x)
        gpu.run_op("k_conv1d_step", xb, wb, ob, [ch, ks])
        xo = x.copy()
        O.oracle().sg_ref_conv1d_causal(fp(xo), fp(w), fp(st_o), fp(st_o), ch, ks)
        assert_close(ob.array[:ch], xo)
        assert np.array_equal(ob.array[ch:], st_o)   # the state shift is exact
        xb.free()


def oracle_gdn_step(inp, w, state, dk, dv, nv, nk, ks, tiled, eps):
    """ref.c's gdn_layer between its projections and its output projection
    (ref.c:1283-1330), composed from the oracle's ops: conv + SiLU, q/k RMS
    (eps 1e-6, no weight) then q / dk and k / sqrt(dk), beta = sigmoid(b),
    decay from -exp(A_log) (the GGUF form), the delta rule per value head
    (tiled or grouped k-head map), RMSNormGated. Returns (out, new state)."""
    o = O.oracle()
    kd, vd = nk * dk, nv * dv
    cd = 2 * kd + vd
    qkv = inp[:cd].copy()
    z, bb, aa = inp[cd:cd + vd], inp[cd + vd:cd + vd + nv], inp[cd + vd + nv:]
    conv_w, ssm_a = w[:cd * ks], w[cd * ks:cd * ks + nv]
    dt, nw = w[cd * ks + nv:cd * ks + 2 * nv], np.ascontiguousarray(w[cd * ks + 2 * nv:])
    keep = ks - 1
    conv = state[:keep * cd].copy()
    Sm = state[keep * cd:].copy()
    o.sg_ref_conv1d_causal(fp(qkv), fp(np.ascontiguousarray(conv_w)), fp(conv), fp(conv), cd, ks)
    o.sg_ref_silu(fp(qkv), cd)
    inv = 1.0 / np.sqrt(np.float64(dk))
    for h in range(nk):
        for off in (0, kd):
            seg = np.ascontiguousarray(qkv[off + h * dk:off + (h + 1) * dk])
            o.sg_ref_rmsnorm(fp(seg), None, dk, 1e-6)
            sc = inv * inv if off == 0 else inv
            qkv[off + h * dk:off + (h + 1) * dk] = (seg.astype(np.float64) * sc).astype(np.float32)
    y = np.zeros(vd, np.float32)
    for h in range(nv):
        hk = h % nk if tiled else h // (nv // nk)
        beta = o.sg_ref_sigmoid(float(bb[h]))
        decay = o.sg_ref_delta_decay_neg_a(float(ssm_a[h]), float(aa[h]), float(dt[h]))
        o.sg_ref_delta_step(fp(Sm[h * dv * dk:]), fp(np.ascontiguousarray(qkv[hk * dk:(hk + 1) * dk])),
                            fp(np.ascontiguousarray(qkv[kd + hk * dk:kd + (hk + 1) * dk])),
                            fp(np.ascontiguousarray(qkv[2 * kd + h * dv:2 * kd + (h + 1) * dv])),
                            beta, decay, fp(y[h * dv:]), dk, dv)
    out = np.zeros(vd, np.float32)
    for h in range(nv):
        yy = y[h * dv:(h + 1) * dv].copy()
        zz = z[h * dv:(h + 1) * dv].copy()
        o.sg_ref_rmsnorm(fp(yy), fp(nw), dv, eps)
        o.sg_ref_swiglu(fp(zz), fp(yy), dv)
        out[h * dv:(h + 1) * dv] = zz
    return out, np.concatenate([conv, Sm])


GDN_CASES = [(16, 16, 128, 128, 4, True), (48, 16, 128, 128, 4, True), (6, 2, 64, 64, 4, False),
             (8, 4, 128, 96, 2, True), (4, 4, 256, 128, 3, False)]


@pytest.mark.parametrize("nv,nk,dk,dv,ks,tiled", GDN_CASES,
                         ids=[f"{a}v{b}k-dk{c}-dv{d}-ks{e}-{'tiled' if f else 'grouped'}" for a, b, c, d, e, f in GDN_CASES])
def test_gdn_decode_step_vs_oracle(gpu, nv, nk, dk, dv, ks, tiled):
    """The decode path's fused DeltaNet step (k_gdn_step: conv ring + SiLU,
    q/k norms and scales, beta/decay, rank-1 update and readout of S held in
    registers, RMSNormGated) against ref.c's gdn_layer composed from the
    oracle: the BASELINE config (16 heads, dk = dv = 128, S N(0, 0.1), conv
    width 4; conv_dim 6144 of which 2048 per q/k/v), the 27B's 48 value heads
    tiled over 16 key heads, a grouped map, other widths and conv sizes.
    Three steps thread the state: outputs and S within 1e-3 (expect ~1e-6),
    the conv tail bit-exact (it holds the inputs)."""
    rng = np.random.default_rng(nv * 7 + dk + ks)
    cd, vd = 2 * nk * dk + nv * dv, nv * dv
    eps = 1e-6
    w = np.concatenate([rng.standard_normal(cd * ks) * 0.5, -np.exp(rng.uniform(-1, 1, nv)),
                        rng.uniform(-0.5, 0.5, nv), 1.0 + 0.1 * rng.standard_normal(dv)]).astype(np.float32)
    state = np.concatenate([rng.standard_normal((ks - 1) * cd), rng.standard_normal(nv * dv * dk) * 0.1])
    state = state.astype(np.float32)
    wb, sb, ob = gpu.buf(w), gpu.buf(state.copy()), gpu.buf(np.zeros(vd, np.float32))
    so = state.copy()
    for step in range(3):
        inp = rng.standard_normal(cd + vd + 2 * nv).astype(np.float32)
        ib = gpu.buf(inp)
        gpu.gdn_step(ib, wb, sb, ob, [dk, dv, nv, nk, ks, int(tiled), 1, S.fbits(eps)])
        want, so = oracle_gdn_step(inp, w, so, dk, dv, nv, nk, ks, tiled, eps)
        assert_close(ob.array, want)
        assert np.array_equal(sb.array[:(ks - 1) * cd], so[:(ks - 1) * cd])
        assert_close(sb.array[(ks - 1) * cd:], so[(ks - 1) * cd:])
        ib.free()


GDN_CHUNK_CASES = [(16, 16, 128, 128, 4, True, 37, 2), (48, 16, 128, 128, 4, True, 130, 19),
                   (6, 2, 64, 64, 4, False, 33, 50), (8, 4, 128, 96, 2, True, 20, 2),
                   (4, 4, 256, 128, 3, False, 18, 5), (8, 4, 32, 32, 4, True, 24, 9)]


@pytest.mark.parametrize("nv,nk,dk,dv,ks,tiled,n1,n2", GDN_CHUNK_CASES,
                         ids=[f"{a}v{b}k-dk{c}-dv{d}-ks{e}-{'tiled' if f else 'grouped'}-{g}+{h}"
                              for a, b, c, d, e, f, g, h in GDN_CHUNK_CASES])
def test_gdn_prefill_chunk_vs_oracle(gpu, nv, nk, dk, dv, ks, tiled, n1, n2):
    """The prefill path's DeltaNet layer core (sg_gpu_run_gdn_chunk: the
    chunk conv k_conv_chunk, with the q/k norm inside it at dk 64 and 128
    and k_qk_norm_chunk after it at 256; the ring k_conv_ring; the scan in
    the build's default form, k_dm_prep + k_dm_scan on the matrix cores at
    dk 64 and 128 and the sequential k_delta_chunk at 256, with the gates
    from the b, a columns; the RMSNormGated rows) against ref.c's gdn_layer
    composed from the oracle, token by token: the BASELINE DeltaNet config
    (16 heads, 128^2, conv width 4), the 27B's 48 value heads tiled over 16
    key heads over a 130-token chunk (eight full 16-token blocks and a
    partial one), a grouped dk 64 map, conv widths 2 and 3, and dk 32 (the
    sequential scan with the separate q/k norm pass). Two chunks in a
    row thread the conv tail and S, the second starting at another ring slot
    (and shorter than the conv tail in one case); outputs and S within 1e-3,
    the conv tail bit-exact (it holds the inputs)."""
    rng = np.random.default_rng(nv * 11 + dk + ks + n1)
    cd, vd = 2 * nk * dk + nv * dv, nv * dv
    row = cd + vd + 2 * nv
    eps = 1e-6
    w = np.concatenate([rng.standard_normal(cd * ks) * 0.5, -np.exp(rng.uniform(-1, 1, nv)),
                        rng.uniform(-0.5, 0.5, nv), 1.0 + 0.1 * rng.standard_normal(dv)]).astype(np.float32)
    state = np.concatenate([rng.standard_normal((ks - 1) * cd), rng.standard_normal(nv * dv * dk) * 0.1])
    state = state.astype(np.float32)
    wb, sb = gpu.buf(w), gpu.buf(state.copy())
    so = state.copy()
    for n, slot in ((n1, 1), (n2, 2)):
        inp = rng.standard_normal((n, row)).astype(np.float32)
        ib, ob = gpu.buf(inp.reshape(-1)), gpu.buf(np.zeros(n * vd, np.float32))
        gpu.gdn_chunk(ib, wb, sb, ob, [dk, dv, nv, nk, ks, int(tiled) | 2 | slot << 2, n, S.fbits(eps)])
        want = np.zeros((n, vd), np.float32)
        for z in range(n):
            want[z], so = oracle_gdn_step(inp[z], w, so, dk, dv, nv, nk, ks, tiled, eps)
        assert_close(ob.array, want.reshape(-1))
        assert np.array_equal(sb.array[:(ks - 1) * cd], so[:(ks - 1) * cd])
        assert_close(sb.array[(ks - 1) * cd:], so[(ks - 1) * cd:])
        ib.free()
        ob.free()


def test_gdn_step_rejects_bad_shapes(gpu):
    b = gpu.buf(np.zeros(1 << 16, np.float32))
    o = gpu.buf(np.zeros(1 << 12, np.float32))
    for p in ([100, 64, 4, 4, 4, 1, 1, 0], [64, 256, 4, 4, 4, 1, 1, 0], [64, 64, 6, 4, 4, 1, 1, 0],
              [64, 64, 4, 4, 5, 1, 1, 0]):
        with pytest.raises(S.SurgeError):
            gpu.gdn_step(b, b, o, o, p)


def test_gdn_chunk_rejects_bad_shapes(gpu):
    """dk outside 32/64/128/256, n_v not a multiple of n_k, ksize 5, an empty
    chunk, a chunk longer than its input rows, state aliasing the input."""
    b = gpu.buf(np.zeros(1 << 16, np.float32))
    st = gpu.buf(np.zeros(1 << 16, np.float32))
    o = gpu.buf(np.zeros(1 << 12, np.float32))
    for p in ([100, 64, 4, 4, 4, 1, 4, 0], [64, 64, 6, 4, 4, 1, 4, 0], [64, 64, 4, 4, 5, 1, 4, 0],
              [64, 64, 4, 4, 4, 1, 0, 0], [64, 64, 4, 4, 4, 1, 1000, 0]):
        with pytest.raises(S.SurgeError):
            gpu.gdn_chunk(b, b, st, o, p)
    with pytest.raises(S.SurgeError):
        gpu.gdn_chunk(b, st, b, o, [32, 16, 1, 1, 4, 1, 1, 0])


# even GQA groups run two query heads per workgroup, odd ones (12/4, 6/6) one
FLASH_CASES = [(24, 4, 256, 1536, 64), (24, 4, 256, 4000, 37), (16, 4, 128, 2100, 100), (12, 4, 128, 1300, 70),
               (6, 6, 64, 900, 33)]


@pytest.mark.parametrize("nh,nkv,hd,base,n", FLASH_CASES, ids=[f"{a}q{b}kv-hd{c}-base{d}-n{e}" for a, b, c, d, e in FLASH_CASES])
def test_attn_prefill_flash_deep_vs_oracle(gpu, nh, nkv, hd, base, n):
    """The prefill path's MFMA flash attention, called through the
    sg_gpu_run_attn_prefill one-shot: a chunk starting deep in the cache, so
    its key tiles are split over several workgroups (one per 512 keys of the
    deepest token, at most 8) and merged by the LSE combine; token t
    (position base+t) against ref.c's decode attention over keys 0..base+t,
    within 1e-3."""
    rng = np.random.default_rng(base + n + hd)
    qs = 2 * hd
    tot = base + n
    q = rng.standard_normal(n * nh * qs).astype(np.float32)
    k16, v16 = f16(rng, tot * nkv * hd), f16(rng, tot * nkv * hd)
    qb, kb, vb = gpu.buf(q), gpu.buf(k16.view(np.uint16)), gpu.buf(v16.view(np.uint16))
    ob = gpu.buf(np.zeros(n * nh * hd, np.float32))
    sc = 1.0 / np.sqrt(hd)
    gpu.run4("attn_prefill", qb, kb, vb, ob, [nh, nkv, hd, base, n, qs, S.fbits(sc)])
    kc, vc = k16.astype(np.float32), v16.astype(np.float32)
    for t in list(range(0, n, 9)) + [n - 1]:
        want = np.zeros(nh * hd, np.float32)
        O.oracle().sg_ref_attn_decode(fp(np.ascontiguousarray(q[t * nh * qs:(t + 1) * nh * qs])), fp(kc), fp(vc),
                                      nh, nkv, hd, base + t + 1, qs, np.float32(sc), fp(want))
        assert_close(ob.array[t * nh * hd:(t + 1) * nh * hd], want)


# ---------------------------------------------------------------- small ops

def test_small_ops(gpu):
    rng = np.random.default_rng(8)
    n = 5000
    x = (rng.standard_normal(n) * 4).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    o = O.oracle()

    def run(kernel, a, b, p):
        ab, bb, ob = gpu.buf(a), gpu.buf(b) if b is not None else None, gpu.buf(np.zeros(len(a), np.float32))
        gpu.run_op(kernel, ab, bb, ob, p)
        return ob.array.copy()

    want = x.copy(); o.sg_ref_rmsnorm(fp(want), fp(w), n, 1e-6)
    assert_close(run("k_rmsnorm", x, w, [n, S.fbits(1e-6), 1]), want)
    want = x.copy(); o.sg_ref_swiglu(fp(want), fp(w), n)
    assert_close(run("k_swiglu", x, w, [n]), want)
    want = x.copy(); o.sg_ref_silu(fp(want), n)
    assert_close(run("k_silu", x, None, [n]), want)
    want = x.copy(); o.sg_ref_gate_sigmoid(fp(want), fp(w), n)
    assert_close(run("k_gate_sigmoid", x, w, [n]), want)
    assert np.array_equal(run("k_add", x, w, [n]), x + w)
    assert np.array_equal(run("k_scale", x, None, [n, S.fbits(0.25)]), x * np.float32(0.25))
    xs = np.concatenate([x[:100], np.float32([-1e30] * 5)])
    want = xs.copy(); o.sg_ref_softmax(fp(want), len(xs))
    assert_close(run("k_softmax", xs, None, [len(xs)]), want)


def test_rope_heads_and_rmsnorm_heads(gpu):
    rng = np.random.default_rng(12)
    hd, rd, nh, stride, pos, theta = 256, 64, 6, 512, 4095, 1e7
    x = rng.standard_normal(nh * stride).astype(np.float32)
    half = rd // 2
    inv = theta ** (-2.0 * np.arange(half) / rd)
    cs = np.concatenate([np.cos(pos * inv), np.sin(pos * inv)]).astype(np.float32)
    xb, cb, ob = gpu.buf(x), gpu.buf(cs), gpu.buf(np.zeros(nh * stride, np.float32))
    gpu.run_op("k_rope_heads", xb, cb, ob, [hd, rd, nh, stride])
    want = x.copy()
    for h in range(nh):
        seg = np.ascontiguousarray(want[h * stride:h * stride + hd])
        O.oracle().sg_ref_rope_partial(fp(seg), hd, rd, pos, theta)
        want[h * stride:h * stride + hd] = seg
    got = ob.array.reshape(nh, stride)[:, :hd]
    assert_close(got, want.reshape(nh, stride)[:, :hd], 1e-5)
    assert np.array_equal(got[:, rd:], x.reshape(nh, stride)[:, rd:hd])
    wn = rng.standard_normal(hd).astype(np.float32)
    ob2 = gpu.buf(np.zeros(nh * stride, np.float32))
    gpu.run_op("k_rmsnorm_heads", xb, gpu.buf(wn), ob2, [hd, nh, S.fbits(1e-6), stride, 1])
    want = x.copy()
    for h in range(nh):
        seg = np.ascontiguousarray(want[h * stride:h * stride + hd])
        O.oracle().sg_ref_rmsnorm(fp(seg), fp(wn), hd, 1e-6)
        assert_close(ob2.array[h * stride:h * stride + hd], seg)


def test_rmsnorm_gated(gpu):
    rng = np.random.default_rng(13)
    dv, nh = 128, 48
    y = rng.standard_normal(dv * nh).astype(np.float32)
    z = rng.standard_normal(dv * nh).astype(np.float32)
    w = rng.standard_normal(dv).astype(np.float32)
    yb, zb, ob = gpu.buf(y), gpu.buf(np.concatenate([z, w])), gpu.buf(np.zeros(dv * nh, np.float32))
    gpu.run_op("k_rmsnorm_gated", yb, zb, ob, [dv, nh, S.fbits(1e-6)])
    want = np.zeros(dv * nh, np.float32)
    for h in range(nh):
        yy = y[h * dv:(h + 1) * dv].copy()
        zz = z[h * dv:(h + 1) * dv].copy()
        O.oracle().sg_ref_rmsnorm(fp(yy), fp(w), dv, 1e-6)
        O.oracle().sg_ref_swiglu(fp(zz), fp(yy), dv)
        want[h * dv:(h + 1) * dv] = zz
    assert_close(ob.array, want)


def test_kv_store_f16_bit_exact(gpu):
    rng = np.random.default_rng(14)
    x = np.concatenate([rng.standard_normal(10000).astype(np.float32) * 10.0 ** rng.integers(-8, 5, 10000),
                        np.float32([65504, 65519, 65520, 1e9, -1e9, 2 ** -25, 2 ** -24, 3e-5, 0, -0.0])])
    x = x.astype(np.float32)
    xb, ob = gpu.buf(x), gpu.buf(np.zeros(len(x) + 8, np.uint16))
    gpu.run_op("k_kv_store_f16", xb, None, ob, [len(x), 8])
    want = np.array([O.oracle().sg_ref_f32_to_f16(float(v)) for v in x], np.uint16)
    assert np.array_equal(ob.array[8:], want)
    assert (ob.array[:8] == 0).all()


@pytest.mark.parametrize("N,M,K", [(70, 130, 256), (300, 260, 96), (1, 32, 32), (129, 384, 1056)])
def test_matmul_q8_prefill_gemm(gpu, N, M, K):
    """Token and row tails (N, M past a 128 tile), an odd block count, a
    single token; (129, 384, 1056) is narrow enough to split K four ways
    (8, 8, 8 and 9 blocks, partials summed in order)."""
    rng = np.random.default_rng(15 + N)
    X = rng.standard_normal(N * K).astype(np.float32)
    raw = q8_matrix(rng, M, K, sigma=1.0)
    xb, wb, yb = gpu.buf(X), gpu.buf(raw), gpu.buf(np.zeros(N * M, np.float32))
    gpu.run_op("k_matmul_q8", xb, wb, yb, [N, M, K])
    want = np.stack([oracle_matvec_q8(raw, np.ascontiguousarray(X[n * K:(n + 1) * K]), M, K) for n in range(N)])
    assert_close(yb.array.reshape(N, M), want)


@pytest.mark.parametrize("kind,slots", [("wide", "14"), ("ws", "28")])
def test_matmul_q8_prefill_gemm_round_split(gpu, monkeypatch, kind, slots):
    """The prefill GEMM's round split on a 256 x 2048 x 1792 product: the wide
    form's 16 tiles (128 x 256) at 14 workgroup slots, and the 128 x 128
    form's 32 tiles at 28 slots, run one full round plus 2 (4) leftover tiles
    whose K is split 7 ways (8 Q8_0 blocks each), partial tiles summed in
    order by k_tile_reduce. Against the oracle, and against the unsplit
    launch (default slots) within fp32 reassociation."""
    N, M, K = 256, 2048, 1792
    rng = np.random.default_rng(31)
    X = rng.standard_normal(N * K).astype(np.float32)
    raw = q8_matrix(rng, M, K, sigma=1.0)
    xb, wb = gpu.buf(X), gpu.buf(raw)
    ys = gpu.buf(np.zeros(N * M, np.float32))
    if kind == "ws":
        monkeypatch.setenv("SURGE_GEMM_WIDE", "0")
    monkeypatch.setenv("SURGE_GEMM_SLOTS", slots)
    gpu.run_op("k_matmul_q8", xb, wb, ys, [N, M, K])
    monkeypatch.delenv("SURGE_GEMM_SLOTS")
    yu = gpu.buf(np.zeros(N * M, np.float32))
    gpu.run_op("k_matmul_q8", xb, wb, yu, [N, M, K])
    rows = [0, 1, 127, 128, 255]
    want = np.stack([oracle_matvec_q8(raw, np.ascontiguousarray(X[n * K:(n + 1) * K]), M, K) for n in rows])
    got = ys.array.reshape(N, M)
    assert_close(got[rows], want)
    unsplit = yu.array.reshape(N, M)
    assert np.abs(got - unsplit).max() <= 1e-5 * np.abs(unsplit).max()


# ---------------------------------------------------------------- prefill chunk hooks

def test_conv1d_chunk_threads_state(gpu):
    rng = np.random.default_rng(21)
    ch, ks, n = 2048, 4, 9
    x = rng.standard_normal(n * ch).astype(np.float32)
    w = rng.standard_normal(ch * ks).astype(np.float32)
    st0 = rng.standard_normal((ks - 1) * ch).astype(np.float32)
    xb, wb, ob, sb = gpu.buf(x), gpu.buf(w), gpu.buf(np.zeros(n * ch, np.float32)), gpu.buf(st0.copy())
    gpu.run4("conv1d_chunk", xb, wb, ob, sb, [ch, ks, n])
    st = st0.copy()
    want = np.zeros(n * ch, np.float32)
    for t in range(n):
        xt = x[t * ch:(t + 1) * ch].copy()
        O.oracle().sg_ref_conv1d_causal(fp(xt), fp(w), fp(st), fp(st), ch, ks)
        want[t * ch:(t + 1) * ch] = xt
    assert_close(ob.array, want)
    assert np.array_equal(sb.array, st)


def test_delta_gates_chunk(gpu):
    rng = np.random.default_rng(22)
    n, nt = 48, 5
    a = rng.standard_normal(n * nt).astype(np.float32)
    b = rng.standard_normal(n * nt).astype(np.float32)
    adt = np.concatenate([-np.exp(rng.uniform(-1, 1, n)), rng.uniform(-0.5, 0.5, n)]).astype(np.float32)
    ab, bb, gb, db = gpu.buf(a), gpu.buf(b), gpu.buf(np.zeros(2 * n * nt, np.float32)), gpu.buf(adt)
    gpu.run4("delta_gates_chunk", ab, bb, gb, db, [n, 1, nt])
    got = gb.array.reshape(nt, 2, n)
    for z in range(nt):
        for h in range(n):
            i = z * n + h
            beta = O.oracle().sg_ref_sigmoid(float(b[i]))
            decay = O.oracle().sg_ref_delta_decay_neg_a(float(adt[h]), float(a[i]), float(adt[n + h]))
            assert abs(got[z, 0, h] - beta) <= 1e-6 and abs(got[z, 1, h] - decay) <= 1e-5 * max(decay, 1e-30) + 1e-7


def test_delta_chunk_scan_matches_token_loop(gpu):
    rng = np.random.default_rng(23)
    nv, nk, dk, dv, nt = 6, 2, 128, 64, 7
    kd = nk * dk
    cd = 2 * kd + nv * dv
    S0 = (rng.standard_normal(nv * dv * dk) * 0.1).astype(np.float32)
    qkv = (rng.standard_normal(nt * cd) * 0.1).astype(np.float32)
    gates = np.concatenate([rng.uniform(0, 1, (nt, nv)), rng.uniform(0.5, 1, (nt, nv))], axis=1).astype(np.float32)
    Sg, qb, ob, gb = gpu.buf(S0.copy()), gpu.buf(qkv), gpu.buf(np.zeros(nt * nv * dv, np.float32)), gpu.buf(gates)
    gpu.run4("delta_chunk", Sg, qb, ob, gb, [dk, dv, nv, nk, kd, 1, nt, cd])
    So, want = S0.copy(), np.zeros(nt * nv * dv, np.float32)
    for z in range(nt):
        row = qkv[z * cd:(z + 1) * cd]
        for h in range(nv):
            hk = h % nk
            O.oracle().sg_ref_delta_step(fp(So[h * dv * dk:]), fp(np.ascontiguousarray(row[hk * dk:])),
                                         fp(np.ascontiguousarray(row[kd + hk * dk:])),
                                         fp(np.ascontiguousarray(row[2 * kd + h * dv:])), float(gates[z, h]),
                                         float(gates[z, nv + h]), fp(want[(z * nv + h) * dv:]), dk, dv)
    assert_close(ob.array, want)
    assert_close(Sg.array, So)


def _delta_chunk_case(gpu, nv, nk, dk, dv, nt, seed, gate_lo=None):
    """Normalised q, k (|k| = 1, |q| = 1/sqrt(dk), as the layer's q/k norm
    leaves them), v N(0, 1), S N(0, 0.1), beta = sigmoid(N(0, 1)), decay =
    exp(-softplus(N(0, 1))) (BASELINE's gates; gate_lo instead draws decays
    in [gate_lo, 1e-3] to reach products far below fp32's range). Returns
    (GPU out, GPU S, oracle out, oracle S) from sg_gpu_run_delta_chunk and
    ref.c's delta step token by token."""
    rng = np.random.default_rng(seed)
    kd = nk * dk
    cd = 2 * kd + nv * dv
    qkv = rng.standard_normal((nt, cd)).astype(np.float32)
    for z in range(nt):
        for hk in range(nk):
            q = qkv[z, hk * dk:(hk + 1) * dk]
            k = qkv[z, kd + hk * dk:kd + (hk + 1) * dk]
            q *= 1.0 / (np.linalg.norm(q) * np.sqrt(dk))
            k *= 1.0 / np.linalg.norm(k)
    qkv = qkv.reshape(-1)
    S0 = (rng.standard_normal(nv * dv * dk) * 0.1).astype(np.float32)
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((nt, nv))))
    if gate_lo is None:
        x = rng.standard_normal((nt, nv))
        decay = np.exp(-(np.maximum(x, 0) + np.log1p(np.exp(-np.abs(x)))))
    else:
        decay = np.exp(rng.uniform(np.log(gate_lo), np.log(1e-3), (nt, nv)))
    gates = np.concatenate([beta, decay], axis=1).astype(np.float32)
    Sg, qb, ob, gb = gpu.buf(S0.copy()), gpu.buf(qkv), gpu.buf(np.zeros(nt * nv * dv, np.float32)), gpu.buf(gates)
    gpu.run4("delta_chunk", Sg, qb, ob, gb, [dk, dv, nv, nk, kd, 1, nt, cd])
    So, want = S0.copy(), np.zeros(nt * nv * dv, np.float32)
    for z in range(nt):
        row = qkv[z * cd:(z + 1) * cd]
        for h in range(nv):
            hk = h % nk
            O.oracle().sg_ref_delta_step(fp(So[h * dv * dk:]), fp(np.ascontiguousarray(row[hk * dk:])),
                                         fp(np.ascontiguousarray(row[kd + hk * dk:])),
                                         fp(np.ascontiguousarray(row[2 * kd + h * dv:])), float(gates[z, h]),
                                         float(gates[z, nv + h]), fp(want[(z * nv + h) * dv:]), dk, dv)
    return ob.array, Sg.array, want, So


@pytest.mark.parametrize("scan", ["mfma", "seq"])
@pytest.mark.parametrize("nv,nk,dk,dv,nt", [(16, 16, 128, 128, 200), (48, 16, 128, 128, 130), (8, 4, 64, 64, 257)],
                         ids=["baseline16x128", "27b-tiled48over16", "dk64"])
def test_delta_chunk_chunked_form_vs_sequential_oracle(gpu, monkeypatch, scan, nv, nk, dk, dv, nt):
    """The prefill scan over many 16-token blocks and a partial one: the
    chunked form on the matrix cores (SURGE_DELTA_SCAN=mfma, the default) and
    the sequential scan (=seq) against ref.c's delta step token by token, at the BASELINE
    DeltaNet shape (16 heads x 128^2), the 27B's 48 value heads tiled over 16
    key heads, and dk = dv = 64; readouts and the final state within the 1e-3
    bar."""
    monkeypatch.setenv("SURGE_DELTA_SCAN", scan)
    got, Sgot, want, Swant = _delta_chunk_case(gpu, nv, nk, dk, dv, nt, seed=31 + nt)
    assert_close(got, want)
    assert_close(Sgot, Swant)


def test_delta_chunk_chunked_form_tiny_decays(gpu, monkeypatch):
    """Decays down to 1e-30 per token: the chunked form's decay products
    (plain products over a 16-token block) underflow to exact zeros instead
    of NaN, as the token loop's do."""
    monkeypatch.setenv("SURGE_DELTA_SCAN", "mfma")
    got, Sgot, want, Swant = _delta_chunk_case(gpu, 8, 4, 128, 128, 150, seed=77, gate_lo=1e-30)
    assert np.isfinite(got).all() and np.isfinite(Sgot).all()
    assert_close(got, want)
    assert_close(Sgot, Swant)


def test_rmsnorm_gated_chunk(gpu):
    rng = np.random.default_rng(24)
    dv, nh, nt = 128, 6, 3
    y = rng.standard_normal(nt * nh * dv).astype(np.float32)
    z = rng.standard_normal(nt * nh * dv).astype(np.float32)
    w = rng.standard_normal(dv).astype(np.float32)
    yb, zb, ob, wb = gpu.buf(y), gpu.buf(z), gpu.buf(np.zeros(nt * nh * dv, np.float32)), gpu.buf(w)
    gpu.run4("rmsnorm_gated_chunk", yb, zb, ob, wb, [dv, nh, S.fbits(1e-6), nt])
    want = np.zeros_like(y)
    for i in range(nt * nh):
        yy, zz = y[i * dv:(i + 1) * dv].copy(), z[i * dv:(i + 1) * dv].copy()
        O.oracle().sg_ref_rmsnorm(fp(yy), fp(w), dv, 1e-6)
        O.oracle().sg_ref_swiglu(fp(zz), fp(yy), dv)
        want[i * dv:(i + 1) * dv] = zz
    assert_close(ob.array, want)


ATTN_CHUNK_CASES = [(24, 4, 256, 64, 1000, 150), (8, 2, 256, 64, 0, 130), (12, 4, 128, 32, 300, 70),
                    (16, 4, 128, 128, 600, 64), (8, 2, 64, 32, 200, 70),
                    (12, 4, 128, 32, 1100, 70), (8, 2, 64, 32, 1100, 40)]


@pytest.mark.parametrize("nh,nkv,hd,rd,base,n", ATTN_CHUNK_CASES,
                         ids=[f"{a}q{b}kv-hd{c}-rope{d}-base{e}-n{f}" for a, b, c, d, e, f in ATTN_CHUNK_CASES])
def test_attn_prefill_chunk_vs_oracle(gpu, nh, nkv, hd, rd, base, n):
    """The prefill path's attention layer core (sg_gpu_run_attn_chunk:
    k_attn_prep's q_norm / k_norm, partial RoPE from the position table and
    f16 K/V store, then the flash pass with its key split and combine and
    the sigmoid output gate) against ref.c's attention mixer composed from
    the oracle token by token (RMSNorm with weight, RoPE in double, K/V
    rounded to f16, decode attention over keys 0..position, gate): the 27B's
    24q/4kv/256 with rope 64 deep enough for a 3-way key split, the 2B's
    8q/2kv/256 from position 0, an odd GQA group (12/4, one query head per
    workgroup) at head_dim 128 / rope 32, a full rope, and head_dim 64 with
    rope 32 (8q/2kv); the odd group and head_dim 64 again deep enough for a
    3-way key split. Outputs within
    1e-3; V stored bit-exact (both round the same f32); K within one f16
    ulp of the oracle's (its f32 before rounding differs in the last bits);
    the keys before the chunk untouched."""
    rng = np.random.default_rng(nh + hd + base + n)
    row = 2 * nh * hd + 2 * nkv * hd
    theta, eps = 1e7, 1e-6
    cap = base + n
    inp = rng.standard_normal((n, row)).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(2 * hd)).astype(np.float32)
    K = np.zeros((cap, nkv, hd), np.float16)
    V = np.zeros((cap, nkv, hd), np.float16)
    K[:base] = rng.standard_normal((base, nkv, hd))
    V[:base] = rng.standard_normal((base, nkv, hd))
    kvb = gpu.buf(np.concatenate([K.reshape(-1), V.reshape(-1)]).view(np.uint16))
    ib, wb = gpu.buf(inp.reshape(-1)), gpu.buf(w)
    ob = gpu.buf(np.zeros(n * nh * hd, np.float32))
    gpu.attn_chunk(ib, wb, kvb, ob, [nh, nkv, hd, rd, base, n, S.fbits(theta), S.fbits(eps)])
    got_kv = kvb.array.view(np.float16).reshape(2, cap, nkv, hd)
    o = O.oracle()
    Ko, Vo = K.astype(np.float32), V.astype(np.float32)
    Kr = K.copy()
    want = np.zeros((n, nh * hd), np.float32)
    sc = np.float32(1.0 / np.sqrt(hd))
    for z in range(n):
        pos = base + z
        r = inp[z]
        q = r[:2 * nh * hd].copy()
        for h in range(nh):
            seg = np.ascontiguousarray(q[2 * h * hd:2 * h * hd + hd])
            o.sg_ref_rmsnorm(fp(seg), fp(np.ascontiguousarray(w[:hd])), hd, eps)
            o.sg_ref_rope_partial(fp(seg), hd, rd, pos, theta)
            q[2 * h * hd:2 * h * hd + hd] = seg
        for kh in range(nkv):
            k = np.ascontiguousarray(r[2 * nh * hd + kh * hd:2 * nh * hd + (kh + 1) * hd])
            o.sg_ref_rmsnorm(fp(k), fp(np.ascontiguousarray(w[hd:])), hd, eps)
            o.sg_ref_rope_partial(fp(k), hd, rd, pos, theta)
            Kr[pos, kh] = k.astype(np.float16)
            Ko[pos, kh] = k
            v = r[2 * nh * hd + (nkv + kh) * hd:2 * nh * hd + (nkv + kh + 1) * hd]
            Vo[pos, kh] = v.astype(np.float16).astype(np.float32)
        kc = Kr.astype(np.float32).reshape(-1)
        out = np.zeros(nh * hd, np.float32)
        o.sg_ref_attn_decode(fp(q), fp(kc), fp(np.ascontiguousarray(Vo.reshape(-1))), nh, nkv, hd, pos + 1,
                             2 * hd, sc, fp(out))
        for h in range(nh):
            oh = np.ascontiguousarray(out[h * hd:(h + 1) * hd])
            o.sg_ref_gate_sigmoid(fp(oh), fp(np.ascontiguousarray(q[2 * h * hd + hd:2 * (h + 1) * hd])), hd)
            want[z, h * hd:(h + 1) * hd] = oh
    assert_close(ob.array, want.reshape(-1))
    assert np.array_equal(got_kv[1, base:].view(np.uint16), Vo[base:].astype(np.float16).view(np.uint16))
    assert np.array_equal(got_kv[0, :base].view(np.uint16), K[:base].view(np.uint16))
    assert np.array_equal(got_kv[1, :base].view(np.uint16), V[:base].view(np.uint16))
    ulp = np.spacing(np.abs(Ko[base:]).astype(np.float16)).astype(np.float32)
    assert (np.abs(got_kv[0, base:].astype(np.float32) - Ko[base:]) <= ulp).all()


def test_attn_chunk_rejects_bad_shapes(gpu):
    """n_heads not a multiple of n_kv, head_dim 96, odd or oversize rope, an
    empty chunk, a chunk longer than its input rows, the cache aliasing the
    input rows."""
    b = gpu.buf(np.zeros(1 << 16, np.float32))
    kv = gpu.buf(np.zeros(1 << 16, np.float32))
    o = gpu.buf(np.zeros(1 << 14, np.float32))
    th, ep = S.fbits(1e7), S.fbits(1e-6)
    for p in ([6, 4, 64, 16, 0, 4], [8, 2, 96, 16, 0, 4], [8, 2, 64, 15, 0, 4], [8, 2, 64, 128, 0, 4],
              [8, 2, 64, 16, 0, 0], [8, 2, 64, 16, 0, 1000]):
        with pytest.raises(S.SurgeError):
            gpu.attn_chunk(b, b, kv, o, p + [th, ep])
    with pytest.raises(S.SurgeError):
        gpu.attn_chunk(b, kv, b, o, [8, 2, 64, 16, 0, 4, th, ep])


@pytest.mark.parametrize("base,n", [(0, 5), (37, 16), (2000, 9)])
def test_attn_prefill_causal(gpu, base, n):
    """Token t of the chunk (position base+t) attends over keys 0..base+t only."""
    rng = np.random.default_rng(base + n)
    nh, nkv, hd = 24, 4, 256
    qs = 2 * hd
    tot = base + n
    q = rng.standard_normal(n * nh * qs).astype(np.float32)
    k16, v16 = f16(rng, tot * nkv * hd), f16(rng, tot * nkv * hd)
    qb, kb, vb = gpu.buf(q), gpu.buf(k16.view(np.uint16)), gpu.buf(v16.view(np.uint16))
    ob = gpu.buf(np.zeros(n * nh * hd, np.float32))
    gpu.run4("attn_prefill", qb, kb, vb, ob, [nh, nkv, hd, base, n, qs, S.fbits(1 / 16)])
    kc, vc = k16.astype(np.float32), v16.astype(np.float32)
    for t in range(n):
        want = np.zeros(nh * hd, np.float32)
        O.oracle().sg_ref_attn_decode(fp(np.ascontiguousarray(q[t * nh * qs:(t + 1) * nh * qs])), fp(kc), fp(vc),
                                      nh, nkv, hd, base + t + 1, qs, np.float32(1 / 16), fp(want))
        assert_close(ob.array[t * nh * hd:(t + 1) * nh * hd], want)
