"""bench.py - decode throughput of the 27B-shape Q8_0 hybrid on one MI355X.

Workload (BASELINE.json metric and configs[4]): random-init 27B-shaped qwen35
hybrid, Q8_0 weights (hidden 5120, 64 layers, 3 DeltaNet : 1 attention,
attention 24q/4kv x 256, DeltaNet 48 v-heads / 16 k-heads x 128, FFN 17408,
vocab 151936). The context is filled with 4096 random token ids through
sg_gpu_prefill (512-token chunks, MFMA GEMMs); then W untimed and K timed greedy decode steps run
device-resident (sg_gpu_decode_greedy: one captured HIP graph per token, the
argmax feeds the next step on the device). One step = one token at batch 1.

Also reported, measured in this run:
  roofline     the dominant kernel (the fused gate/up Q8_0 GEMV with its
               RMSNorm prologue and SwiGLU epilogue, one launch per layer):
               algorithmic bytes / average launch time, timed with HIP events
               on the library's stream over all 64 layers' launches;
  decode_hbm   the whole decode step's algorithmic bytes per token (weights +
               KV + DeltaNet state + conv state) / time per token;
  cpu_baseline the reference's own CPU path (oracle/_ref, scalar, double; else
               this repository's oracle) timed on this host on a bounded
               sample of the same workload and composed to one token.

Prints one JSON line. --gpus N > 1 exits: this build measures one GPU.
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import surge_amd as S  # noqa: E402

HBM_PEAK_GBS = 8000.0
METRIC = "decode tok/s (27B-shape Q8_0, bs=1, 4k ctx); Q8_0 GEMV HBM GB/s vs peak"


def q8_bytes(rows, cols):
    return rows * cols // 32 * 34


def step_bytes(cfg, ctx):
    """Algorithmic HBM bytes of one decode token at `ctx` keys."""
    H, F, V = cfg["hidden"], cfg["ffn_hidden"], cfg["vocab"]
    hd, nh, nkv = cfg["head_dim"], cfg["n_heads"], cfg["n_kv_heads"]
    nk, nv, dk, dv = cfg["n_k_heads"], cfg["n_v_heads"], cfg["head_k_dim"], cfg["head_v_dim"]
    kd, vd = nk * dk, nv * dv
    conv = 2 * kd + vd
    n_attn = cfg["n_layers"] // cfg["full_attn_interval"]
    n_gdn = cfg["n_layers"] - n_attn
    w = cfg["n_layers"] * 3 * q8_bytes(F, H)
    w += n_attn * (q8_bytes(2 * nh * hd + 2 * nkv * hd, H) + q8_bytes(H, nh * hd))
    w += n_gdn * (q8_bytes(conv + vd + 2 * nv, H) + q8_bytes(H, vd))
    w += q8_bytes(V, H) * (1 if cfg["tied_embeddings"] else 1)   # lm_head (+1 embedding row, negligible)
    kv = n_attn * 2 * ctx * nkv * hd * 2
    state = n_gdn * 2 * nv * dv * dk * 4
    convb = n_gdn * 4 * conv * 4
    return w + kv + state + convb, dict(weights=w, kv=kv, deltanet_state=state, conv=convb)


class HipEvents:
    """hipEvent timing on a given stream (libamdhip64 through ctypes)."""

    def __init__(self):
        self.h = C.CDLL("libamdhip64.so")
        for f in ("hipEventCreate", "hipEventRecord", "hipEventSynchronize", "hipEventElapsedTime",
                  "hipEventDestroy"):
            getattr(self.h, f).restype = C.c_int

    def event(self):
        e = C.c_void_p()
        assert self.h.hipEventCreate(C.byref(e)) == 0
        return e

    def record(self, e, stream):
        assert self.h.hipEventRecord(e, C.c_void_p(stream)) == 0

    def ms(self, a, b):
        assert self.h.hipEventSynchronize(b) == 0
        t = C.c_float()
        assert self.h.hipEventElapsedTime(C.byref(t), a, b) == 0
        return t.value


def gemv_roofline(gpu, cfg, reps=3):
    """Average duration of the gate/up GEMV over every layer's launch."""
    ev = HipEvents()
    a, b = ev.event(), ev.event()
    L = cfg["n_layers"]
    for layer in range(L):                     # warm the code path
        gpu.enqueue_gemv(layer, 2)
    gpu.sync()
    ev.record(a, gpu.stream())
    for _ in range(reps):
        for layer in range(L):
            gpu.enqueue_gemv(layer, 2)
    ev.record(b, gpu.stream())
    avg_s = ev.ms(a, b) / 1e3 / (reps * L)
    rows, cols = 2 * cfg["ffn_hidden"], cfg["hidden"]
    algo = q8_bytes(rows, cols) + 2 * cols * 4 + (rows // 2) * 4
    gbs = algo / avg_s / 1e9
    return dict(bound="hbm", achieved=round(gbs, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                frac=round(gbs / HBM_PEAK_GBS, 4), traffic=None,
                kernel="k_gemv_ring gate|up %dx%d (RMSNorm prologue, SwiGLU epilogue)" % (rows, cols),
                avg_us=round(avg_s * 1e6, 2), algo_bytes=int(algo), launches=reps * L)


def decode_floor(gpu, ctx, reps=20):
    """The sequential-launch floor of this decode token (sg_gpu_time_floor):
    its launch sequence captured in one HIP graph with every kernel replaced
    by a plain streaming read of that kernel's algorithmic bytes, and by an
    empty kernel. What kernels run one after another cannot beat. With
    SURGE_HIP_GRAPH=0 (the decode launched kernel by kernel, as under a kernel
    trace) the reads are launched one by one too, so a trace of the run pairs
    each decode kernel with the read of its bytes."""
    if os.environ.get("SURGE_HIP_GRAPH") == "0":
        rd_us, n, nb = gpu.time_floor(ctx, 2, reps)
        return dict(kernels=n, bytes_per_token=int(nb), launch="one by one (SURGE_HIP_GRAPH=0)",
                    plain_read_us_per_token=round(rd_us, 1), plain_read_tok_s=round(1e6 / rd_us, 2), reps=reps)
    rd_us, n, nb = gpu.time_floor(ctx, 1, reps)
    em_us, _, _ = gpu.time_floor(ctx, 0, reps)
    return dict(kernels=n, bytes_per_token=int(nb), launch="one captured graph", plain_read_us_per_token=round(rd_us, 1),
                plain_read_tok_s=round(1e6 / rd_us, 2), plain_read_frac=round(nb / rd_us / 1e3 / HBM_PEAK_GBS, 4),
                empty_us_per_token=round(em_us, 1), reps=reps)


def calib_copy(nbytes):
    """One plain device-to-device copy of known size: rocprofv3 counter runs
    scale the GEMV's FETCH_SIZE/WRITE_SIZE by what the copy kernel reads."""
    h = C.CDLL("libamdhip64.so")
    a, b = C.c_void_p(), C.c_void_p()
    assert h.hipMalloc(C.byref(a), C.c_size_t(nbytes)) == 0 and h.hipMalloc(C.byref(b), C.c_size_t(nbytes)) == 0
    assert h.hipMemcpy(b, a, C.c_size_t(nbytes), 3) == 0          # hipMemcpyDeviceToDevice
    assert h.hipDeviceSynchronize() == 0
    h.hipFree(a)
    h.hipFree(b)


def measured_traffic(kernel_prefix):
    """HBM bytes per gate/up GEMV launch from the committed rocprofv3 counter
    summary (profiles/gemv_gate_up_traffic.json: FETCH_SIZE + WRITE_SIZE per
    dispatch, calibrated against a plain copy kernel). None when the file is
    absent, names another kernel, or was measured on another build (its
    kernels_sha256 is not the sha256 of this tree's kernels.hip)."""
    from surge_amd.profile_summary import kernels_sha256
    path = os.path.join(ROOT, "profiles", "gemv_gate_up_traffic.json")
    if not os.path.exists(path):
        return None
    try:
        d = json.load(open(path))
        if d.get("kernels_sha256") != kernels_sha256() or not d["kernel"].startswith(kernel_prefix):
            return None
        return int(d["bytes_per_dispatch"])
    except (ValueError, KeyError):
        return None


def cpu_baseline(syn, cfg, ctx, budget_s=15.0):
    """Reference CPU path on this host: per-op timings at the real shapes,
    composed to one decode token (a full scalar token takes tens of seconds)."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    kind = "reference" if O.ref_available() else "port"
    Lb = O.ref() if kind == "reference" else O.oracle()
    if kind == "port":
        Lb.sg_ref_set_threads(1)
    m = syn.model.contents
    H, F = cfg["hidden"], cfg["ffn_hidden"]
    x = np.random.default_rng(0).standard_normal(max(H, F)).astype(np.float32)
    y = np.zeros(max(F, cfg["vocab"]), np.float32)
    fp = lambda a: a.ctypes.data_as(C.POINTER(C.c_float))
    # 1. Q8_0 matvec throughput over the real gate_proj matrices of successive layers
    done_w, t0, li = 0, time.perf_counter(), 0
    while time.perf_counter() - t0 < budget_s * 0.7 and li < cfg["n_layers"]:
        Lb.sg_ref_matvec_q8(m.layers[li].gate_proj, fp(x), fp(y), F, H)
        done_w += F * H
        li += 1
    mv_s = time.perf_counter() - t0
    rate = done_w / mv_s
    total_w = 0
    n_attn = cfg["n_layers"] // cfg["full_attn_interval"]
    n_gdn = cfg["n_layers"] - n_attn
    nh, nkv, hd = cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"]
    vd = cfg["n_v_heads"] * cfg["head_v_dim"]
    conv = 2 * cfg["n_k_heads"] * cfg["head_k_dim"] + vd
    total_w += cfg["n_layers"] * 3 * F * H
    total_w += n_attn * ((2 * nh * hd + 2 * nkv * hd) * H + H * nh * hd)
    total_w += n_gdn * ((conv + vd + 2 * cfg["n_v_heads"]) * H + H * vd)
    total_w += cfg["vocab"] * H
    # 2. attention over ctx keys for one layer (all heads), the reference's direct decode
    rng = np.random.default_rng(1)
    q = rng.standard_normal(nh * 2 * hd).astype(np.float32)
    kc = rng.standard_normal(ctx * nkv * hd).astype(np.float32)
    vc = rng.standard_normal(ctx * nkv * hd).astype(np.float32)
    out = np.zeros(nh * hd, np.float32)
    t1 = time.perf_counter()
    Lb.sg_ref_attn_decode(fp(q), fp(kc), fp(vc), nh, nkv, hd, ctx, 2 * hd, 1 / 16, fp(out))
    att_s = time.perf_counter() - t1
    # 3. one DeltaNet layer's delta rule (all value heads)
    dk, dv, nv = cfg["head_k_dim"], cfg["head_v_dim"], cfg["n_v_heads"]
    Sm = (rng.standard_normal(dv * dk) * 0.1).astype(np.float32)
    qq, kk, vv = (rng.standard_normal(dk).astype(np.float32) * 0.1 for _ in range(3))
    yy = np.zeros(dv, np.float32)
    t2 = time.perf_counter()
    for _ in range(nv):
        Lb.sg_ref_delta_step(fp(Sm), fp(qq), fp(kk), fp(vv), 0.5, 0.9, fp(yy), dk, dv)
    dn_s = time.perf_counter() - t2
    tok_s = total_w / rate + n_attn * att_s + n_gdn * dn_s
    return dict(value=round(1.0 / tok_s, 5), unit="tok/s", cores=1, kind=kind,
                sample=("sg_ref_matvec_q8 over %d real 27B gate_proj matrices (%.2f Gweights, %.1f s) "
                        "+ sg_ref_attn_decode %dq/%dkv/%d at %d keys (one layer) + %d sg_ref_delta_step "
                        "128x128 (one layer), composed to one token: %.1f s/token"
                        % (li, done_w / 1e9, mv_s, nh, nkv, hd, ctx, nv, tok_s)),
                seconds_per_token=round(tok_s, 2), nproc=os.cpu_count())


def secondary_2b(steps=64, ctx=128, cpu=True, cpu_positions=4):
    """BASELINE's 2B configuration beside the headline: random-init 2B-shaped
    Q8_0 hybrid, a 128-token random-id prompt prefilled, then greedy decode on
    the GPU (device-resident, one HIP graph per token), tok/s over `steps`
    steps; and the reference's own ref.c (oracle/_ref; else this repository's
    oracle) timed on this host over the first `cpu_positions` positions of the
    same prompt, one thread, scaled to tok/s (the whole 128 + 64 run would take
    minutes of scalar CPU time)."""
    cfg = S.CFG_2B
    syn = S.Synth(cfg, S.SG_T_Q8_0, seed=0)
    gpu = S.Gpu()
    gpu.load_model(syn.model)
    gpu.state_new(ctx + 8 + 2 * steps + 8)
    prompt = np.random.default_rng(0).integers(0, cfg["vocab"], ctx).astype(np.int32)
    lg = gpu.prefill(prompt, chunk=ctx)
    w = gpu.decode_greedy(int(np.argmax(lg)), ctx, 8)
    gpu.sync()
    t0 = time.perf_counter()
    gpu.decode_greedy(int(w[-1]), ctx + 8, steps)
    dt = time.perf_counter() - t0
    bytes_tok, _ = step_bytes(cfg, ctx + 8 + steps // 2)
    fl_us, fl_n, _ = gpu.time_floor(ctx + 8 + steps // 2, 1, 20)
    gpu.close()
    out = dict(workload="2B-shape qwen35 hybrid Q8_0 (hidden 2048, 24 layers, 8q/2kv x 256, DeltaNet 16/16 x 128, "
                        "FFN 6144, vocab 151936), greedy decode bs=1 after a 128-token prompt",
               value=round(steps / dt, 2), unit="tok/s", steps=steps, ms_per_step=round(dt * 1e3 / steps, 4),
               decode_hbm_frac=round(bytes_tok * steps / dt / 1e9 / HBM_PEAK_GBS, 4),
               plain_read_floor_tok_s=round(1e6 / fl_us, 1), floor_kernels=fl_n, cpu_baseline=None)
    if cpu:
        sys.path.insert(0, os.path.join(ROOT, "tests"))
        import oracle_lib as O
        kind = "reference" if O.ref_available() else "port"
        L = O.ref() if kind == "reference" else O.oracle()
        if kind == "port":
            L.sg_ref_set_threads(1)
        rm = O.RefModel(L, syn.model, cpu_positions + 1)
        t0 = time.perf_counter()
        for p in range(cpu_positions):
            rm.forward(int(prompt[p]), p)
        cs = (time.perf_counter() - t0) / cpu_positions
        rm.close()
        out["cpu_baseline"] = dict(value=round(1.0 / cs, 4), unit="tok/s", cores=1, kind=kind,
                                   sample=f"sg_ref_forward of the first {cpu_positions} prompt positions of the "
                                          f"same 2B model: {cs:.2f} s/token", nproc=os.cpu_count())
    syn.close()
    return out


def micro(reps_gpu=200, rotate=1 << 30):
    """The BASELINE per-kernel configs on the product kernels, seeded as
    BASELINE.json states them: GPU microseconds per launch with every timed
    launch reading a different copy of its inputs (copies spanning >= 1 GiB,
    so nothing is served from the 256 MB MALL) and cache resident (one copy),
    the algorithmic bytes and their GB/s, and beside each the reference's
    ref.c (oracle/_ref; else this repository's oracle) on this host, one
    thread, the median of several runs. One JSON line per unit."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    kind = "reference" if O.ref_available() else "port"
    R = O.ref() if kind == "reference" else O.oracle()
    if kind == "port":
        R.sg_ref_set_threads(1)
    fp = lambda a: a.ctypes.data_as(C.POINTER(C.c_float))

    def cpu_median(fn, budget_s=3.0, min_n=3, max_n=50):
        ts = []
        t_end = time.perf_counter() + budget_s
        while len(ts) < min_n or (len(ts) < max_n and time.perf_counter() < t_end):
            t = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t)
        return float(np.median(ts)) * 1e6, len(ts)

    def line(unit, algo, gpu_rot, gpu_hot, cpu_us, cpu_n, extra):
        d = {"unit": unit, "algo_bytes": int(algo),
             "gpu_us": round(gpu_rot, 3), "gpu_GBs": round(algo / gpu_rot / 1e3, 1),
             "frac": round(algo / gpu_rot / 1e3 / HBM_PEAK_GBS, 4),
             "gpu_us_cache_resident": round(gpu_hot, 3), "gpu_GBs_cache_resident": round(algo / gpu_hot / 1e3, 1),
             "rotate_bytes": rotate, "gpu_reps": reps_gpu,
             "cpu_us_median": round(cpu_us, 1), "cpu_GBs": round(algo / cpu_us / 1e3, 3), "cpu_runs": cpu_n,
             "cpu_kind": kind, "cpu_cores": 1, "nproc": os.cpu_count()}
        d.update(extra)
        print(json.dumps(d), flush=True)

    gpu = S.Gpu()
    # 1. Q8_0 GEMV 4096 x 4096: 32 int8 uniform in [-127, 127] + f16 scale |N(0, 0.02)| / 127, x N(0, 1)
    rng = np.random.default_rng(0)
    rows = cols = 4096
    nb = cols // 32
    qv = rng.integers(-127, 128, size=(rows, nb, 32), dtype=np.int8)
    dv = (np.abs(rng.standard_normal((rows, nb))) * 0.02 / 127).astype(np.float16)
    raw = np.zeros((rows, nb, 34), np.uint8)
    raw[:, :, :2] = dv.view(np.uint8).reshape(rows, nb, 2)
    raw[:, :, 2:] = qv.view(np.uint8)
    raw = raw.reshape(-1)
    x = rng.standard_normal(cols).astype(np.float32)
    wb, xb, yb = gpu.buf(raw), gpu.buf(x), gpu.buf(np.zeros(rows, np.float32))
    rot = gpu.time_matvec_q8(wb, xb, yb, rows, cols, rotate, reps_gpu)
    hot = gpu.time_matvec_q8(wb, xb, yb, rows, cols, 0, reps_gpu)
    y = np.zeros(rows, np.float32)
    cpu_us, n = cpu_median(lambda: R.sg_ref_matvec_q8(raw.ctypes.data, fp(x), fp(y), rows, cols))
    line("Q8_0 GEMV 4096x4096 (k_gemv_q8)", rows * nb * 34 + 4 * cols + 4 * rows, rot, hot, cpu_us, n,
         {"max_abs_diff_vs_cpu": float(np.abs(yb.array - y).max())})
    for b in (wb, xb, yb):
        b.free()
    # 2. split-K GQA decode attention 16 q / 4 kv x 256, f16 K/V N(0, 1), q N(0, 1), scale 1/16
    nh, nkv, hd = 16, 4, 256
    for seq in (512, 4096, 32768):
        ns = S.lib().sg_gpu_splitk_gqa_n_splits(seq)
        rng = np.random.default_rng(seq)
        q = rng.standard_normal(nh * hd).astype(np.float32)
        k16 = rng.standard_normal(seq * nkv * hd).astype(np.float16)
        v16 = rng.standard_normal(seq * nkv * hd).astype(np.float16)
        qb, kb, vb = gpu.buf(q), gpu.buf(k16.view(np.uint16)), gpu.buf(v16.view(np.uint16))
        ob = gpu.buf(np.zeros(nh * hd, np.float32))
        p = [nh, nkv, hd, seq, hd, S.fbits(1 / 16), ns]
        rp, rc = gpu.time_attn(qb, kb, vb, ob, p, rotate, reps_gpu)
        hp, hc = gpu.time_attn(qb, kb, vb, ob, p, 0, reps_gpu)
        kc, vc = k16.astype(np.float32), v16.astype(np.float32)
        out = np.zeros(nh * hd, np.float32)
        cpu_us, n = cpu_median(lambda: R.sg_ref_attn_decode_splitk(fp(q), fp(kc), fp(vc), nh, nkv, hd, seq, hd,
                                                                     np.float32(1 / 16), ns, fp(out)))
        algo = 4096 * seq + 2 * nh * hd * 4          # K + V f16, q and out f32
        line(f"split-K GQA attention 16q/4kv/256 at {seq} keys, {ns} splits (k_attn_partial_wv + k_attn_combine)",
             algo, rp + rc, hp + hc, cpu_us, n,
             {"gpu_us_partial": round(rp, 3), "gpu_us_combine": round(rc, 3),
              "partial_GBs": round(algo / rp / 1e3, 1), "max_abs_diff_vs_cpu": float(np.abs(ob.array - out).max())})
        for b in (qb, kb, vb, ob):
            b.free()
    # 3. Gated-DeltaNet step: 16 heads, dk = dv = 128, S N(0, 0.1) (rotated copies are seeded fills),
    #    conv width 4 (2048 channels per q / k / v: conv_dim 6144), gates from N(0, 1)
    nv = nk = 16
    dk = dvv = 128
    ks = 4
    cd, vd = 2 * nk * dk + nv * dvv, nv * dvv
    rng = np.random.default_rng(3)
    inp = rng.standard_normal(cd + vd + 2 * nv).astype(np.float32)
    w = np.concatenate([rng.standard_normal(cd * ks) * 0.5, -np.ones(nv), np.zeros(nv), np.ones(dvv)]).astype(np.float32)
    ib, wb, ob = gpu.buf(inp), gpu.buf(w), gpu.buf(np.zeros(vd, np.float32))
    p = [dk, dvv, nv, nk, ks, 1, 1, S.fbits(1e-6)]
    rot = gpu.time_gdn_step(ib, wb, ob, p, rotate, reps_gpu)
    hot = gpu.time_gdn_step(ib, wb, ob, p, 0, reps_gpu)
    Sm = (rng.standard_normal(nv * dvv * dk) * 0.1).astype(np.float32)
    conv_st = np.zeros((ks - 1) * cd, np.float32)
    qkv = inp[:cd].copy()
    yy = np.zeros(vd, np.float32)
    wconv = np.ascontiguousarray(w[:cd * ks])

    def cpu_step():
        xx = qkv.copy()
        R.sg_ref_conv1d_causal(fp(xx), fp(wconv), fp(conv_st), fp(conv_st), cd, ks)
        for h in range(nv):
            R.sg_ref_delta_step(fp(Sm[h * dvv * dk:]), fp(xx[h * dk:]), fp(xx[nk * dk + h * dk:]),
                                fp(xx[2 * nk * dk + h * dvv:]), 0.5, 0.9, fp(yy[h * dvv:]), dk, dvv)
    cpu_us, n = cpu_median(cpu_step)
    # S read + write, the conv ring's 4 slots read and one written, the projection rows, conv
    # weights, gates/norm, output
    algo = 2 * nv * dvv * dk * 4 + 5 * cd * 4 + (cd + vd + 2 * nv) * 4 + cd * ks * 4 + (2 * nv + dvv) * 4 + vd * 4
    line("Gated-DeltaNet step 16 heads x 128 x 128, conv 6144 channels (k_gdn_step: conv, norms, gates, "
         "rank-1 update, RMSNormGated)", algo, rot, hot, cpu_us, n,
         {"cpu_sample": "sg_ref_conv1d_causal over 6144 channels + 16 sg_ref_delta_step 128x128"})
    # 4. the floors under every decode kernel: a plain streaming read of the decode GEMVs' sizes
    #    (lm_head 826 MB, gate/up 190 MB, the output projection 33 MB) and an empty kernel
    for nb in (826 << 20, 190 << 20, 33 << 20):
        rot = gpu.time_read(nb, rotate, 50)
        hot = gpu.time_read(nb, 0, 50)
        print(json.dumps({"unit": f"plain streaming read of {nb >> 20} MiB (k_read, 1024 workgroups)",
                          "algo_bytes": nb, "gpu_us": round(rot, 3), "gpu_GBs": round(nb / rot / 1e3, 1),
                          "frac": round(nb / rot / 1e3 / HBM_PEAK_GBS, 4), "gpu_us_cache_resident": round(hot, 3),
                          "rotate_bytes": rotate, "gpu_reps": 50}), flush=True)
    eager, graph = gpu.time_empty(2000, False), gpu.time_empty(2000, True)
    print(json.dumps({"unit": "empty kernel launch (k_empty)", "gpu_us_per_launch_eager": round(eager, 3),
                      "gpu_us_per_launch_in_graph": round(graph, 3), "reps": 2000}), flush=True)
    gpu.close()


def gemv_shapes(reps=3):
    """Every decode GEMV shape of the 27B model timed per kernel variant:
    average microseconds per launch over back-to-back launches across the
    layers' distinct weight matrices (HIP events on the library stream), the
    kernel choice forced by SURGE_GEMV and the row-group override.
    One JSON line per (shape, variant)."""
    cfg = S.CFG_27B
    syn = S.Synth(cfg, S.SG_T_Q8_0, seed=0)
    gpu = S.Gpu()
    gpu.load_model(syn.model)
    gpu.state_new(64)
    ev = HipEvents()
    a, b = ev.event(), ev.event()
    L = cfg["n_layers"]
    shapes = {0: "input projection (DeltaNet 16480x5120)", 1: "output projection 5120x6144",
              2: "gate|up 34816x5120", 3: "down 5120x17408", 4: "lm_head 151936x5120"}
    variants = [("default", None, 0), ("k_gemv_q8 (SURGE_GEMV=q8)", "q8", 0), ("k_gemv_bal contiguous", "bal", 0),
                ("k_gemv_bal interleaved", "bali", 0), ("k_gemv_q8 R=1", None, 1), ("k_gemv_q8 R=4", None, 4)]
    for which, name in shapes.items():
        layers = [0] if which == 4 else [l for l in range(L) if (l + 1) % cfg["full_attn_interval"] != 0]
        n = 8 if which == 4 else reps
        for vname, env, tune in variants:
            if env:
                os.environ["SURGE_GEMV"] = env
            else:
                os.environ.pop("SURGE_GEMV", None)
            for l in layers:
                gpu.enqueue_gemv(l, which, tune)
            gpu.sync()
            ev.record(a, gpu.stream())
            for _ in range(n):
                for l in layers:
                    gpu.enqueue_gemv(l, which, tune)
            ev.record(b, gpu.stream())
            us = ev.ms(a, b) * 1e3 / (n * len(layers))
            print(json.dumps({"shape": name, "variant": vname, "us": round(us, 2), "launches": n * len(layers)}),
                  flush=True)
    os.environ.pop("SURGE_GEMV", None)
    gpu.close()
    syn.close()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--shape", default="27b", choices=["27b", "2b"])
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-2b", action="store_true", help="skip the 2B-shape line beside the 27B headline")
    ap.add_argument("--no-floor", action="store_true",
                    help="skip the sequential-launch floor (its 341 x 20 reads are slow under counter collection)")
    ap.add_argument("--chunk", type=int, default=512, help="prefill chunk (tokens)")
    ap.add_argument("--fill", action="store_true",
                    help="no prefill: seeded K/V and DeltaNet state up to --ctx (decode at depth)")
    ap.add_argument("--calib-mb", type=int, default=0,
                    help="also run one device-to-device copy of this many MiB (counter calibration)")
    ap.add_argument("--micro", action="store_true",
                    help="the per-kernel BASELINE configs instead (GEMV 4096^2, split-K attention at "
                         "512/4096/32768 keys, the 16-head DeltaNet step, plain-read and empty-launch "
                         "floors): one JSON line each")
    ap.add_argument("--gemv-shapes", action="store_true",
                    help="every 27B decode GEMV shape timed per kernel variant instead: one JSON line each")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {a.gpus}); this build has no "
              "multi-GPU path", file=sys.stderr)
        sys.exit(2)
    if a.micro:
        micro()
        return
    if a.gemv_shapes:
        gemv_shapes()
        return
    cfg = S.CFG_27B if a.shape == "27b" else S.CFG_2B
    log = lambda *x: print("[bench]", *x, file=sys.stderr, flush=True)
    t = time.time()
    syn = S.Synth(cfg, S.SG_T_Q8_0, seed=0)
    log(f"synthesised {a.shape} model: {syn.nbytes() / 1e9:.2f} GB in {time.time() - t:.1f} s")
    gpu = S.Gpu()
    t = time.time()
    gpu.load_model(syn.model)
    log(f"loaded to HBM in {time.time() - t:.1f} s ({gpu.alloc_bytes() / 1e9:.2f} GB allocated)")
    need = a.ctx + a.warmup + 2 * a.steps + 8
    if need > S.SG_KV_CAP_MAX:
        print(f"--ctx {a.ctx} with {a.warmup} + {a.steps} steps needs {need} positions; the cap is "
              f"{S.SG_KV_CAP_MAX}", file=sys.stderr)
        sys.exit(2)
    gpu.state_new(need)
    # the row's GEMM gate reading, taken before the run as the reference's
    # surge-bench takes it (cli_bench.c:346, 490): the prefill GEMM on layer
    # 0's gate/up weight for one 512-token chunk, useful flops / time
    gemm_us = gpu.time_gemm(0, 2, 512, 5)
    gemm_tflops = 2.0 * 512 * 2 * cfg["ffn_hidden"] * cfg["hidden"] / (gemm_us * 1e-6) / 1e12
    log(f"GEMM gate reading: gate/up {2 * cfg['ffn_hidden']}x{cfg['hidden']} over 512 tokens in {gemm_us:.1f} us "
        f"({gemm_tflops:.1f} TFLOP/s)")
    t = time.time()
    if a.fill:
        gpu.fill_synthetic(a.ctx, seed=0)
        pf_s = time.time() - t
        log(f"filled K/V and DeltaNet state to depth {a.ctx} in {pf_s:.2f} s (no prefill)")
        tok = 0
    else:
        prompt = np.random.default_rng(0).integers(0, cfg["vocab"], a.ctx).astype(np.int32)
        lg = gpu.prefill(prompt, chunk=a.chunk)
        gpu.sync()
        pf_s = time.time() - t
        log(f"prefilled {a.ctx} context tokens in {pf_s:.2f} s ({a.ctx / pf_s:.0f} tok/s, chunk {a.chunk})")
        tok = int(np.argmax(lg))
    pos = a.ctx
    if a.warmup:
        w = gpu.decode_greedy(tok, pos, a.warmup)
        tok, pos = int(w[-1]), pos + a.warmup
    gpu.sync()
    t0 = time.perf_counter()
    toks = gpu.decode_greedy(tok, pos, a.steps)       # ends with a stream synchronize
    dt = time.perf_counter() - t0
    tps = a.steps / dt
    log(f"decoded {a.steps} tokens in {dt * 1e3:.1f} ms: {tps:.1f} tok/s; first ids {toks[:8].tolist()}")
    bytes_tok, parts = step_bytes(cfg, a.ctx + a.warmup + a.steps // 2)
    decode_gbs = bytes_tok * tps / 1e9
    # surge-bench's decode-by-slope over per-token times (reference cli_bench.c:627-693):
    # K more greedy steps with a HIP event after each, fitted by sg_bench_slope
    t_slope = time.perf_counter()
    _, t_cum = gpu.decode_greedy_timed(int(toks[-1]), pos + a.steps, a.steps)
    slope_wall = time.perf_counter() - t_slope
    tc = np.ascontiguousarray(t_cum)
    warm = S.lib().sg_bench_default_warmup(a.steps)
    tcp = tc.ctypes.data_as(C.POINTER(C.c_double))
    slope = S.lib().sg_bench_slope(tcp, a.steps, warm)
    avg = S.lib().sg_bench_avg_tps(tcp, a.steps, warm)
    log(f"decode by slope over {a.steps} timed steps (warmup {warm}): {slope:.1f} tok/s (endpoint average {avg:.1f})")
    roof = gemv_roofline(gpu, cfg)
    if a.calib_mb:
        calib_copy(a.calib_mb << 20)
    roof["traffic"] = measured_traffic("k_gemv_ring<2, 1, 2>")
    log(f"gate/up GEMV: {roof['avg_us']} us/launch, {roof['achieved']} GB/s ({roof['frac'] * 100:.1f}% of peak)")
    floor = None
    if not a.no_floor:
        floor = decode_floor(gpu, a.ctx + a.warmup + a.steps // 2)
        log(f"sequential-launch floor ({floor['launch']}): {floor['kernels']} plain reads "
            f"{floor['plain_read_us_per_token']} us/token ({floor['plain_read_tok_s']} tok/s)"
            + (f", {floor['kernels']} empty kernels {floor['empty_us_per_token']} us" if "empty_us_per_token" in floor else ""))
    row = S.BenchRow()
    row.model = f"qwen35-{a.shape}-shape-q8_0-random".encode()
    row.engine = b"surge_amd (MI355X, HIP)"
    row.prefill_tps = -1.0 if a.fill else a.ctx / pf_s
    row.prefill_wall_s = pf_s
    row.prefill_compute_tps = row.prefill_tps
    row.prefill_segments = 0 if a.fill else S.lib().sg_gpu_prefill_segments(gpu.handle)
    row.decode_tps_slope, row.decode_tps_avg = slope, avg
    row.decode_wall_s = slope_wall
    row.decode_compute_tps = a.steps / slope_wall
    row.decode_rest_s = 0.0
    row.gpu_alloc_gib = gpu.alloc_bytes() / 2 ** 30
    row.peak_ram_gib = peak_rss_gib()
    row.n_prompt_tok, row.n_gen = a.ctx, a.steps
    row.wall_s = pf_s + dt + slope_wall
    row.gemm_tflops = gemm_tflops
    ok = C.c_bool(False)
    # the prompt's ids all went in (the fill sets the same depth without ids)
    S.lib().sg_bench_check_ingestion(a.ctx, need, a.ctx, a.ctx, C.byref(ok))
    row.ingestion_ok = ok.value and gpu.used() == pos + 2 * a.steps
    row.log_id = f"ctx{a.ctx}_{a.shape}_surge_amd".encode()
    S.lib().sg_bench_finalize_status(C.byref(row))
    gpu.close()
    cpu = None
    if not a.no_cpu:
        cpu = cpu_baseline(syn, cfg, a.ctx)
    sec = None
    if a.shape == "27b" and not a.no_2b:
        sec = secondary_2b(cpu=not a.no_cpu)
        log(f"2B shape: {sec['value']} tok/s"
            + (f", ref.c {sec['cpu_baseline']['value']} tok/s on one core" if sec["cpu_baseline"] else ""))
    if cpu:
        log(f"cpu baseline: {cpu['sample']}")
    syn.close()
    line = {
        "metric": METRIC, "value": round(tps, 3), "unit": "tok/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(dt * 1e3 / a.steps, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32 (int8 Q8_0 weights, f16 KV)",
        "data": "synthetic (seeded random-init weights, random token ids)",
        "config": {"workload": f"{a.shape.upper()}-shape qwen35 hybrid Q8_0, greedy decode bs=1 at "
                               f"{a.ctx}-token context (device-resident greedy loop, one HIP graph per token"
                               + ("; K/V and DeltaNet state filled with seeded values, no prefill)" if a.fill else ")"),
                   "ctx": a.ctx, "batch": 1, "model_bytes": syn_bytes_hint(cfg)},
        "decode_hbm": {"bytes_per_token": int(bytes_tok), "parts": parts,
                       "achieved_GBs": round(decode_gbs, 1), "frac": round(decode_gbs / HBM_PEAK_GBS, 4)},
        "prefill": ({"tokens": a.ctx, "synthetic_fill": True, "seconds": round(pf_s, 3)} if a.fill else
                    {"tokens": a.ctx, "chunk": a.chunk, "seconds": round(pf_s, 3),
                     "tok_per_s": round(a.ctx / pf_s, 1)}),
        "roofline": roof,
        "decode_floor": floor,
        "cpu_baseline": cpu,
        "secondary_2b": sec,
        "decode_by_slope": {"tok_s": round(slope, 3), "endpoint_avg_tok_s": round(avg, 3), "steps": a.steps,
                            "warmup": int(warm), "clock": "HIP events after each step"},
        "bench_row": {"md": row.md(), "json": json.loads(row.json())},
    }
    print(json.dumps(line), flush=True)


def peak_rss_gib():
    """The process's peak resident set (VmHWM), GiB."""
    try:
        for ln in open("/proc/self/status"):
            if ln.startswith("VmHWM:"):
                return int(ln.split()[1]) / 2 ** 20
    except OSError:
        pass
    return 0.0


def syn_bytes_hint(cfg):
    return step_bytes(cfg, 0)[1]["weights"]


if __name__ == "__main__":
    main()
