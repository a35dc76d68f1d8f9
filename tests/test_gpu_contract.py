"""GPU tests of the boundary's contract (no numerics beyond identity): the
decode-selection switches read at sg_gpu_state_new and the diagnostics that
report them (reference surge.h:1011-1050, 1179-1254; the checks follow
tests/test_gpu_fwd.c:1395-1500), the sg_kv module on the GPU backend that
sg_gpu_init registers (tests/test_gpu_mem.c:259-311), and the device argmax
against sg_argmax_f32 (src/greedy.c:17-27)."""
import ctypes as C

import numpy as np
import pytest

import surge_amd as S

pytestmark = pytest.mark.gpu

TINY = dict(n_layers=4, n_heads=4, n_kv_heads=2, head_dim=128, hidden=256, ffn_hidden=512,
            vocab=500, rope_theta=1e7, rms_eps=1e-6, tied_embeddings=False, rope_dim=64,
            full_attn_interval=4, n_k_heads=2, n_v_heads=4, head_k_dim=64, head_v_dim=64,
            conv_kernel=4, attn_output_gate=True)
SWITCHES = ("SURGE_KV_DTYPE", "SURGE_ATTN_SPLITK", "SURGE_ATTN_SPLITK_GQA", "SURGE_ATTN_SPLITK_ONLINE",
            "SURGE_SPLITK_GQA_CAP")


@pytest.fixture()
def tiny(gpu, monkeypatch):
    for k in SWITCHES:
        monkeypatch.delenv(k, raising=False)
    syn = S.Synth(TINY, S.SG_T_Q8_0, seed=3)
    gpu.load_model(syn.model)
    yield syn
    for k in SWITCHES:
        monkeypatch.delenv(k, raising=False)
    gpu.state_new(8)
    syn.close()


def test_delta_scan_switch_rejected_not_ignored(gpu, tiny, monkeypatch):
    """SURGE_DELTA_SCAN names the prefill DeltaNet scan's form: mfma (the
    default) or seq; a misspelt value is refused at sg_gpu_state_new and
    by the prefill and chunk entry points, not silently run as another form."""
    for bad in ("MFMA", "wy", "seq ", "sequential", "1"):
        monkeypatch.setenv("SURGE_DELTA_SCAN", bad)
        with pytest.raises(S.SurgeError, match="SURGE_DELTA_SCAN"):
            gpu.state_new(64)
    for good in ("mfma", "seq", ""):
        monkeypatch.setenv("SURGE_DELTA_SCAN", good)
        gpu.state_new(64)
    monkeypatch.setenv("SURGE_DELTA_SCAN", "Wy")
    with pytest.raises(S.SurgeError, match="SURGE_DELTA_SCAN"):
        gpu.prefill([1, 2, 3, 4], chunk=4)
    monkeypatch.delenv("SURGE_DELTA_SCAN")
    gpu.prefill([1, 2, 3, 4], chunk=4)


def test_online_switch_rejected_not_ignored(gpu, tiny, monkeypatch):
    """SURGE_ATTN_SPLITK_ONLINE takes exactly "0" or "1"; anything else is an
    error at sg_gpu_state_new (an ignored value would make its A/B vacuous)."""
    deep = 65536
    for bad in ("on", "true", "yes", "2", "-1", "01", "1 ", " 1", "00", "x"):
        monkeypatch.setenv("SURGE_ATTN_SPLITK_ONLINE", bad)
        with pytest.raises(S.SurgeError):
            gpu.state_new(64)
    monkeypatch.setenv("SURGE_ATTN_SPLITK_ONLINE", "0")
    gpu.state_new(64)
    assert not gpu.online_selected(24, 4, 256, deep) and not gpu.online_selected(32, 8, 128, deep)
    monkeypatch.setenv("SURGE_ATTN_SPLITK_ONLINE", "1")
    gpu.state_new(64)
    assert gpu.online_selected(24, 4, 256, deep) and gpu.online_selected(32, 8, 128, deep)
    # head_dim bound, GQA band
    for hd in (257, 512, 0):
        assert not gpu.online_selected(24, 4, hd, deep)
    for nh, nkv in ((8, 8), (18, 2), (32, 5), (32, 0)):
        assert not gpu.online_selected(nh, nkv, 128, deep)
    # mutual exclusion: with both switches on, the online arm takes the
    # state's shape and the GQA predicate answers false for it
    monkeypatch.setenv("SURGE_ATTN_SPLITK_GQA", "1")
    gpu.state_new(64)
    assert gpu.online_selected(4, 2, 128, deep)
    assert not gpu.gqa_selected(4, 2, deep)
    monkeypatch.setenv("SURGE_ATTN_SPLITK_ONLINE", "0")
    gpu.state_new(64)
    assert gpu.gqa_selected(4, 2, deep) and not gpu.online_selected(4, 2, 128, deep)
    # split-K off: neither arm
    monkeypatch.setenv("SURGE_ATTN_SPLITK", "0")
    gpu.state_new(64)
    assert not gpu.gqa_selected(4, 2, deep) and not gpu.online_selected(4, 2, 128, deep)


def test_warned_switches_keep_their_defaults(gpu, tiny, monkeypatch, capfd):
    """SURGE_ATTN_SPLITK, SURGE_ATTN_SPLITK_GQA and SURGE_KV_DTYPE warn on an
    unrecognised value and keep the default; SURGE_KV_DTYPE=f32 is refused
    because no f32 cache is built."""
    monkeypatch.setenv("SURGE_ATTN_SPLITK", "yes")
    monkeypatch.setenv("SURGE_ATTN_SPLITK_GQA", "on")
    monkeypatch.setenv("SURGE_KV_DTYPE", "bf16")
    gpu.state_new(64)
    err = capfd.readouterr().err
    assert "SURGE_ATTN_SPLITK='yes'" in err and "SURGE_ATTN_SPLITK_GQA='on'" in err and "SURGE_KV_DTYPE" in err
    assert gpu.gqa_selected(4, 2, 1000)
    gpu.forward(1, 0)
    assert gpu.dispatch_counts() == (0, 1, 0)
    monkeypatch.setenv("SURGE_KV_DTYPE", "f32")
    with pytest.raises(S.SurgeError, match="f32"):
        gpu.state_new(64)
    monkeypatch.setenv("SURGE_KV_DTYPE", "f16")
    gpu.state_new(64)


def test_counters_reset_at_state_new_and_skip_one_shots(gpu, tiny, monkeypatch):
    gpu.state_new(64)
    for p in range(5):
        gpu.forward(7, p)
    assert gpu.dispatch_counts() == (0, 5, 0)
    # a one-shot partial is not counted
    nh, nkv, hd, seq, ns = 4, 2, 128, 10, 2
    bufs = [gpu.buf(np.ones(nh * hd, np.float32)), gpu.buf(np.zeros(seq * nkv * hd, np.uint16)),
            gpu.buf(np.zeros(seq * nkv * hd, np.uint16)), gpu.buf(np.zeros(nh * ns, np.float32)),
            gpu.buf(np.zeros(nh * ns, np.float32)), gpu.buf(np.zeros(nh * ns * hd, np.float32))]
    gpu.attn_partial(*bufs, [nh, nkv, hd, seq, hd, S.fbits(0.1), ns])
    assert gpu.dispatch_counts() == (0, 5, 0)
    gpu.state_reset()                      # a reset keeps counting
    gpu.forward(7, 0)
    assert gpu.dispatch_counts() == (0, 6, 0)
    gpu.state_new(64)
    assert gpu.dispatch_counts() == (0, 0, 0)
    monkeypatch.setenv("SURGE_ATTN_SPLITK_GQA", "0")
    gpu.state_new(64)
    gpu.decode_greedy(3, 0, 4)
    assert gpu.dispatch_counts() == (4, 0, 0)


def test_kv_module_on_gpu_backend(gpu):
    """sg_gpu_init registers the GPU allocator as the sg_kv backend: a
    single-layer 8 kv heads x 128 f16 cache at 76800 positions is exactly
    300 MiB (sg_kv_bytes) and sg_gpu_current_alloc_bytes grows by at least
    90% of it (reference tests/test_gpu_mem.c:259-311); buffers are GPU
    handles with host mirrors; reset zeroes S through the mirror."""
    L = S.lib()
    c = S.make_cfg(n_layers=1, n_kv_heads=8, head_dim=128, full_attn_interval=1)
    budget = L.sg_kv_bytes(C.byref(c), 76800, 1)
    assert budget == 300 * 1024 * 1024
    before = gpu.alloc_bytes()
    kv = C.c_void_p()
    S.check(L.sg_kv_new(gpu.handle, C.byref(c), 76800, 1, C.byref(kv)))
    assert gpu.alloc_bytes() - before >= 0.9 * budget
    k0 = L.sg_kv_k(kv, 0)
    assert k0 and L.sg_gpu_buf_device(k0) and L.sg_gpu_buf_host(k0)
    L.sg_kv_free(kv)
    assert gpu.alloc_bytes() == before
    h = S.make_cfg(**TINY)
    S.check(L.sg_kv_new(gpu.handle, C.byref(h), 32, 1, C.byref(kv)))
    s0 = L.sg_gpu_buf_host(L.sg_kv_s(kv, 0))
    C.memset(s0, 0x7F, 256)
    L.sg_kv_reset(kv)
    assert not any((C.c_uint8 * 256).from_address(s0))
    L.sg_kv_free(kv)


def test_device_argmax_matches_host_rule(gpu):
    """The greedy loop's device argmax reproduces sg_argmax_f32 (strict '>'
    scanning upward from v[0]): ties to the lowest index, NaN never wins,
    a NaN at index 0 is never beaten, all -inf gives 0."""
    L = S.lib()
    rng = np.random.default_rng(5)
    n = 151936
    base = rng.standard_normal(n).astype(np.float32)
    cases = []
    v = base.copy(); v[[10, 99999, 150000]] = 9.0; cases.append(v)                 # tie
    v = base.copy(); v[0] = np.nan; cases.append(v)                                # NaN first
    v = base.copy(); v[[5, 77, 123456]] = np.nan; v[600] = 7.0; cases.append(v)    # NaN elsewhere
    cases.append(np.full(n, -np.inf, np.float32))
    v = np.full(n, np.nan, np.float32); cases.append(v)
    v = base.copy(); v[n - 1] = 50.0; cases.append(v)
    v = np.zeros(n, np.float32); v[3] = -0.0; cases.append(v)
    out = gpu.buf(np.zeros(1, np.uint32))
    for v in cases:
        vb = gpu.buf(v)
        gpu.run_op("k_argmax", vb, None, out, [n])
        want = L.sg_argmax_f32(v.ctypes.data_as(C.POINTER(C.c_float)), n)
        assert int(out.array[0]) == want
        vb.free()
