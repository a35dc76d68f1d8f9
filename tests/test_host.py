"""Host-side tests that need no GPU: the C-ABI library loads and exports every
function include/surge.h declares; the host C code (f16 conversions, GGUF
reader, model mapping, KV sizing, argmax, bench math, model synthesiser)
agrees with the oracle and with the reference's own loader."""
import ctypes as C
import os
import re
import tempfile

import numpy as np
import pytest

import fixture
import oracle_lib as O
import surge_amd as S

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
need_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")


def declared_functions():
    src = open(os.path.join(ROOT, "include", "surge.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = set()
    for m in re.finditer(r"^(?!static|typedef)[A-Za-z_][\w \*]*?\b(sg_\w+)\s*\(", src, flags=re.M):
        names.add(m.group(1))
    return sorted(names)


def test_library_exports_every_declared_function():
    names = declared_functions()
    assert len(names) > 60
    L = C.CDLL(S.LIB_PATH)
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_f16_conversions_match_oracle():
    L = S.lib()
    h = np.arange(65536, dtype=np.uint16)
    got = np.array([L.sg_f16_to_f32(int(v)) for v in h], np.float32)
    want = h.view(np.float16).astype(np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin], want[fin])
    rng = np.random.default_rng(3)
    xs = np.concatenate([(rng.standard_normal(30000) * 10.0 ** rng.integers(-9, 6, 30000)).astype(np.float32),
                         np.float32([65504, 65519.99, 65520, 2 ** -25, 2 ** -24, 3 * 2 ** -26, -0.0, 1e-30])])
    for v in xs:
        assert L.sg_f32_to_f16(float(v)) == O.oracle().sg_ref_f32_to_f16(float(v))
    assert L.sg_f32_to_f16(float("nan")) == 0x7E00
    assert L.sg_f32_to_f16(float("-inf")) == 0xFC00


def test_argmax_and_bench_math():
    L = S.lib()
    v = np.float32([0, 5, -1, 5, 4])
    assert L.sg_argmax_f32(v.ctypes.data_as(C.POINTER(C.c_float)), 5) == 1
    assert L.sg_argmax_f32(None, 5) == 0
    t = np.ascontiguousarray(1e9 + np.arange(50) / 40.0)       # 40 tok/s at an epoch offset
    p = t.ctypes.data_as(C.POINTER(C.c_double))
    assert abs(L.sg_bench_slope(p, 50, 1) - 40.0) < 1e-6
    assert abs(L.sg_bench_avg_tps(p, 50, 1) - 40.0) < 1e-4   # endpoint difference at a 1e9 s offset
    assert L.sg_bench_slope(p, 2, 1) == 0.0
    assert L.sg_bench_default_warmup(64) == 1 and L.sg_bench_default_warmup(1000) == 20


def test_kv_sizes():
    L = S.lib()
    c = S.make_cfg(**S.CFG_27B)
    # 16 attention layers x K,V x 4 kv heads x 256 x 2 bytes x 262144 = 16 GiB
    assert L.sg_kv_bytes(C.byref(c), 262144, S.SG_T_F16) == 16 << 30
    assert L.sg_kv_bytes(C.byref(c), 262145, S.SG_T_F16) == 0
    assert L.sg_kv_bytes(C.byref(c), 4096, 8) == 0
    # 48 DeltaNet layers x (3 x 10240 conv + 48 x 128 x 128 S) x 4 bytes
    assert L.sg_kv_state_bytes(C.byref(c)) == 48 * (3 * 10240 + 48 * 128 * 128) * 4


@need_ref
def test_kv_sizes_match_reference():
    R = C.CDLL(O.REF_PATH)
    R.sg_kv_bytes.restype = C.c_uint64
    R.sg_kv_state_bytes.restype = C.c_uint64
    for cfg in (S.CFG_2B, S.CFG_27B):
        c = S.make_cfg(**cfg)
        for cap in (1, 4096, 262144):
            assert S.lib().sg_kv_bytes(C.byref(c), cap, S.SG_T_F16) == R.sg_kv_bytes(C.byref(c), cap, S.SG_T_F16)
        assert S.lib().sg_kv_state_bytes(C.byref(c)) == R.sg_kv_state_bytes(C.byref(c))


def _tensor_bytes(m, field_ptr, n):
    return C.string_at(field_ptr, n) if field_ptr else None


@need_ref
def test_gguf_model_mapping_matches_reference_loader():
    """mini_fwd/model.gguf through this library's reader+mapper and through
    the reference's (oracle/_ref): same config, same flags, and every tensor
    pointer at the same offset into the file."""
    R = C.CDLL(O.REF_PATH)
    R.sg_gguf_open.restype = S.SgErr
    R.sg_gguf_open.argtypes = [C.c_char_p, C.POINTER(C.c_void_p)]
    R.sg_model_from_gguf.restype = S.SgErr
    R.sg_model_from_gguf.argtypes = [C.c_void_p, C.POINTER(S.SgModel)]
    path = os.path.join(fixture.GOLDEN, "mini_fwd", "model.gguf")
    ours = S.GGUFModel(path)
    rg = C.c_void_p()
    S.check(R.sg_gguf_open(path.encode(), C.byref(rg)))
    rm = S.SgModel()
    S.check(R.sg_model_from_gguf(rg, C.byref(rm)))
    a, b = ours.m, rm
    for f, _ in S.SgCfg._fields_:
        assert getattr(a.cfg, f) == getattr(b.cfg, f), f
    for f in ("wtype", "ssm_a_form", "v_heads_tiled", "ssm_a_type", "ssm_norm_type", "dense_type",
              "norms_are_residual"):
        assert getattr(a, f) == getattr(b, f), f
    base_a, base_b = a.tok_emb, b.tok_emb
    assert a.lm_head - base_a == b.lm_head - base_b
    assert a.out_norm - base_a == b.out_norm - base_b
    for i in range(a.cfg.n_layers):
        for f in S._LAYER_FIELDS:
            pa, pb = getattr(a.layers[i], f), getattr(b.layers[i], f)
            assert (pa is None) == (pb is None), (i, f)
            if pa is not None:
                assert pa - base_a == pb - base_b, (i, f)
    ours.close()


def test_gguf_reader_edge_cases():
    with pytest.raises(S.SurgeError):
        S.GGUFModel(os.path.join(fixture.GOLDEN, "mini.gguf"))    # valid v3, but not a model
    g = C.c_void_p()
    S.check(S.lib().sg_gguf_open(os.path.join(fixture.GOLDEN, "mini.gguf").encode(), C.byref(g)))
    S.lib().sg_gguf_close(g)
    data = open(os.path.join(fixture.GOLDEN, "mini_fwd", "model.gguf"), "rb").read()
    with tempfile.TemporaryDirectory() as d:
        for cut in (10, 200, len(data) - 100):
            p = os.path.join(d, "t.gguf")
            open(p, "wb").write(data[:cut])
            err = S.lib().sg_gguf_open(p.encode(), C.byref(g))
            assert err.msg is not None                               # truncated: an error, not a crash


def test_synth_gguf_round_trip_and_oracle_forward():
    cfg = dict(n_layers=4, n_heads=4, n_kv_heads=2, head_dim=32, hidden=64, ffn_hidden=96, vocab=50,
               rope_theta=1e6, rms_eps=1e-6, tied_embeddings=False, rope_dim=16, full_attn_interval=2,
               n_k_heads=2, n_v_heads=6, head_k_dim=32, head_v_dim=32, conv_kernel=4,
               attn_output_gate=True)
    syn = S.Synth(cfg, S.SG_T_Q8_0, seed=9)
    again = S.Synth(cfg, S.SG_T_Q8_0, seed=9)
    assert C.string_at(syn.model.contents.tok_emb, 50 * 2 * 34) == C.string_at(again.model.contents.tok_emb, 50 * 2 * 34)
    with tempfile.TemporaryDirectory() as d:
        p = os.path.join(d, "m.gguf")
        syn.write_gguf(p)
        gm = S.GGUFModel(p)
        assert gm.m.cfg.n_v_heads == 6 and gm.m.wtype == S.SG_T_Q8_0 and not gm.m.cfg.tied_embeddings
        a = O.RefModel(O.oracle(), syn.model, 8)
        b = O.RefModel(O.oracle(), gm.model, 8)
        for p_, t in enumerate([3, 1, 4, 1, 5]):
            assert np.array_equal(a.forward(t, p_), b.forward(t, p_))
        a.close(); b.close(); gm.close()
    syn.close(); again.close()


def test_gpu_init_fails_cleanly_without_a_device():
    """Here (no GPU) sg_gpu_init must return an error, not crash; on a GPU box
    it succeeds. Either way the product never falls back to the CPU."""
    h = C.c_void_p()
    err = S.lib().sg_gpu_init(C.byref(h))
    if err.msg is None:
        S.lib().sg_gpu_free(h)
    else:
        assert b"no HIP device" in err.msg


# ---------------------------------------------------------------- the C ABI against the reference header

REF_HEADER = "/root/reference/surge.h"


def _aux_prototypes(include_dir):
    """gcc -aux-info over a unit that includes <include_dir>/surge.h: every
    declared function as its prototype with parameter names dropped."""
    import subprocess
    with tempfile.TemporaryDirectory() as d:
        src, aux = os.path.join(d, "u.c"), os.path.join(d, "aux.txt")
        open(src, "w").write('#include "surge.h"\n')
        subprocess.check_call(["gcc", "-std=c11", "-fsyntax-only", "-aux-info", aux, "-I", include_dir, src])
        out = {}
        for line in open(aux):
            m = re.search(r"\*/\s*(.*?\b(sg_\w+)\s*\(.*\));", line)
            if m:
                out[m.group(2)] = re.sub(r"\s+", " ", m.group(1)).replace("extern ", "")
        return out


@pytest.mark.skipif(not os.path.exists(REF_HEADER), reason="reference sources absent")
def test_abi_prototypes_match_reference_header():
    """Every sg_gpu_* / sg_kv_* function the reference's surge.h declares, and
    the peak-memory probe's (sg_mem_tracker_*, sg_proc_phys_footprint), is
    declared here with the identical prototype (types as gcc prints them),
    so the reference's own callers compile and link against this library."""
    ref = _aux_prototypes(os.path.dirname(REF_HEADER))
    ours = _aux_prototypes(os.path.join(ROOT, "include"))
    wanted = sorted(n for n in ref if n.startswith(("sg_gpu_", "sg_kv_", "sg_mem_tracker_", "sg_proc_phys_")))
    assert len(wanted) >= 50
    missing = [n for n in wanted if n not in ours]
    assert not missing, missing
    differ = {n: (ref[n], ours[n]) for n in wanted if ref[n] != ours[n]}
    assert not differ, differ
    L = C.CDLL(S.LIB_PATH)
    assert all(hasattr(L, n) for n in wanted)


# ---------------------------------------------------------------- sg_kv with a host backend

# sg_err is one pointer, returned in a register: the callbacks return the
# message pointer (NULL = success) as a c_void_p.
_KV_ALLOC = C.CFUNCTYPE(C.c_void_p, C.c_void_p, C.c_uint64, C.POINTER(C.c_void_p), C.POINTER(C.c_void_p))
_KV_FREE = C.CFUNCTYPE(None, C.c_void_p)
_KV_HOST = C.CFUNCTYPE(C.c_void_p, C.c_void_p)


class _MallocBackend:
    """A malloc-backed sg_kv backend (the reference's test_kv.c mock): the
    handle is the zero-filled memory itself."""

    def __init__(self):
        self.live = {}
        libc = C.CDLL(None)
        self.calloc, self.free_ = libc.calloc, libc.free
        self.calloc.restype, self.calloc.argtypes = C.c_void_p, [C.c_size_t, C.c_size_t]
        self.free_.argtypes = [C.c_void_p]

        def alloc(g, n, buf, host):
            p = self.calloc(1, n)
            if not p:
                return None
            self.live[p] = n
            buf[0] = p
            if host:
                host[0] = p
            return None

        def free(b):
            if b:
                self.live.pop(b)
                self.free_(b)

        self.cbs = (_KV_ALLOC(alloc), _KV_FREE(free), _KV_HOST(lambda b: b))

    def register(self, L):
        L.sg_kv_set_backend.argtypes = [_KV_ALLOC, _KV_FREE, _KV_HOST]
        L.sg_kv_set_backend(*self.cbs)


def _kv_cfg(**kw):
    c = dict(n_layers=8, n_heads=4, n_kv_heads=2, head_dim=8, hidden=32, ffn_hidden=64, vocab=100,
             rope_theta=1e4, rms_eps=1e-6, tied_embeddings=False, rope_dim=8, full_attn_interval=4,
             n_k_heads=2, n_v_heads=4, head_k_dim=4, head_v_dim=4, conv_kernel=3, attn_output_gate=False)
    c.update(kw)
    return S.make_cfg(**c)


def test_kv_module_object_with_host_backend():
    """The reference's tests/test_kv.c object and rejection checks: layer-kind
    routing, sizes, advance bounds, reset zeroing conv/S but not K/V, cap 0
    -> default, cap above the maximum and unsupported dtypes refused, and no
    backend -> an error."""
    L = S.lib()
    be = _MallocBackend()
    be.register(L)
    c = _kv_cfg()
    kv = C.c_void_p()
    S.check(L.sg_kv_new(None, C.byref(c), 16, S.SG_T_F16, C.byref(kv)))
    try:
        assert L.sg_kv_cap(kv) == 16 and L.sg_kv_used(kv) == 0
        for l in range(8):
            attn = (l + 1) % 4 == 0
            assert bool(L.sg_kv_k(kv, l)) == attn and bool(L.sg_kv_v(kv, l)) == attn
            assert bool(L.sg_kv_conv(kv, l)) != attn and bool(L.sg_kv_s(kv, l)) != attn
        assert not L.sg_kv_k(kv, 8) and not L.sg_kv_conv(kv, 8)
        # sizes: K/V [cap, n_kv, hd] f16; conv [ksize-1, conv_dim] and S [n_v, dv, dk] f32
        assert be.live[L.sg_kv_k(kv, 3)] == 16 * 2 * 8 * 2
        assert be.live[L.sg_kv_conv(kv, 0)] == 2 * 32 * 4 and be.live[L.sg_kv_s(kv, 0)] == 4 * 4 * 4 * 4
        total = sum(be.live.values())
        assert total == L.sg_kv_bytes(C.byref(c), 16, S.SG_T_F16) + L.sg_kv_state_bytes(C.byref(c))
        S.check(L.sg_kv_advance(kv, 10))
        S.check(L.sg_kv_advance(kv, 6))
        assert L.sg_kv_used(kv) == 16
        assert L.sg_kv_advance(kv, 1).msg and L.sg_kv_used(kv) == 16
        L.sg_kv_reset(kv)
        assert L.sg_kv_advance(kv, 0xFFFFFFFF).msg and L.sg_kv_used(kv) == 0
        conv0, s0, k3 = L.sg_kv_conv(kv, 0), L.sg_kv_s(kv, 0), L.sg_kv_k(kv, 3)
        C.memset(conv0, 0xAB, 64)
        C.memset(s0, 0xCD, 64)
        C.cast(k3, C.POINTER(C.c_uint16))[0] = 0xBEEF
        S.check(L.sg_kv_advance(kv, 5))
        L.sg_kv_reset(kv)
        assert L.sg_kv_used(kv) == 0
        assert not any((C.c_uint8 * 64).from_address(conv0)) and not any((C.c_uint8 * 64).from_address(s0))
        assert C.cast(k3, C.POINTER(C.c_uint16))[0] == 0xBEEF
    finally:
        L.sg_kv_free(kv)
    assert not be.live
    # dense (every layer attention, no DeltaNet dims)
    d = _kv_cfg(n_layers=6, full_attn_interval=1, n_k_heads=0, n_v_heads=0, head_k_dim=0, head_v_dim=0,
                conv_kernel=0)
    S.check(L.sg_kv_new(None, C.byref(d), 16, S.SG_T_F32, C.byref(kv)))
    assert all(L.sg_kv_k(kv, l) and not L.sg_kv_s(kv, l) for l in range(6))
    L.sg_kv_free(kv)
    # rejections
    for cap, dt in [(S.SG_KV_CAP_MAX + 1, S.SG_T_F16), (8, S.SG_T_Q8_0)]:
        e = L.sg_kv_new(None, C.byref(c), cap, dt, C.byref(kv))
        assert e.msg and not kv.value
    assert b"cap" in L.sg_kv_new(None, C.byref(c), S.SG_KV_CAP_MAX + 1, S.SG_T_F16, C.byref(kv)).msg
    S.check(L.sg_kv_new(None, C.byref(c), 0, S.SG_T_F16, C.byref(kv)))
    assert L.sg_kv_cap(kv) == 131072
    L.sg_kv_free(kv)
    wide = _kv_cfg(head_k_dim=1 << 24)
    assert L.sg_kv_new(None, C.byref(wide), 8, S.SG_T_F16, C.byref(kv)).msg
    L.sg_kv_set_backend(_KV_ALLOC(), _KV_FREE(), _KV_HOST())
    assert b"backend" in L.sg_kv_new(None, C.byref(c), 8, S.SG_T_F16, C.byref(kv)).msg
    assert not be.live


# ---------------------------------------------------------------- the surge-bench row

def _row(**kw):
    r = S.BenchRow()
    r.model, r.engine = b"qwen27b-q8", b"surge_amd mi355x"
    r.prefill_tps, r.decode_tps_slope, r.decode_tps_avg = 5348.2, 170.794, 170.51
    r.peak_ram_gib, r.recall_hits, r.recall_total, r.wall_s = 27.54, 7, 8, 125.0
    r.status, r.log_id = b"DONE", b"ctx4k_27b_20261202"
    r.n_prompt_tok, r.n_gen, r.gemm_tflops, r.ingestion_ok = 4096, 128, 301.0, True
    for k, v in kw.items():
        setattr(r, k, v)
    return r


def test_bench_row_md_json_and_admission():
    """The leaderboard row's contract (reference surge.h:1916-1955): the
    8-column pipe row with prefill "%.0f" or "-", decode "%.2f", "%.1f GiB",
    hits/total and wall in whole minutes (lround); the JSON object has every
    field under its struct name (in the reference's key order), numbers at
    %.6g, a JSON bool,
    escaped strings, and stays in its buffer; admission is strict on the GEMM
    floor and needs ingestion_ok."""
    r = _row()
    assert r.md() == "| qwen27b-q8 | surge_amd mi355x | 5348 | 170.79 | 27.5 GiB | 7/8 | 2 min | DONE |"
    assert _row(prefill_tps=-1.0, wall_s=150.0).md().split(" | ")[2] == "-"
    assert _row(wall_s=150.0).md().endswith("| 3 min | DONE |")       # lround(2.5) = 3
    import json
    d = json.loads(r.json())
    assert sorted(d) == sorted(f for f, _ in S.BenchRow._fields_)
    assert list(d)[:10] == ["model", "engine", "prefill_tps", "decode_tps_slope", "decode_tps_avg", "prefill_wall_s",
                            "decode_wall_s", "prefill_rest_s", "prefill_compute_tps", "prefill_segments"]
    assert d["decode_tps_slope"] == float("%.6g" % 170.794) and d["n_prompt_tok"] == 4096
    assert d["ingestion_ok"] is True and d["status"] == "DONE" and d["log_id"] == "ctx4k_27b_20261202"
    odd = _row(model=b'a"b\\c\x01d\x1f')
    assert json.loads(odd.json())["model"] == 'a"b\\c\x01d\x1f'
    assert '"model":"a\\"b\\\\c\\u0001d\\u001f"' in odd.json()
    small = C.create_string_buffer(b"\xff" * 32)
    S.lib().sg_bench_format_json(C.byref(r), small, 10)
    assert small.raw[:10] == b"{\"model\":\x00" and small.raw[10:32] == b"\xff" * 22
    L = S.lib()
    assert not L.sg_bench_admitted(None)
    for tf, ok, want in [(20.5, True, "VOID"), (20.51, True, "DONE"), (300.0, False, "VOID")]:
        x = _row(gemm_tflops=tf, ingestion_ok=ok, status=b"")
        assert bool(L.sg_bench_admitted(C.byref(x))) == (want == "DONE")
        L.sg_bench_finalize_status(C.byref(x))
        assert x.status.decode() == want


# ---------------------------------------------------------------- the reference's GPU callers link unchanged

REF_ROOT = "/root/reference"
REF_CALLERS = ["test_gpu_fwd", "test_metal_ops", "test_gpu_prefill", "test_gpu_mem", "bench_splitk"]
# what the callers take from elsewhere than the GPU layer: the reference's CPU
# oracle (ref.c) and its safetensors reader (out of this build's scope)
NOT_OURS = ("sg_ref_", "sg_st_", "sg_model_from_st")


@pytest.mark.skipif(not os.path.isdir(os.path.join(REF_ROOT, "tests")) or not O.ref_available(),
                    reason="reference sources (or oracle/_ref) absent")
@pytest.mark.parametrize("caller", REF_CALLERS)
def test_reference_gpu_caller_links_against_library(caller):
    """The reference's own GPU test / bench source, compiled unchanged with the
    reference's surge.h, links against libsurge_amd.so, and every sg_*
    function it calls that is not the CPU oracle's or the safetensors
    reader's resolves from this library (the oracle part from oracle/_ref,
    the reference's ref.c compiled from its sources). Linked, not run."""
    import subprocess
    src = os.path.join(REF_ROOT, "tests", caller + ".c")
    lib_dir = os.path.dirname(S.LIB_PATH)
    with tempfile.TemporaryDirectory() as d:
        obj, exe = os.path.join(d, caller + ".o"), os.path.join(d, caller)
        cc = ["gcc", "-std=c11", "-D_GNU_SOURCE", "-w", "-I", REF_ROOT, "-I", os.path.join(REF_ROOT, "src"),
              "-I", os.path.join(REF_ROOT, "tests")]
        subprocess.check_call(cc + ["-c", src, "-o", obj])
        und = subprocess.check_output(["nm", "-u", obj], text=True).split()
        ours = set(subprocess.check_output(["nm", "-D", "--defined-only", S.LIB_PATH], text=True).split())
        used = sorted({s for s in und if s.startswith("sg_")})
        elsewhere = [s for s in used if s not in ours]
        assert all(s.startswith(NOT_OURS) for s in elsewhere), elsewhere
        assert any(s.startswith("sg_gpu_") for s in used)
        subprocess.check_call(["gcc", obj, "-o", exe, "-L", lib_dir, "-lsurge_amd", "-Wl,-rpath," + lib_dir,
                               O.REF_PATH, "-lm"])
        assert os.path.exists(exe)


def test_mem_tracker_and_phys_footprint():
    """The peak-memory probe (reference tests/test_gpu_mem.c tier 1: the
    tracker's running max, unit-exact; tier 2: the footprint is a live,
    non-zero reading that grows with touched host memory)."""
    L = S.lib()
    for n, (res, args) in {"sg_mem_tracker_reset": (None, [C.c_void_p]),
                           "sg_mem_tracker_sample": (None, [C.c_void_p, C.c_uint64, C.c_uint64]),
                           "sg_mem_tracker_peak": (C.c_uint64, [C.c_void_p]),
                           "sg_proc_phys_footprint": (C.c_uint64, [])}.items():
        getattr(L, n).restype, getattr(L, n).argtypes = res, args
    t = C.c_uint64(12345)
    L.sg_mem_tracker_reset(C.byref(t))
    assert L.sg_mem_tracker_peak(C.byref(t)) == 0
    for cur, phys, want in [(10, 20, 20), (5, 5, 20), (100, 3, 100), (0, 0, 100), (2 ** 63, 1, 2 ** 63)]:
        L.sg_mem_tracker_sample(C.byref(t), cur, phys)
        assert L.sg_mem_tracker_peak(C.byref(t)) == want
    L.sg_mem_tracker_reset(C.byref(t))
    assert L.sg_mem_tracker_peak(C.byref(t)) == 0
    L.sg_mem_tracker_sample(None, 1, 2)          # NULL tracker: no-op
    assert L.sg_mem_tracker_peak(None) == 0
    before = L.sg_proc_phys_footprint()
    assert before > 0
    block = np.ones(64 << 20, np.uint8)           # 64 MiB, touched
    after = L.sg_proc_phys_footprint()
    assert after >= before + (32 << 20), (before, after)
    del block


def test_bench_ingestion_guard():
    """sg_bench_check_ingestion (reference surge.h:1980-1993): true iff the
    ids fit the context and their count is in the expected range; a NULL
    ok is a no-op."""
    L = S.lib()
    ok = C.c_bool(False)
    for n, cap, lo, hi, want in [(4096, 4096, 4096, 4096, True), (4097, 4096, 0, 10 ** 6, False),
                                 (100, 4096, 101, 200, False), (150, 4096, 101, 200, True),
                                 (201, 4096, 101, 200, False), (0, 0, 0, 0, True)]:
        ok.value = not want
        L.sg_bench_check_ingestion(n, cap, lo, hi, C.byref(ok))
        assert ok.value == want, (n, cap, lo, hi)
    L.sg_bench_check_ingestion(1, 1, 1, 1, None)
