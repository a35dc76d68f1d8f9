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
    for m in re.finditer(r"^(?!static)[A-Za-z_][\w \*]*?\b(sg_\w+)\s*\(", src, flags=re.M):
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
