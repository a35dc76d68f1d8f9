"""surge_amd - Python binding of the MI355X decode engine's C ABI.

The product is ``libsurge_amd.so`` (C11 host code + gfx950 HIP kernels) and
its C header ``include/surge.h``, which keeps the reference engine's
``sg_gpu_*`` interface (reference surge.h:640-1408). This module is a thin
ctypes mirror of that interface for Python callers (tests, bench.py): the
same entry points, the same argument meanings, the same errors (an ``sg_err``
message becomes a :class:`SurgeError`).

Nothing here computes anything: every call goes through the HIP library, and
loading fails loudly when the library has not been built.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsurge_amd.so")

SG_T_F32, SG_T_F16, SG_T_Q8_0, SG_T_BF16 = 0, 1, 8, 30
SG_KV_CAP_MAX = 262144      # the f16 KV cache's largest context (include/surge.h)


class SurgeError(RuntimeError):
    """An sg_err returned by the C library."""


class SgErr(C.Structure):
    _fields_ = [("msg", C.c_char_p)]


class SgCfg(C.Structure):
    """sg_cfg (reference surge.h:115-151), field for field."""
    _fields_ = [
        ("n_layers", C.c_uint32), ("n_heads", C.c_uint32), ("n_kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32), ("hidden", C.c_uint32), ("ffn_hidden", C.c_uint32),
        ("vocab", C.c_uint32), ("rope_theta", C.c_float), ("rms_eps", C.c_float),
        ("tied_embeddings", C.c_bool), ("rope_dim", C.c_uint32),
        ("full_attn_interval", C.c_uint32), ("n_k_heads", C.c_uint32),
        ("n_v_heads", C.c_uint32), ("head_k_dim", C.c_uint32), ("head_v_dim", C.c_uint32),
        ("conv_kernel", C.c_uint32), ("attn_output_gate", C.c_bool),
    ]


_LAYER_FIELDS = ["q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm", "gate_proj",
                 "up_proj", "down_proj", "ln1", "ln2", "ssm_in_qkv", "ssm_in_z", "ssm_in_b",
                 "ssm_in_a", "ssm_a", "ssm_dt_bias", "ssm_conv1d", "ssm_norm", "ssm_out"]


class SgLayerW(C.Structure):
    _fields_ = [(f, C.c_void_p) for f in _LAYER_FIELDS]


class SgModel(C.Structure):
    """sg_model (reference surge.h:286-330), field for field."""
    _fields_ = [
        ("cfg", SgCfg), ("tok_emb", C.c_void_p), ("out_norm", C.c_void_p),
        ("lm_head", C.c_void_p), ("layers", C.POINTER(SgLayerW)), ("wtype", C.c_int),
        ("ssm_a_form", C.c_int), ("v_heads_tiled", C.c_bool), ("ssm_a_type", C.c_int),
        ("ssm_norm_type", C.c_int), ("dense_type", C.c_int), ("norms_are_residual", C.c_bool),
    ]


def make_cfg(**kw) -> SgCfg:
    c = SgCfg()
    for k, v in kw.items():
        setattr(c, k, v)
    return c


# The BASELINE configs' model shapes (qwen35 hybrid, 3 DeltaNet : 1 attention).
CFG_2B = dict(n_layers=24, n_heads=8, n_kv_heads=2, head_dim=256, hidden=2048,
              ffn_hidden=6144, vocab=151936, rope_theta=1e7, rms_eps=1e-6,
              tied_embeddings=True, rope_dim=64, full_attn_interval=4, n_k_heads=16,
              n_v_heads=16, head_k_dim=128, head_v_dim=128, conv_kernel=4,
              attn_output_gate=True)
CFG_27B = dict(n_layers=64, n_heads=24, n_kv_heads=4, head_dim=256, hidden=5120,
               ffn_hidden=17408, vocab=151936, rope_theta=1e7, rms_eps=1e-6,
               tied_embeddings=False, rope_dim=64, full_attn_interval=4, n_k_heads=16,
               n_v_heads=48, head_k_dim=128, head_v_dim=128, conv_kernel=4,
               attn_output_gate=True)

_SIGS = {
    # name: (restype, argtypes)
    "sg_gpu_init": (SgErr, [C.POINTER(C.c_void_p)]),
    "sg_gpu_free": (None, [C.c_void_p]),
    "sg_gpu_wrap": (SgErr, [C.c_void_p, C.c_void_p, C.c_uint64, C.POINTER(C.c_void_p)]),
    "sg_gpu_alloc": (SgErr, [C.c_void_p, C.c_uint64, C.POINTER(C.c_void_p), C.POINTER(C.c_void_p)]),
    "sg_gpu_buf_free": (None, [C.c_void_p]),
    "sg_gpu_buf_host": (C.c_void_p, [C.c_void_p]),
    "sg_gpu_buf_device": (C.c_void_p, [C.c_void_p]),
    "sg_gpu_buf_upload": (SgErr, [C.c_void_p]),
    "sg_gpu_buf_download": (SgErr, [C.c_void_p]),
    "sg_gpu_wrap_device": (SgErr, [C.c_void_p, C.c_void_p, C.c_uint64, C.POINTER(C.c_void_p)]),
    "sg_gpu_current_alloc_bytes": (C.c_uint64, [C.c_void_p]),
    "sg_gpu_run_op": (SgErr, [C.c_void_p, C.c_char_p, C.c_void_p, C.c_void_p, C.c_void_p,
                              C.POINTER(C.c_uint32)]),
    "sg_gpu_run_attn_decode_f16": (SgErr, [C.c_void_p] * 5 + [C.POINTER(C.c_uint32)]),
    "sg_gpu_run_attn_decode_f16_noalloc": (SgErr, [C.c_void_p] * 5 + [C.POINTER(C.c_uint32)]),
    "sg_gpu_run_attn_splitk_partial": (SgErr, [C.c_void_p] * 7 + [C.POINTER(C.c_uint32)]),
    "sg_gpu_run_attn_splitk_partial_gqa": (SgErr, [C.c_void_p] * 7 + [C.POINTER(C.c_uint32)]),
    "sg_gpu_run_attn_splitk_combine": (SgErr, [C.c_void_p] * 5 + [C.POINTER(C.c_uint32)]),
    "sg_gpu_run_delta_multi": (SgErr, [C.c_void_p] * 5 + [C.POINTER(C.c_uint32)]),
    "sg_gpu_run_conv1d_chunk": (SgErr, [C.c_void_p] * 5 + [C.POINTER(C.c_uint32)]),
    "sg_gpu_run_delta_gates_chunk": (SgErr, [C.c_void_p] * 5 + [C.POINTER(C.c_uint32)]),
    "sg_gpu_run_delta_chunk": (SgErr, [C.c_void_p] * 5 + [C.POINTER(C.c_uint32)]),
    "sg_gpu_run_rmsnorm_gated_chunk": (SgErr, [C.c_void_p] * 5 + [C.POINTER(C.c_uint32)]),
    "sg_gpu_run_attn_prefill": (SgErr, [C.c_void_p] * 5 + [C.POINTER(C.c_uint32)]),
    "sg_gpu_run_attn_splitk_partial_gqa_online": (SgErr, [C.c_void_p] * 7 + [C.POINTER(C.c_uint32)]),
    "sg_gpu_run_gdn_step": (SgErr, [C.c_void_p] * 5 + [C.POINTER(C.c_uint32)]),
    "sg_gpu_run_gdn_chunk": (SgErr, [C.c_void_p] * 5 + [C.POINTER(C.c_uint32)]),
    "sg_gpu_run_attn_chunk": (SgErr, [C.c_void_p] * 5 + [C.POINTER(C.c_uint32)]),
    "sg_gpu_splitk_online_dispatches": (C.c_uint64, [C.c_void_p]),
    "sg_gpu_splitk_online_selected": (C.c_bool, [C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32,
                                                 C.c_uint32]),
    "sg_gpu_splitk_gqa_selected": (C.c_bool, [C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32]),
    "sg_gpu_splitk_dispatch_counts": (None, [C.c_void_p, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
    "sg_gpu_prefill_segments": (C.c_uint64, [C.c_void_p]),
    "sg_gpu_splitk_n_splits": (C.c_uint32, [C.c_uint32]),
    "sg_gpu_splitk_gqa_n_splits": (C.c_uint32, [C.c_uint32]),
    "sg_gpu_splitk_gqa_n_splits_at": (C.c_uint32, [C.c_void_p, C.c_uint32]),
    "sg_gpu_splitk_gqa_cap": (C.c_uint32, [C.c_void_p]),
    "sg_gpu_load_model": (SgErr, [C.c_void_p, C.POINTER(SgModel)]),
    "sg_gpu_state_new": (SgErr, [C.c_void_p, C.POINTER(SgModel), C.c_uint32]),
    "sg_gpu_state_reset": (None, [C.c_void_p]),
    "sg_gpu_forward": (SgErr, [C.c_void_p, C.POINTER(SgModel), C.c_int32, C.c_uint32,
                               C.POINTER(C.POINTER(C.c_float))]),
    "sg_gpu_forward_nosync": (SgErr, [C.c_void_p, C.POINTER(SgModel), C.c_int32, C.c_uint32]),
    "sg_gpu_decode_greedy": (SgErr, [C.c_void_p, C.POINTER(SgModel), C.c_int32, C.c_uint32,
                                     C.c_uint32, C.POINTER(C.c_int32)]),
    "sg_gpu_state_fill_synthetic": (SgErr, [C.c_void_p, C.c_uint32, C.c_uint32]),
    "sg_gpu_time_read": (SgErr, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint32, C.POINTER(C.c_double)]),
    "sg_gpu_time_empty": (SgErr, [C.c_void_p, C.c_uint32, C.c_int, C.POINTER(C.c_double)]),
    "sgk_device_cus": (C.c_uint32, []),     # kernel-library helper: the current device's CU count
    "sg_gpu_time_floor": (SgErr, [C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32, C.POINTER(C.c_double),
                                  C.POINTER(C.c_uint32), C.POINTER(C.c_uint64)]),
    "sg_gpu_time_gemm": (SgErr, [C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.POINTER(C.c_double)]),
    "sg_gpu_decode_greedy_timed": (SgErr, [C.c_void_p, C.POINTER(SgModel), C.c_int32, C.c_uint32,
                                           C.c_uint32, C.POINTER(C.c_int32), C.POINTER(C.c_double)]),
    "sg_bench_format_md_row": (None, [C.c_void_p, C.c_char_p, C.c_size_t]),
    "sg_bench_format_json": (None, [C.c_void_p, C.c_char_p, C.c_size_t]),
    "sg_bench_admitted": (C.c_bool, [C.c_void_p]),
    "sg_bench_finalize_status": (None, [C.c_void_p]),
    "sg_bench_check_ingestion": (None, [C.c_uint64, C.c_uint32, C.c_uint64, C.c_uint64, C.POINTER(C.c_bool)]),
    "sg_gpu_prefill": (SgErr, [C.c_void_p, C.POINTER(SgModel), C.POINTER(C.c_int32), C.c_uint32,
                               C.c_uint32, C.POINTER(C.POINTER(C.c_float))]),
    "sg_gpu_sync": (SgErr, [C.c_void_p]),
    "sg_gpu_argmax": (SgErr, [C.c_void_p, C.POINTER(C.c_uint32)]),
    "sg_gpu_used": (C.c_uint32, [C.c_void_p]),
    "sg_gpu_stream": (C.c_void_p, [C.c_void_p]),
    "sg_gpu_enqueue_gemv": (SgErr, [C.c_void_p, C.c_uint32, C.c_uint32]),
    "sg_gpu_enqueue_gemv_tuned": (SgErr, [C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32]),
    "sg_gpu_time_matvec_q8": (SgErr, [C.c_void_p] * 4 + [C.c_uint32, C.c_uint32, C.c_uint64, C.c_uint32,
                                                          C.POINTER(C.c_double)]),
    "sg_gpu_time_attn": (SgErr, [C.c_void_p] * 5 + [C.POINTER(C.c_uint32), C.c_uint64, C.c_uint32,
                                                     C.POINTER(C.c_double)]),
    "sg_gpu_time_gdn_step": (SgErr, [C.c_void_p] * 4 + [C.POINTER(C.c_uint32), C.c_uint64, C.c_uint32,
                                                         C.POINTER(C.c_double)]),
    "sg_gguf_open": (SgErr, [C.c_char_p, C.POINTER(C.c_void_p)]),
    "sg_gguf_close": (None, [C.c_void_p]),
    "sg_model_from_gguf": (SgErr, [C.c_void_p, C.POINTER(SgModel)]),
    "sg_model_free": (None, [C.POINTER(SgModel)]),
    "sg_kv_bytes": (C.c_uint64, [C.POINTER(SgCfg), C.c_uint32, C.c_int]),
    "sg_kv_state_bytes": (C.c_uint64, [C.POINTER(SgCfg)]),
    "sg_kv_new": (SgErr, [C.c_void_p, C.POINTER(SgCfg), C.c_uint32, C.c_int, C.POINTER(C.c_void_p)]),
    "sg_kv_free": (None, [C.c_void_p]),
    "sg_kv_reset": (None, [C.c_void_p]),
    "sg_kv_advance": (SgErr, [C.c_void_p, C.c_uint32]),
    "sg_kv_used": (C.c_uint32, [C.c_void_p]),
    "sg_kv_cap": (C.c_uint32, [C.c_void_p]),
    "sg_kv_k": (C.c_void_p, [C.c_void_p, C.c_uint32]),
    "sg_kv_v": (C.c_void_p, [C.c_void_p, C.c_uint32]),
    "sg_kv_conv": (C.c_void_p, [C.c_void_p, C.c_uint32]),
    "sg_kv_s": (C.c_void_p, [C.c_void_p, C.c_uint32]),
    "sg_f32_to_f16": (C.c_uint16, [C.c_float]),
    "sg_f16_to_f32": (C.c_float, [C.c_uint16]),
    "sg_argmax_f32": (C.c_uint32, [C.POINTER(C.c_float), C.c_uint32]),
    "sg_bench_slope": (C.c_double, [C.POINTER(C.c_double), C.c_uint32, C.c_uint32]),
    "sg_bench_avg_tps": (C.c_double, [C.POINTER(C.c_double), C.c_uint32, C.c_uint32]),
    "sg_bench_default_warmup": (C.c_uint32, [C.c_uint32]),
    "sg_synth_new": (SgErr, [C.POINTER(SgCfg), C.c_int, C.c_uint64, C.POINTER(C.c_void_p)]),
    "sg_synth_model": (C.POINTER(SgModel), [C.c_void_p]),
    "sg_synth_bytes": (C.c_uint64, [C.c_void_p]),
    "sg_synth_write_gguf": (SgErr, [C.c_void_p, C.c_char_p]),
    "sg_synth_free": (None, [C.c_void_p]),
}

_lib: Optional[C.CDLL] = None


def lib() -> C.CDLL:
    """The product library, with argument types set. Raises if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise SurgeError(f"{LIB_PATH} is not built: run __graft_entry__.build() "
                             "(make -C surge_amd)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(err: SgErr) -> None:
    if err.msg:
        raise SurgeError(err.msg.decode())


def params(vals: Sequence[int]) -> C.Array:
    p = (C.c_uint32 * 8)()
    for i, v in enumerate(vals):
        p[i] = int(v) & 0xFFFFFFFF
    return p


def fbits(x: float) -> int:
    """The uint32 bit pattern of an f32 (how params[] carry floats)."""
    return int(np.array([x], dtype=np.float32).view(np.uint32)[0])


class Buf:
    """A device buffer with a host mirror (sg_gpu_alloc). ``array`` views the
    mirror; one-shot entry points upload it before and download after."""

    def __init__(self, gpu: "Gpu", init, dtype=None):
        self.gpu = gpu
        if isinstance(init, (int, np.integer)):
            arr = np.zeros(int(init), dtype=dtype or np.uint8)
        else:
            arr = np.ascontiguousarray(init, dtype=dtype)
        self.nbytes = max(arr.nbytes, 1)
        h, host = C.c_void_p(), C.c_void_p()
        check(lib().sg_gpu_alloc(gpu.handle, self.nbytes, C.byref(h), C.byref(host)))
        self.handle = h
        raw = (C.c_uint8 * self.nbytes).from_address(host.value)
        self._raw = np.frombuffer(raw, dtype=np.uint8)
        self.array = self._raw[: arr.nbytes].view(arr.dtype).reshape(arr.shape)
        self.array[...] = arr

    def free(self):
        if self.handle:
            lib().sg_gpu_buf_free(self.handle)
            self.handle = None

    def view(self, dtype, shape=None):
        v = self._raw.view(dtype)
        return v if shape is None else v[: int(np.prod(shape))].reshape(shape)


class Gpu:
    """sg_gpu: one HIP device, one stream (sg_gpu_init .. sg_gpu_free)."""

    def __init__(self):
        h = C.c_void_p()
        check(lib().sg_gpu_init(C.byref(h)))
        self.handle = h
        self.model = None

    def close(self):
        if self.handle:
            lib().sg_gpu_free(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def buf(self, init, dtype=None) -> Buf:
        return Buf(self, init, dtype)

    def run_op(self, kernel: str, a: Buf, b: Optional[Buf], out: Buf, p: Sequence[int]):
        check(lib().sg_gpu_run_op(self.handle, kernel.encode(), a.handle,
                                  b.handle if b is not None else None, out.handle, params(p)))

    def attn_partial(self, q, k, v, m, s, acc, p, gqa=True):
        f = lib().sg_gpu_run_attn_splitk_partial_gqa if gqa else lib().sg_gpu_run_attn_splitk_partial
        check(f(self.handle, q.handle, k.handle, v.handle, m.handle, s.handle, acc.handle, params(p)))

    def attn_combine(self, m, s, acc, out, p):
        check(lib().sg_gpu_run_attn_splitk_combine(self.handle, m.handle, s.handle, acc.handle,
                                                   out.handle, params(p)))

    def attn_decode_f16(self, q, k, v, out, p):
        check(lib().sg_gpu_run_attn_decode_f16(self.handle, q.handle, k.handle, v.handle,
                                               out.handle, params(p)))

    def gdn_step(self, inp, w, state, out, p):
        check(lib().sg_gpu_run_gdn_step(self.handle, inp.handle, w.handle, state.handle, out.handle,
                                         params(p)))

    def gdn_chunk(self, inp, w, state, out, p):
        check(lib().sg_gpu_run_gdn_chunk(self.handle, inp.handle, w.handle, state.handle, out.handle,
                                          params(p)))

    def attn_chunk(self, inp, w, kv, out, p):
        check(lib().sg_gpu_run_attn_chunk(self.handle, inp.handle, w.handle, kv.handle, out.handle,
                                           params(p)))

    def dispatch_counts(self):
        """(per_head, gqa, online) partial dispatches encoded since sg_gpu_state_new."""
        ph, gq = C.c_uint64(), C.c_uint64()
        lib().sg_gpu_splitk_dispatch_counts(self.handle, C.byref(ph), C.byref(gq))
        return ph.value, gq.value, lib().sg_gpu_splitk_online_dispatches(self.handle)

    def gqa_selected(self, nh, nkv, seq) -> bool:
        return bool(lib().sg_gpu_splitk_gqa_selected(self.handle, nh, nkv, seq))

    def online_selected(self, nh, nkv, hd, seq) -> bool:
        return bool(lib().sg_gpu_splitk_online_selected(self.handle, nh, nkv, hd, seq))

    def delta_multi(self, S, qkv, out, gates, p):
        check(lib().sg_gpu_run_delta_multi(self.handle, S.handle, qkv.handle, out.handle,
                                           gates.handle, params(p)))

    def run4(self, entry: str, a, b, c, d, p):
        """Any four-buffer one-shot: sg_gpu_run_<entry>(g, a, b, c, d, params)."""
        check(getattr(lib(), "sg_gpu_run_" + entry)(self.handle, a.handle, b.handle, c.handle, d.handle,
                                                       params(p)))

    # ---- decode
    def load_model(self, model_ptr):
        check(lib().sg_gpu_load_model(self.handle, model_ptr))
        self.model = model_ptr

    def state_new(self, max_ctx: int):
        check(lib().sg_gpu_state_new(self.handle, self.model, max_ctx))

    def state_reset(self):
        lib().sg_gpu_state_reset(self.handle)

    def split_cap(self) -> int:
        return int(lib().sg_gpu_splitk_gqa_cap(self.handle))

    def n_splits_at(self, seq: int) -> int:
        return int(lib().sg_gpu_splitk_gqa_n_splits_at(self.handle, seq))

    def forward(self, token: int, pos: int) -> np.ndarray:
        lg = C.POINTER(C.c_float)()
        check(lib().sg_gpu_forward(self.handle, self.model, token, pos, C.byref(lg)))
        vocab = self.model.contents.cfg.vocab
        return np.ctypeslib.as_array(lg, shape=(vocab,)).copy()

    def forward_nosync(self, token: int, pos: int):
        check(lib().sg_gpu_forward_nosync(self.handle, self.model, token, pos))

    def decode_greedy(self, token: int, pos: int, n: int) -> np.ndarray:
        out = (C.c_int32 * n)()
        check(lib().sg_gpu_decode_greedy(self.handle, self.model, token, pos, n, out))
        return np.array(out, dtype=np.int32)

    def decode_greedy_timed(self, token: int, pos: int, n: int):
        """(tokens, cumulative seconds at the end of each step)."""
        out = (C.c_int32 * n)()
        t = (C.c_double * n)()
        check(lib().sg_gpu_decode_greedy_timed(self.handle, self.model, token, pos, n, out, t))
        return np.array(out, dtype=np.int32), np.array(t, dtype=np.float64)

    def fill_synthetic(self, n_tokens: int, seed: int = 0) -> None:
        """Seeded K/V and DeltaNet state up to depth n_tokens (decode then starts at n_tokens)."""
        check(lib().sg_gpu_state_fill_synthetic(self.handle, n_tokens, seed))

    def prefill(self, tokens, chunk: int = 0) -> np.ndarray:
        ids = np.ascontiguousarray(tokens, dtype=np.int32)
        lg = C.POINTER(C.c_float)()
        check(lib().sg_gpu_prefill(self.handle, self.model,
                                   ids.ctypes.data_as(C.POINTER(C.c_int32)), len(ids), chunk,
                                   C.byref(lg)))
        vocab = self.model.contents.cfg.vocab
        return np.ctypeslib.as_array(lg, shape=(vocab,)).copy()

    def sync(self):
        check(lib().sg_gpu_sync(self.handle))

    def argmax(self) -> int:
        t = C.c_uint32()
        check(lib().sg_gpu_argmax(self.handle, C.byref(t)))
        return t.value

    def used(self) -> int:
        return lib().sg_gpu_used(self.handle)

    def stream(self) -> int:
        return lib().sg_gpu_stream(self.handle)

    def time_matvec_q8(self, w: Buf, x: Buf, y: Buf, rows: int, cols: int, rotate: int, reps: int) -> float:
        us = C.c_double()
        check(lib().sg_gpu_time_matvec_q8(self.handle, w.handle, x.handle, y.handle, rows, cols, rotate, reps,
                                          C.byref(us)))
        return us.value

    def time_read(self, nbytes: int, rotate: int, reps: int) -> float:
        us = C.c_double()
        check(lib().sg_gpu_time_read(self.handle, nbytes, rotate, reps, C.byref(us)))
        return us.value

    def time_gemm(self, layer: int, which: int, n: int, reps: int) -> float:
        """Average microseconds of the prefill GEMM on a loaded weight
        (which: 0 input, 1 output, 2 gate/up, 3 down) for n tokens."""
        us = C.c_double()
        check(lib().sg_gpu_time_gemm(self.handle, layer, which, n, reps, C.byref(us)))
        return us.value

    def time_empty(self, reps: int, graph: bool) -> float:
        us = C.c_double()
        check(lib().sg_gpu_time_empty(self.handle, reps, 1 if graph else 0, C.byref(us)))
        return us.value

    def time_floor(self, ctx: int, mode: int, reps: int):
        """(us per token, kernels, bytes) of the decode token's launch sequence
        as plain reads of each kernel's bytes (mode 1) or empty kernels (mode 0)."""
        us, n, nb = C.c_double(), C.c_uint32(), C.c_uint64()
        check(lib().sg_gpu_time_floor(self.handle, ctx, mode, reps, C.byref(us), C.byref(n), C.byref(nb)))
        return us.value, n.value, nb.value

    def time_attn(self, q: Buf, k: Buf, v: Buf, out: Buf, p, rotate: int, reps: int):
        us = (C.c_double * 2)()
        check(lib().sg_gpu_time_attn(self.handle, q.handle, k.handle, v.handle, out.handle, params(p), rotate,
                                     reps, us))
        return us[0], us[1]

    def time_gdn_step(self, inp: Buf, w: Buf, out: Buf, p, rotate: int, reps: int) -> float:
        us = C.c_double()
        check(lib().sg_gpu_time_gdn_step(self.handle, inp.handle, w.handle, out.handle, params(p), rotate, reps,
                                         C.byref(us)))
        return us.value

    def enqueue_gemv(self, layer: int, which: int, tune_r: int = 0, tune_blocks: int = 0):
        if tune_r or tune_blocks:
            check(lib().sg_gpu_enqueue_gemv_tuned(self.handle, layer, which, tune_r, tune_blocks))
        else:
            check(lib().sg_gpu_enqueue_gemv(self.handle, layer, which))

    def alloc_bytes(self) -> int:
        return lib().sg_gpu_current_alloc_bytes(self.handle)


class BenchRow(C.Structure):
    """sg_bench_row (reference surge.h:1845-1914), field for field."""
    _fields_ = [
        ("model", C.c_char * 64), ("engine", C.c_char * 64), ("prefill_tps", C.c_double),
        ("decode_tps_slope", C.c_double), ("decode_tps_avg", C.c_double), ("prefill_wall_s", C.c_double),
        ("decode_wall_s", C.c_double), ("prefill_segments", C.c_ulonglong), ("prefill_rest_s", C.c_double),
        ("prefill_compute_tps", C.c_double), ("decode_rest_s", C.c_double), ("decode_compute_tps", C.c_double),
        ("decode_rests", C.c_uint32), ("decode_clamp_events", C.c_uint32), ("decode_baseline_ms", C.c_double),
        ("peak_ram_gib", C.c_double), ("gpu_alloc_gib", C.c_double), ("recall_hits", C.c_uint32),
        ("recall_total", C.c_uint32), ("assoc_hits", C.c_uint32), ("n_prompt_tok", C.c_uint64),
        ("n_gen", C.c_uint32), ("wall_s", C.c_double), ("gemm_tflops", C.c_double), ("ingestion_ok", C.c_bool),
        ("status", C.c_char * 16), ("log_id", C.c_char * 96),
    ]

    def md(self) -> str:
        buf = C.create_string_buffer(1024)
        lib().sg_bench_format_md_row(C.byref(self), buf, len(buf))
        return buf.value.decode()

    def json(self) -> str:
        buf = C.create_string_buffer(4096)
        lib().sg_bench_format_json(C.byref(self), buf, len(buf))
        return buf.value.decode()


class Synth:
    """A seeded random-init qwen35-shaped model in host memory (sg_synth_*)."""

    def __init__(self, cfg: dict, wtype: int = SG_T_Q8_0, seed: int = 0):
        self.cfg = make_cfg(**cfg)
        h = C.c_void_p()
        check(lib().sg_synth_new(C.byref(self.cfg), wtype, seed, C.byref(h)))
        self.handle = h
        self.model = lib().sg_synth_model(h)

    def nbytes(self) -> int:
        return lib().sg_synth_bytes(self.handle)

    def write_gguf(self, path: str):
        check(lib().sg_synth_write_gguf(self.handle, path.encode()))

    def close(self):
        if self.handle:
            lib().sg_synth_free(self.handle)
            self.handle = None


class GGUFModel:
    """sg_gguf_open + sg_model_from_gguf."""

    def __init__(self, path: str):
        self.g = C.c_void_p()
        check(lib().sg_gguf_open(path.encode(), C.byref(self.g)))
        self.m = SgModel()
        err = lib().sg_model_from_gguf(self.g, C.byref(self.m))
        if err.msg:
            lib().sg_gguf_close(self.g)
            raise SurgeError(err.msg.decode())
        self.model = C.pointer(self.m)

    def close(self):
        if self.g:
            lib().sg_model_free(C.byref(self.m))
            lib().sg_gguf_close(self.g)
            self.g = None
