"""ctypes access to the CPU oracles (test infrastructure only).

Two libraries expose the same sg_ref_* functions (reference surge.h:349-638):
  ORACLE - this repository's restatement, oracle/liboracle.so;
  REF    - the reference's own src/ref.c compiled from its sources into
           oracle/_ref/libsurge_ref.so (present only where the reference
           sources were available to build it).
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_PATH = os.path.join(ROOT, "oracle", "liboracle.so")
REF_PATH = os.path.join(ROOT, "oracle", "_ref", "libsurge_ref.so")

F = C.POINTER(C.c_float)
U16 = C.POINTER(C.c_uint16)
u32, f32 = C.c_uint32, C.c_float

_COMMON = {
    "sg_ref_rmsnorm": (None, [F, F, u32, f32]),
    "sg_ref_sigmoid": (f32, [f32]),
    "sg_ref_softplus": (f32, [f32]),
    "sg_ref_delta_decay": (f32, [f32, f32, f32]),
    "sg_ref_delta_decay_neg_a": (f32, [f32, f32, f32]),
    "sg_ref_silu": (None, [F, u32]),
    "sg_ref_swiglu": (None, [F, F, u32]),
    "sg_ref_gate_sigmoid": (None, [F, F, u32]),
    "sg_ref_softmax": (None, [F, u32]),
    "sg_ref_attn_combine": (None, [F, F, F, u32, u32, F]),
    "sg_ref_attn_decode": (None, [F, F, F, u32, u32, u32, u32, u32, f32, F]),
    "sg_ref_attn_decode_splitk": (None, [F, F, F, u32, u32, u32, u32, u32, f32, u32, F]),
    "sg_ref_rope_partial": (None, [F, u32, u32, u32, f32]),
    "sg_ref_rope": (None, [F, u32, u32, f32]),
    "sg_ref_matvec_f32": (None, [F, F, F, u32, u32]),
    "sg_ref_matvec_bf16": (None, [U16, F, F, u32, u32]),
    "sg_ref_matvec_q8": (None, [C.c_void_p, F, F, u32, u32]),
    "sg_ref_conv1d_causal": (None, [F, F, F, F, u32, u32]),
    "sg_ref_delta_step": (None, [F, F, F, F, f32, f32, F, u32, u32]),
    "sg_ref_state_new": (None, None),
    "sg_ref_state_free": (None, [C.c_void_p]),
    "sg_ref_state_reset": (None, [C.c_void_p]),
    "sg_ref_forward": (None, None),
}
_ORACLE_ONLY = {
    "sg_ref_f16_to_f32": (f32, [C.c_uint16]),
    "sg_ref_f32_to_f16": (C.c_uint16, [f32]),
    "sg_ref_argmax_f32": (u32, [F, u32]),
    "sg_ref_attn_partials": (None, [F, F, F, u32, u32, u32, u32, u32, f32, u32, F, F, F]),
    "sg_ref_state_set_kv_f16": (None, [C.c_void_p, C.c_bool]),
    "sg_ref_set_threads": (C.c_int, [C.c_int]),
    "sg_ref_state_fill_synthetic": (None, None),
}


def _load(path, extra):
    import surge_amd as S
    L = C.CDLL(path)
    sigs = dict(_COMMON)
    sigs.update(extra)
    sigs["sg_ref_state_new"] = (S.SgErr, [C.POINTER(S.SgModel), u32, C.POINTER(C.c_void_p)])
    sigs["sg_ref_forward"] = (S.SgErr, [C.c_void_p, C.POINTER(S.SgModel), C.c_int32, u32,
                                        C.POINTER(F)])
    if "sg_ref_state_fill_synthetic" in sigs:
        sigs["sg_ref_state_fill_synthetic"] = (S.SgErr, [C.c_void_p, u32, u32])
    for name, (res, args) in sigs.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    return L


_cache = {}


def oracle():
    if "o" not in _cache:
        _cache["o"] = _load(ORACLE_PATH, _ORACLE_ONLY)
    return _cache["o"]


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref():
    if "r" not in _cache:
        _cache["r"] = _load(REF_PATH, {})
    return _cache["r"]


def fp(a: np.ndarray):
    """float* to a contiguous f32 numpy array (caller keeps it alive)."""
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(F)


class RefModel:
    """sg_ref_state over an sg_model pointer, for either library."""

    def __init__(self, L, model_ptr, max_ctx, kv_f16=False):
        import surge_amd as S
        self.L, self.model = L, model_ptr
        self.st = C.c_void_p()
        err = L.sg_ref_state_new(model_ptr, max_ctx, C.byref(self.st))
        if err.msg:
            raise S.SurgeError(err.msg.decode())
        if kv_f16:
            L.sg_ref_state_set_kv_f16(self.st, True)
        self.vocab = model_ptr.contents.cfg.vocab

    def forward(self, token, pos):
        import surge_amd as S
        lg = F()
        err = self.L.sg_ref_forward(self.st, self.model, token, pos, C.byref(lg))
        if err.msg:
            raise S.SurgeError(err.msg.decode())
        return np.ctypeslib.as_array(lg, shape=(self.vocab,)).copy()

    def fill_synthetic(self, n_tokens, seed=0):
        """The seeded state sg_gpu_state_fill_synthetic writes (oracle only)."""
        import surge_amd as S
        err = self.L.sg_ref_state_fill_synthetic(self.st, n_tokens, seed)
        if err.msg:
            raise S.SurgeError(err.msg.decode())

    def close(self):
        if self.st:
            self.L.sg_ref_state_free(self.st)
            self.st = None
