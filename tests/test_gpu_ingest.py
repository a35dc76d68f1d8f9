"""The reference's 262144-position ingest gate (tests/test_gpu_prefill.c:433-441,
gate B) on the BASELINE 2B shape (random-init Q8_0 hybrid, hidden 2048, 24
layers, 8q/2kv x 256, vocab 151936): the whole context filled as 262112
prefill positions plus 32 greedy decode steps, since the cache's cap
(262144, SG_KV_CAP_MAX) leaves no slot after a full-cap prefill.

The reference's clauses: used == 262144 at the end, no device fault, the
prefill's last logits finite (non-degenerate), and 32 decoded ids in range,
not one id repeated. Added here: the same ids prefilled again in 1024-token
chunks (other flash key splits and GEMM rounds at every depth) give last
logits within 1e-3 relative and the same argmax, so the deep chunks compute
the same attention, not just finite numbers.
"""
import numpy as np
import pytest

import surge_amd as S

pytestmark = pytest.mark.gpu

N_PREFILL = 262112
N_GEN = 32


def rel(got, want):
    return float(np.abs(got.astype(np.float64) - want).max() / np.abs(want).max())


def test_2b_262144_ingest_then_decode(gpu):
    cfg = S.CFG_2B
    print("[ingest] synthesising and loading the 2B-shape model", flush=True)
    syn = S.Synth(cfg, S.SG_T_Q8_0, seed=3)
    gpu.load_model(syn.model)
    ids = np.random.default_rng(262144).integers(0, cfg["vocab"], N_PREFILL).astype(np.int32)
    try:
        gpu.state_new(N_PREFILL + N_GEN)
        print(f"[ingest] prefill of {N_PREFILL} ids in 512-token chunks", flush=True)
        last = gpu.prefill(ids, chunk=512)
        assert gpu.used() == N_PREFILL
        assert np.isfinite(last).all()
        gen = gpu.decode_greedy(int(np.argmax(last)), N_PREFILL, N_GEN)
        assert gpu.used() == N_PREFILL + N_GEN == 262144
        assert ((gen >= 0) & (gen < cfg["vocab"])).all()
        assert len(set(gen.tolist())) > 1, gen.tolist()
        print(f"[ingest] used {gpu.used()}, decoded {gen.tolist()[:8]} ...", flush=True)
        gpu.state_new(N_PREFILL + N_GEN)
        print("[ingest] the same ids in 1024-token chunks", flush=True)
        last2 = gpu.prefill(ids, chunk=1024)
        gap = rel(last2, last)
        print(f"[ingest] 512 vs 1024-token chunks: last-logit relative gap {gap:.3e}", flush=True)
        assert int(np.argmax(last2)) == int(np.argmax(last))
        assert gap < 1e-3, gap
    finally:
        gpu.state_new(8)
        syn.close()
