"""Decode at depth against the oracle: the attention read path at 32768 and
131072 keys (the reference gated its split-K at 32768 and 262144,
docs/16082026_splitk_decode_gate.md:35-38).

Both sides start from the same seeded state: sg_gpu_state_fill_synthetic
writes K/V rows [0, n) of every attention layer, every DeltaNet S and conv
tail, and the oracle's sg_ref_state_fill_synthetic writes the same values in
its own layouts. Then a few decode steps run on both, each writing its new
K/V row at the end of the cache. The model has the 27B's attention shape
(24 q / 4 kv heads x 256, rope 64, GQA 6) and DeltaNet shape (48 value heads
tiled over 16 key heads x 128) on a small hidden size, so the default split
policy runs 128 splits of 256 (or 1024) keys: four (or sixteen) 64-key rounds
per split, the new row stored in the last split's last round. Logits within
1e-3 relative and the same argmax at every step.
"""
import numpy as np
import pytest

import oracle_lib as O
import surge_amd as S

pytestmark = pytest.mark.gpu

DEEP = dict(n_layers=4, n_heads=24, n_kv_heads=4, head_dim=256, hidden=256, ffn_hidden=512,
            vocab=1000, rope_theta=1e7, rms_eps=1e-6, tied_embeddings=False, rope_dim=64,
            full_attn_interval=4, n_k_heads=16, n_v_heads=48, head_k_dim=128, head_v_dim=128,
            conv_kernel=4, attn_output_gate=True)


def rel(got, want):
    return float(np.abs(got.astype(np.float64) - want).max() / np.abs(want).max())


# the default cap (one partial workgroup per CU: 256 CUs / 4 kv heads = 64
# splits on an MI355X) at 32768 keys, and the cap raised to 128 splits (two
# workgroups per CU) at 131072
@pytest.mark.parametrize("depth,cap", [(32768, None), (131072, "128")])
def test_decode_at_depth_vs_oracle(gpu, depth, cap, monkeypatch):
    syn = S.Synth(DEEP, S.SG_T_Q8_0, seed=51)
    gpu.load_model(syn.model)
    if cap:
        monkeypatch.setenv("SURGE_SPLITK_GQA_CAP", cap)
    else:
        monkeypatch.delenv("SURGE_SPLITK_GQA_CAP", raising=False)
    gpu.state_new(depth + 8)
    assert gpu.n_splits_at(depth + 1) == (int(cap) if cap else min(128, S.lib().sgk_device_cus() // DEEP["n_kv_heads"]))
    gpu.fill_synthetic(depth, seed=7)
    rm = O.RefModel(O.oracle(), syn.model, depth + 8, kv_f16=True)
    rm.fill_synthetic(depth, seed=7)
    rng = np.random.default_rng(depth)
    worst = 0.0
    tok = int(rng.integers(0, DEEP["vocab"]))
    for p in range(depth, depth + 4):
        g = gpu.forward(tok, p)
        o = rm.forward(tok, p)
        worst = max(worst, rel(g, o))
        assert int(np.argmax(g)) == int(np.argmax(o)), f"argmax differs at position {p}"
        tok = int(np.argmax(o))
    rm.close()
    gpu.state_new(8)
    syn.close()
    assert worst < 1e-3, worst
