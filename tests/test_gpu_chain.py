"""Decode through the chain (SURGE_CHAIN=1): every run of decode stages
between attention layers (embedding, the Q8_0 GEMVs, the DeltaNet steps,
lm_head) is one persistent launch with device-wide barriers instead of kernel
boundaries; an attention layer's split-K partial and combine run as kernels
between runs. SURGE_CHAIN=2 runs only each DeltaNet layer's step and output
projection as one two-stage launch (the projection's weights are requested
while the step runs) and everything else as kernels. Both replay from
captured HIP graphs: the barrier counters need no per-token value.

- Per-position logits within 1e-3 (scale-relative) of the f16-KV oracle and
  identical argmax, for both DeltaNet shapes the chain takes at dk 128 and
  dk 64, over enough positions that the attention partial runs several splits
  and the conv ring wraps many times.
- The same logits as the per-kernel path within 1e-4 (float reassociation
  only: a chain GEMV row is summed in the per-kernel GEMV's order unless its
  row group is split between two waves, and the RMS factor's partial sums are
  grouped per 512 instead of 256 threads; measured about 1.3e-5).
- The device greedy loop gives the host loop's tokens; the 2B BASELINE
  configuration gives the reference ref.c's 64 tokens.
- A barrier that does not resolve fails the call (forced from the host with
  a one-poll spin bound, so every launch still runs to its end), and a new
  state decodes correctly afterwards.
"""
import json
import os

import numpy as np
import pytest

import fixture
import oracle_lib as O
import surge_amd as S

pytestmark = pytest.mark.gpu

BASE = dict(n_layers=8, n_heads=4, n_kv_heads=2, head_dim=256, hidden=1024, ffn_hidden=2048,
            vocab=3000, rope_theta=1e7, rms_eps=1e-6, tied_embeddings=False, rope_dim=64,
            full_attn_interval=4, conv_kernel=4, attn_output_gate=True)
CHAIN128 = dict(BASE, n_k_heads=4, n_v_heads=8, head_k_dim=128, head_v_dim=128)
CHAIN64 = dict(BASE, n_k_heads=8, n_v_heads=16, head_k_dim=64, head_v_dim=64)
CFGS = {"dk128": CHAIN128, "dk64": CHAIN64}


def rel(got, want):
    return float(np.abs(got.astype(np.float64) - want).max() / np.abs(want).max())


@pytest.mark.parametrize("mode", ["1", "2"])
@pytest.mark.parametrize("name", list(CFGS))
def test_chain_per_position_vs_oracle(gpu, monkeypatch, name, mode):
    cfg = CFGS[name]
    syn = S.Synth(cfg, S.SG_T_Q8_0, seed=21)
    gpu.load_model(syn.model)
    monkeypatch.setenv("SURGE_CHAIN", mode)
    gpu.state_new(400)
    assert gpu.chain_active()
    rng = np.random.default_rng(8)
    ids = rng.integers(0, cfg["vocab"], 300).tolist()
    rm = O.RefModel(O.oracle(), syn.model, 400, kv_f16=True)
    worst = 0.0
    for p, t in enumerate(ids):
        g = gpu.forward(t, p)
        o = rm.forward(t, p)
        if p % 29 == 0 or p >= len(ids) - 3:
            worst = max(worst, rel(g, o))
            assert np.argmax(g) == np.argmax(o), f"{name}: argmax differs at position {p}"
    rm.close()
    syn.close()
    assert worst < 1e-3, worst


@pytest.mark.parametrize("mode", ["1", "2"])
def test_chain_matches_per_kernel_path_and_greedy_loops(gpu, monkeypatch, mode):
    syn = S.Synth(CHAIN128, S.SG_T_Q8_0, seed=3)
    gpu.load_model(syn.model)
    ids = np.random.default_rng(2).integers(0, CHAIN128["vocab"], 40).tolist()
    monkeypatch.setenv("SURGE_CHAIN", "0")
    gpu.state_new(128)
    assert not gpu.chain_active()
    plain = np.stack([gpu.forward(t, p) for p, t in enumerate(ids)])
    plain_gen = gpu.decode_greedy(int(np.argmax(plain[-1])), len(ids), 24)
    monkeypatch.setenv("SURGE_CHAIN", mode)
    gpu.state_new(128)
    assert gpu.chain_active()
    chain = np.stack([gpu.forward(t, p) for p, t in enumerate(ids)])
    assert rel(chain, plain) < 1e-4
    assert (chain.argmax(1) == plain.argmax(1)).all()
    # device loop == per-kernel path's device loop == host loop
    gen = gpu.decode_greedy(int(np.argmax(chain[-1])), len(ids), 24)
    assert gen.tolist() == plain_gen.tolist()
    gpu.state_new(128)
    lg = None
    for p, t in enumerate(ids):
        lg = gpu.forward(t, p)
    host, tok = [], int(np.argmax(lg))
    for i in range(24):
        tok = int(np.argmax(gpu.forward(tok, len(ids) + i)))
        host.append(tok)
    assert host == gen.tolist()
    # reruns are bit-identical
    gpu.state_new(128)
    again = np.stack([gpu.forward(t, p) for p, t in enumerate(ids)])
    assert np.array_equal(again, chain)
    syn.close()


@pytest.mark.parametrize("mode", ["1", "2"])
def test_chain_2b_greedy_64_tokens_identical_to_reference(gpu, monkeypatch, mode):
    path = os.path.join(fixture.GOLDEN, "greedy_2b_ref.json")
    gold = json.load(open(path))
    syn = S.Synth(gold["cfg"], S.SG_T_Q8_0, seed=gold["seed"])
    gpu.load_model(syn.model)
    monkeypatch.setenv("SURGE_CHAIN", mode)
    gpu.state_new(len(gold["prompt_ids"]) + len(gold["gen_ids"]) + 1)
    assert gpu.chain_active()
    prompt = gold["prompt_ids"]
    for p, t in enumerate(prompt[:-1]):
        gpu.forward_nosync(t, p)
    gen = gpu.decode_greedy(prompt[-1], len(prompt) - 1, len(gold["gen_ids"]))
    syn.close()
    assert gen.tolist() == gold["gen_ids"]


@pytest.mark.parametrize("mode", ["1", "2"])
def test_chain_barrier_give_up_fails_the_call(gpu, monkeypatch, mode):
    syn = S.Synth(CHAIN128, S.SG_T_Q8_0, seed=4)
    gpu.load_model(syn.model)
    monkeypatch.setenv("SURGE_CHAIN", mode)
    monkeypatch.setenv("SURGE_CHAIN_SPIN", "1")
    gpu.state_new(64)
    assert gpu.chain_active()
    raised = False
    for p in range(8):
        try:
            gpu.forward(5 + p, p)
        except S.SurgeError as e:
            assert "chain" in str(e)
            raised = True
            break
    assert raised
    monkeypatch.delenv("SURGE_CHAIN_SPIN")
    gpu.state_new(64)
    ids = [7, 99, 1234, 5]
    rm = O.RefModel(O.oracle(), syn.model, 64, kv_f16=True)
    for p, t in enumerate(ids):
        assert rel(gpu.forward(t, p), rm.forward(t, p)) < 1e-3
    rm.close()
    syn.close()
