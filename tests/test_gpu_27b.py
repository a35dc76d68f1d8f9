"""The BASELINE target shape end to end: the random-init 27B-shaped Q8_0
hybrid (hidden 5120, 64 layers, 3 DeltaNet : 1 attention, attention 24q/4kv
x 256 with rope 64, DeltaNet 48 value heads tiled over 16 key heads x 128,
FFN 17408, vocab 151936, separate lm_head), about 27.5 GB of weights.

- Greedy decode after a 16-token prompt gives the 16 tokens the reference's
  own ref.c produced (tests/golden/greedy_27b_ref.json, written by
  tests/golden/make_greedy.py from oracle/_ref): the reference's own gate for
  its 27B (docs/11082026_m34_q8_gate.md: top-1 identical to ref.c).
- Chunked prefill of 1536 ids in 512-token chunks (so chunks 2 and 3 run the
  flash pass's key split) against the serial decode of the same ids: last
  logits within 2e-4 relative, same argmax, and the next decode step within
  2e-4 (the reference's prefill bar, tests/test_gpu_prefill.c:1-30).
"""
import json
import os

import numpy as np
import pytest

import fixture
import surge_amd as S

pytestmark = pytest.mark.gpu


def rel(got, want):
    return float(np.abs(got.astype(np.float64) - want).max() / np.abs(want).max())


@pytest.fixture(scope="module")
def model27(gpu):
    print("[27b] synthesising and loading the 27B-shape model", flush=True)
    syn = S.Synth(S.CFG_27B, S.SG_T_Q8_0, seed=0)
    gpu.load_model(syn.model)
    yield syn
    gpu.state_new(8)
    syn.close()


def test_27b_greedy_identical_to_reference(gpu, model27):
    path = os.path.join(fixture.GOLDEN, "greedy_27b_ref.json")
    gold = json.load(open(path))
    assert gold["cfg"] == S.CFG_27B and gold["seed"] == 0
    prompt, want = gold["prompt_ids"], gold["gen_ids"]
    gpu.state_new(len(prompt) + len(want) + 1)
    for p, t in enumerate(prompt[:-1]):
        gpu.forward_nosync(t, p)
    gen = gpu.decode_greedy(prompt[-1], len(prompt) - 1, len(want))
    assert gen.tolist() == want
    # the host loop (sg_gpu_forward + sg_argmax_f32) gives the same tokens
    gpu.state_reset()
    lg = None
    for p, t in enumerate(prompt):
        lg = gpu.forward(t, p)
    host = []
    for i in range(len(want)):
        host.append(int(np.argmax(lg)))
        lg = gpu.forward(host[-1], len(prompt) + i)
    assert host == want


def test_27b_prefill_512_chunks_matches_serial(gpu, model27):
    rng = np.random.default_rng(27)
    n = 1536
    prompt = rng.integers(0, S.CFG_27B["vocab"], n).tolist()
    gpu.state_new(n + 4)
    serial = None
    for p, t in enumerate(prompt):
        if p < n - 1:
            gpu.forward_nosync(t, p)
        else:
            serial = gpu.forward(t, p)
    nxt_serial = gpu.forward(int(np.argmax(serial)), n)
    last = gpu.prefill(prompt, chunk=512)
    assert gpu.used() == n
    assert rel(last, serial) < 2e-4
    assert int(np.argmax(last)) == int(np.argmax(serial))
    nxt = gpu.forward(int(np.argmax(last)), n)
    assert rel(nxt, nxt_serial) < 2e-4
    assert int(np.argmax(nxt)) == int(np.argmax(nxt_serial))
