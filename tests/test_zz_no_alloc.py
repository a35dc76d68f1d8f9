"""The no-allocation variant of the single-call decode attention
(sg_gpu_run_attn_decode_f16_noalloc, partials in the library's static device
workspace) against the allocating entry point it mirrors, through the C ABI.

A fresh sg_gpu (no one-shot scratch yet) calls the no-allocation entry FIRST,
at a size whose partials the allocating entry must allocate for: the
allocation counter (sg_gpu_current_alloc_bytes) does not move. The allocating
entry then runs on the same inputs, and the counter does move, so the check
would have seen an allocation. Outputs are bit-identical, on two calls in a
row, the second smaller. A call too large for the workspace is refused."""
import numpy as np
import pytest

import surge_amd as S

pytestmark = pytest.mark.gpu


def _call(gpu, entry, bufs, nh, nkv, hd, seq):
    qb, kb, vb, ob = bufs
    p = S.params([nh, nkv, hd, seq, hd, S.fbits(1.0 / np.sqrt(hd))])
    before = gpu.alloc_bytes()
    S.check(getattr(S.lib(), entry)(gpu.handle, qb.handle, kb.handle, vb.handle, ob.handle, p))
    return ob.array.copy(), gpu.alloc_bytes() - before


def test_no_alloc_decode_attention_matches_allocating_entry():
    rng = np.random.default_rng(99)
    with S.Gpu() as gpu:
        for i, (nh, nkv, hd, seq) in enumerate([(24, 4, 256, 8192), (16, 4, 128, 700)]):   # second smaller
            q = rng.standard_normal(nh * hd).astype(np.float32)
            k = rng.standard_normal(seq * nkv * hd).astype(np.float16).view(np.uint16)
            v = rng.standard_normal(seq * nkv * hd).astype(np.float16).view(np.uint16)
            bufs = [gpu.buf(q), gpu.buf(k), gpu.buf(v), gpu.buf(np.full(nh * hd, np.nan, np.float32))]
            got, grew = _call(gpu, "sg_gpu_run_attn_decode_f16_noalloc", bufs, nh, nkv, hd, seq)
            assert grew == 0
            bufs[3].array[:] = np.nan
            S.check(S.lib().sg_gpu_buf_upload(bufs[3].handle))
            want, grew_alloc = _call(gpu, "sg_gpu_run_attn_decode_f16", bufs, nh, nkv, hd, seq)
            if i == 0:   # the fresh gpu's one-shot scratch is allocated here
                ns = S.lib().sg_gpu_splitk_n_splits(seq)
                assert grew_alloc >= nh * ns * (hd + 2) * 4
            assert np.isfinite(got).all()
            assert np.array_equal(got, want)
            for b in bufs:
                b.free()
        # 64 heads x 128 splits x 258 floats is above the 4 MiB workspace
        nh, nkv, hd, seq = 64, 8, 256, 8192
        bufs = [gpu.buf(np.zeros(nh * hd, np.float32)), gpu.buf(np.zeros(seq * nkv * hd, np.uint16)),
                gpu.buf(np.zeros(seq * nkv * hd, np.uint16)), gpu.buf(np.zeros(nh * hd, np.float32))]
        with pytest.raises(S.SurgeError, match="workspace"):
            _call(gpu, "sg_gpu_run_attn_decode_f16_noalloc", bufs, nh, nkv, hd, seq)
        for b in bufs:
            b.free()
