"""The all-tier re-encode of every token (_codes_all,
spherical_kv_pipeline.py:1536-1553) on the GPU (sphkv_encode_codes through
sphkv_ops.encode_codes_all) against the oracle's restatement of
_encode_keys_with_codebooks (:1130-1144) called over each (sequence, kv
head)'s whole token list, as the reference calls it: radii and codes
bit-exact, for fp32 and fp16 K, at dh 128 and 64, including a head whose
token count is not a multiple of 16 and single-token heads (torch's M = 1
order)."""
import numpy as np
import pytest
import torch

import oracle
import sphkv_ops as ops
import sphkv_synth as synth
from gpu_helpers import log

pytestmark = pytest.mark.gpu


def _check(wl, gpu, fp32):
    k = torch.as_tensor(wl.k_rows(), device=gpu)
    if fp32:
        k = k.float()
    cbs = {t: torch.as_tensor(np.ascontiguousarray(c, np.float32), device=gpu) for t, c in wl.codebooks.items()}
    got = ops.encode_codes_all(k, wl.row_base(), wl.lengths, wl.num_kv, cbs)
    n = 0
    for s in range(wl.num_seqs):
        for h in range(wl.num_kv):
            K, _ = wl.head_kv(s, h)
            for t, cb in wl.codebooks.items():
                r_want, c_want = oracle.encode_groups(K.astype(np.float32), cb[h])
                r_got, c_got = (x.cpu().numpy() for x in got[(s, h)][t])
                assert r_got.shape == r_want.shape
                assert (r_got.view(np.uint32) == np.asarray(r_want, np.float32).view(np.uint32)).all(), (s, h, t)
                assert (c_got == c_want).all(), (s, h, t, int((c_got != c_want).sum()))
                n += c_got.size
    return n


@pytest.mark.parametrize("fp32", [True, False])
def test_codes_all_matches_the_reference_encode(gpu, fp32):
    wl = synth.make_decode_workload(2, ctx_override=1000)          # 1000 tokens: a 8-token last page
    n = _check(wl, gpu, fp32)
    log(f"codes_all config 2 (ctx 1000, fp32 k={fp32}): {n} codes bit-exact")


def test_codes_all_dh64_and_short_heads(gpu):
    wl = synth.make_decode_workload(1, ctx_override=300)
    n = _check(wl, gpu, True)
    # single-token and two-token sequences: torch's M = 1 and small-bmm orders
    wl1 = synth.make_decode_workload(4, ctx_override=2, num_seqs_override=3)
    wl1 = synth.Workload(**{**wl1.__dict__, "lengths": [1, 2, 1],
                            "K": [k[:, :L] for k, L in zip(wl1.K, [1, 2, 1])],
                            "V": [v[:, :L] for v, L in zip(wl1.V, [1, 2, 1])]})
    n += _check(wl1, gpu, True)
    log(f"codes_all dh 64 and 1-2 token heads: {n} codes bit-exact")
