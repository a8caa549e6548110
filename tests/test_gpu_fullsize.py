"""Decode at the full sizes of BASELINE configs 4 and 5, with K and V drawn on
the device (sphkv_synth kv_device) and the pools encoded by the GPU encoder.

* config 4: 64 sequences of U[2048, 32768] tokens, 8 kv heads (GQA 4), pages
  scattered over one shared pool of ~1.2M 16-token pages (V slots up to
  1.2M, i.e. beyond 2^20, where a 32-bit V-page offset would overflow);
* config 5: 4 sequences of 131,072 tokens, 64 q / 8 kv heads (GQA 8).

Every output must be finite, no page may be reported malformed, and a seeded
sample of (seq, kv head) pairs must match the fp64 oracle (pages and V
bit-exact against the oracle's encode of that head, outputs within 2e-3).
"""
import numpy as np
import pytest
import torch

import sphkv_ops as ops
import sphkv_synth as synth
from gpu_helpers import check_sampled_heads, log

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("config,heads", [(4, 16), (5, 6)])
def test_full_size_decode_matches_oracle_on_sampled_heads(gpu, config, heads):
    log(f"full-size config {config}: drawing K/V on the device and planning")
    wl = synth.make_decode_workload(config, kv_device=gpu)
    log(f"  seqs {wl.num_seqs} rows {wl.plan.num_rows} vpages {wl.plan.num_vpages} "
        f"max vslot {int(wl.plan.vslot.max())} pool bytes {wl.plan.pages_bytes}")
    pool, _, _ = ops.build_pool_gpu(wl, gpu)
    q = torch.as_tensor(wl.q, device=gpu)
    out = ops.decode_paged(pool, q, wl.gqa, wl.rope_theta, check=True)
    torch.cuda.synchronize()
    log("  decoded; checking finiteness and sampled heads")
    assert torch.isfinite(out).all()
    if config == 4:
        assert int(wl.plan.vslot.max()) >= (1 << 20)
    check_sampled_heads(wl, pool, out, heads, seed=100 + config)
