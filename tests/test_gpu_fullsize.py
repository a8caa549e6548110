"""Decode at the full sizes of BASELINE configs 4 and 5, with K and V drawn on
the device (sphkv_synth kv_device) and the pools encoded by the GPU encoder.

* config 4: 64 sequences of U[2048, 32768] tokens, 8 kv heads (GQA 4), pages
  scattered over one shared pool of ~1.2M 16-token pages (V slots up to
  1.2M, i.e. beyond 2^20, where a 32-bit V-page offset would overflow);
* config 5: 4 sequences of 131,072 tokens, 64 q / 8 kv heads (GQA 8).

Every output must be finite, no page may be reported malformed, and a seeded
sample of (seq, kv head) pairs must match the fp64 oracle (pages and V
bit-exact against the oracle's encode of that head, outputs within 2e-3).

Every (seq, kv head), at full size, also meets two size-independent
properties:
* with q = 0 every logit is exactly 0 and every weight exactly 1, so each
  output is the plain mean of that head's V rows (a page or token dropped,
  doubled or mis-masked by the work split, the page loop or the merge moves
  it);
* with the seeded q, the output does not depend on how the head's rows are
  split into work items (another split moves every item boundary, every
  wave's page set and the merge's inputs; only fp32 summation order and the
  fp16 rounding of P against another running maximum may differ).
"""
import dataclasses

import numpy as np
import pytest
import torch

import sphkv_ops as ops
import sphkv_synth as synth
from gpu_helpers import check_sampled_heads, log

pytestmark = pytest.mark.gpu


def _mean_v_per_head(wl, pool):
    """fp64 mean of each (seq, kv head)'s V rows, from the pool's V pages
    (dim-major: token n of dim d at d * page_size + n) over the plan's rows."""
    plan, dev, dh = wl.plan, pool.device, wl.dh
    num_sh = wl.num_seqs * wl.num_kv
    vs = torch.as_tensor(plan.vslot.astype(np.int64), device=dev)
    cnt = torch.as_tensor(plan.count.astype(np.int64), device=dev)
    shr = torch.as_tensor(plan.seq_head.astype(np.int64), device=dev)
    tot = torch.zeros((num_sh, dh), dtype=torch.float64, device=dev)
    tok = torch.zeros(num_sh, dtype=torch.float64, device=dev)
    slot = torch.arange(plan.page_size, device=dev)
    for a in range(0, plan.num_rows, 65536):
        b = min(a + 65536, plan.num_rows)
        v = pool.v_pool.index_select(0, vs[a:b]).view(b - a, dh, plan.page_size).double()
        m = (slot[None, :] < cnt[a:b, None]).double()
        tot.index_add_(0, shr[a:b], (v * m[:, None, :]).sum(-1))
        tok.index_add_(0, shr[a:b], cnt[a:b].double())
    assert bool((tok > 0).all())
    return tot / tok[:, None]


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
    log("  q = 0 on every head: outputs against each head's mean V row")
    out0 = ops.decode_paged(pool, torch.zeros_like(q), wl.gqa, wl.rope_theta, check=True)
    want = _mean_v_per_head(wl, pool).view(wl.num_seqs, wl.num_kv, 1, wl.dh)
    want = want.expand(-1, -1, wl.gqa, -1).reshape(wl.num_seqs, wl.num_kv * wl.gqa, wl.dh)
    err = float((out0.double() - want).abs().max())
    log(f"  every head, q = 0: max abs err {err:.3e}")
    assert err <= 1e-3
    rpi = 97                                           # an odd split: item boundaries move everywhere
    work, work_start = ops._work_device(wl.plan.row_start, rpi, gpu)
    assert work.shape[0] != pool.num_items
    out2 = ops.decode_paged(dataclasses.replace(pool, work=work, work_start=work_start), q, wl.gqa,
                            wl.rope_theta, check=True)
    err2 = float((out2.float() - out.float()).abs().max())
    log(f"  every head, {work.shape[0]} items of {rpi} rows against {pool.num_items}: max abs diff {err2:.3e}")
    assert err2 <= 1e-3
