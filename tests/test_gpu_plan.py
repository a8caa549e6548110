"""GPU parity of the device page planner (sphkv_plan_pages_count / _fill,
sphkv_ops.plan_pages_gpu) with the host planner sphkv_format.plan_pages
(logical placement), which restates the grouping, sort, chunking and offsets
of _build_per_head_pages (spherical_kv_pipeline.py:1146-1228).  Integer work:
every array must be identical.  End to end, a pool planned on the device
decodes bit-identically to one planned on the host."""
import numpy as np
import pytest
import torch

import sphkv_format as fmt
import sphkv_ops as ops
import sphkv_synth as synth
from gpu_helpers import log

pytestmark = pytest.mark.gpu


def _device_inputs(tier_of, lengths, num_kv, gpu, positions_of=None):
    L_max = max(lengths) if lengths else 1
    t = np.zeros((len(tier_of), max(L_max, 1)), np.uint8)
    for sh, arr in enumerate(tier_of):
        t[sh, :len(arr)] = np.asarray(arr, np.int64) & 0xFF
    lens = torch.tensor(np.asarray(lengths, np.int32), device=gpu)
    pos = None
    if positions_of is not None:
        p = np.zeros((len(lengths), max(L_max, 1)), np.int32)
        for s, arr in enumerate(positions_of):
            p[s, :len(arr)] = arr
        pos = torch.from_numpy(p).to(gpu)
    return torch.from_numpy(t).to(gpu), lens, pos


def _row_base(lengths, num_kv):
    base, acc = [], 0
    for L in lengths:
        for h in range(num_kv):
            base.append(acc + h * L)
        acc += num_kv * L
    return np.asarray(base, np.int64)


def _compare(dp, want, base):
    got = dp.to_host()
    for f in ("tier", "count", "tokens", "positions", "seq_head", "row_start", "ptable", "vslot"):
        assert np.array_equal(np.asarray(getattr(got, f)), np.asarray(getattr(want, f))), f
    assert got.pages_bytes == want.pages_bytes and got.num_vpages == want.num_vpages
    if dp.src_rows is not None:
        tk = want.tokens
        src = np.where(tk >= 0, tk + base[want.seq_head][:, None], -1)
        assert np.array_equal(dp.src_rows.cpu().numpy(), src)


@pytest.mark.parametrize("cfg,ctx", [(1, None), (2, 4096), (4, 2500)])
def test_device_plan_equals_host_plan(gpu, cfg, ctx):
    wl = synth.make_decode_workload(cfg, ctx_override=ctx)
    t, lens, _ = _device_inputs(wl.tier_of, wl.lengths, wl.num_kv, gpu)
    base = _row_base(wl.lengths, wl.num_kv)
    dp = ops.plan_pages_gpu(t, lens, wl.num_kv, wl.dh, row_base=torch.from_numpy(base).to(gpu))
    want = fmt.plan_pages(wl.tier_of, None, wl.num_seqs, wl.num_kv, wl.dh, 16)
    log(f"config {cfg}: rows {dp.rows} pool bytes {dp.pages_bytes}")
    _compare(dp, want, base)


def test_device_plan_edge_cases_and_positions(gpu):
    rng = np.random.default_rng(9)
    num_kv, dh = 4, 128
    lengths = [40, 1, 300]
    tier_of = []
    for s, L in enumerate(lengths):
        for h in range(num_kv):
            if h == 1:
                t = np.zeros(L, np.int32)                          # everything dropped
            elif h == 2:
                t = np.full(L, fmt.DENSE_TIER_ID, np.int32)        # all dense
            else:
                t = rng.choice(np.array([0, 1, 2, 3, fmt.DENSE_TIER_ID]), size=L).astype(np.int32)
                if L > 5:
                    t[:3] = [3, fmt.DENSE_TIER_ID, 2]              # first appearance order 3, dense, 2, ...
            tier_of.append(t)
    pos = [np.sort(rng.choice(10 ** 6, size=L, replace=False)).astype(np.int32) for L in lengths]
    t, lens, p = _device_inputs(tier_of, lengths, num_kv, gpu, pos)
    base = _row_base(lengths, num_kv)
    dp = ops.plan_pages_gpu(t, lens, num_kv, dh, positions=p, row_base=torch.from_numpy(base).to(gpu))
    _compare(dp, fmt.plan_pages(tier_of, pos, len(lengths), num_kv, dh, 16), base)
    for dh2 in (64,):
        dp2 = ops.plan_pages_gpu(t, lens, num_kv, dh2, positions=p)
        _compare(dp2, fmt.plan_pages(tier_of, pos, len(lengths), num_kv, dh2, 16), base)
    bad = t.clone()
    bad[0, 0] = 7
    with pytest.raises(ValueError, match="tier id"):
        ops.plan_pages_gpu(bad, lens, num_kv, dh)


def test_device_planned_pool_decodes_like_host_planned(gpu):
    wl = synth.make_decode_workload(2, ctx_override=4096)
    host_plan = fmt.plan_pages(wl.tier_of, None, wl.num_seqs, wl.num_kv, wl.dh, 16)
    wl_host = synth.Workload(**{**wl.__dict__, "plan": host_plan})
    t, lens, _ = _device_inputs(wl.tier_of, wl.lengths, wl.num_kv, gpu)
    dp = ops.plan_pages_gpu(t, lens, wl.num_kv, wl.dh, row_base=torch.from_numpy(wl_host.row_base()).to(gpu))
    k = torch.as_tensor(wl.k_rows(), device=gpu)
    v = torch.as_tensor(wl.v_rows(), device=gpu)
    pool_d = ops.PagedPool.allocate_device(dp, wl.codebooks, gpu)
    ops.encode_pages(pool_d, k, v, dp.src_rows)
    pool_h, _, _ = ops.build_pool_gpu(wl_host, gpu)
    assert torch.equal(pool_d.pages, pool_h.pages) and torch.equal(pool_d.v_pool, pool_h.v_pool)
    q = torch.as_tensor(wl.q, device=gpu)
    a = ops.decode_paged(pool_d, q, wl.gqa, wl.rope_theta)
    b = ops.decode_paged(pool_h, q, wl.gqa, wl.rope_theta)
    assert torch.equal(a, b)
