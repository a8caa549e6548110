"""GPU page planner (sphkv_plan_pages_count / _fill, sphkv_ops.plan_pages_gpu)
against the oracle's restatement of _build_per_head_pages' grouping, sort,
chunking and offsets (oracle/paging.py, spherical_kv_pipeline.py:1146-1228).

* Grouping: every (seq, head)'s rows are, in order, the oracle's chunks (tier,
  count, token indices, positions, section offsets relative to the page).
* Placement (the build's own: absolute 16-byte aligned offsets, V slots):
  the layout invariants the kernels rely on (sphkv_ops.validate_plan), pages
  disjoint inside the pool, every V slot used once.
* End to end: a device-planned pool encoded on the GPU is byte-identical to
  the oracle's encode at that placement, and decodes to the oracle's output
  within 2e-3.
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import paging
import sphkv_format as fmt
import sphkv_ops as ops
import sphkv_synth as synth
from gpu_helpers import log, max_err

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


def _check(dp, tier_of, lengths, num_kv, base=None, positions_of=None, sink=0, recent=0):
    plan = dp.to_host()
    groups = paging.group_pages(paging.retained_tokens(tier_of, len(lengths), num_kv, sink=sink, recent=recent))
    paging.check_plan(plan, groups, positions_of=positions_of)
    # placement invariants
    ops.validate_plan(plan)
    size = np.array([fmt.page_nbytes(int(t), int(n), plan.dh) for t, n in zip(plan.tier, plan.count)], np.int64)
    off = plan.ptable[:, 0].astype(np.int64)
    o = np.argsort(off, kind="stable")
    assert (off[o][1:] >= off[o][:-1] + size[o][:-1]).all(), "pages overlap"
    assert plan.num_rows == 0 or int((off + size).max()) <= plan.pages_bytes
    assert np.unique(plan.vslot).size == plan.num_rows and plan.num_vpages >= plan.num_rows
    # the placement is the host planner's logical placement, offset for offset
    host = fmt.plan_pages(tier_of, positions_of, len(lengths), num_kv, plan.dh)
    assert np.array_equal(plan.ptable, host.ptable) and plan.pages_bytes == host.pages_bytes
    assert np.array_equal(plan.row_start, host.row_start)
    if base is not None and dp.src_rows is not None:
        tk = plan.tokens
        src = np.where(tk >= 0, tk + base[plan.seq_head][:, None], -1)
        assert np.array_equal(dp.src_rows.cpu().numpy(), src)


@pytest.mark.parametrize("cfg,ctx", [(1, None), (2, 4096), (4, 2500)])
def test_device_plan_is_the_reference_grouping(gpu, cfg, ctx):
    wl = synth.make_decode_workload(cfg, ctx_override=ctx)
    t, lens, _ = _device_inputs(wl.tier_of, wl.lengths, wl.num_kv, gpu)
    base = _row_base(wl.lengths, wl.num_kv)
    dp = ops.plan_pages_gpu(t, lens, wl.num_kv, wl.dh, row_base=torch.from_numpy(base).to(gpu))
    log(f"config {cfg}: rows {dp.rows} pool bytes {dp.pages_bytes}")
    _check(dp, wl.tier_of, wl.lengths, wl.num_kv, base)


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
    _check(dp, tier_of, lengths, num_kv, base, positions_of=pos)
    dp2 = ops.plan_pages_gpu(t, lens, num_kv, 64, positions=p)
    _check(dp2, tier_of, lengths, num_kv, positions_of=pos)
    bad = t.clone()
    bad[0, 0] = 7
    with pytest.raises(ValueError, match="tier id"):
        ops.plan_pages_gpu(bad, lens, num_kv, dh)


def test_device_planned_pool_matches_the_oracle(gpu):
    wl = synth.make_decode_workload(2, ctx_override=4096)
    t, lens, _ = _device_inputs(wl.tier_of, wl.lengths, wl.num_kv, gpu)
    dp = ops.plan_pages_gpu(t, lens, wl.num_kv, wl.dh, row_base=torch.from_numpy(wl.row_base()).to(gpu))
    k = torch.as_tensor(wl.k_rows(), device=gpu)
    v = torch.as_tensor(wl.v_rows(), device=gpu)
    pool = ops.PagedPool.allocate_device(dp, wl.codebooks, gpu)
    ops.encode_pages(pool, k, v, dp.src_rows)
    q = torch.as_tensor(wl.q, device=gpu)
    got = ops.decode_paged(pool, q, wl.gqa, wl.rope_theta, check=True).float().cpu().numpy()
    # the oracle encodes the reference grouping's chunks at the device plan's placement
    wl_d = synth.Workload(**{**wl.__dict__, "plan": dp.to_host()})
    cpu = oracle.build_pool(wl_d)
    assert (pool.pages.cpu().numpy() == cpu["pages"]).all()
    assert (pool.v_pool.cpu().numpy().view(np.uint16) == cpu["v_pool"].view(np.uint16)).all()
    want = oracle.decode_mode_b(cpu, wl_d.plan, wl.codebooks, wl.q, wl.gqa, wl.rope_theta)
    err = max_err(got, want)
    log(f"  device-planned pool: decode max abs err {err:.3e}")
    assert err <= 2e-3


def test_device_plan_many_ranges_and_many_chunks(gpu):
    # 1300 (seq, head) ranges: more than the scan's 1024 threads, so threads
    # place several ranges each; then one head of 140000 tokens: 69 chunks of
    # 2048, more than one 64-chunk step of the chunk scan
    rng = np.random.default_rng(11)
    ids = np.array([0, 1, 2, 3, fmt.DENSE_TIER_ID])
    num_kv, lengths = 4, [int(x) for x in rng.integers(0, 90, size=325)]
    tier_of = [rng.choice(ids, size=L).astype(np.int32) for L in lengths for _ in range(num_kv)]
    t, lens, _ = _device_inputs(tier_of, lengths, num_kv, gpu)
    base = _row_base(lengths, num_kv)
    dp = ops.plan_pages_gpu(t, lens, num_kv, 128, row_base=torch.from_numpy(base).to(gpu))
    log(f"1300 ranges: rows {dp.rows} pool bytes {dp.pages_bytes}")
    _check(dp, tier_of, lengths, num_kv, base)
    lengths = [140000]
    tier_of = [rng.choice(ids, size=lengths[0], p=[0.1, 0.3, 0.3, 0.2, 0.1]).astype(np.int32)]
    t, lens, _ = _device_inputs(tier_of, lengths, 1, gpu)
    dp = ops.plan_pages_gpu(t, lens, 1, 64)
    log(f"140000 tokens: rows {dp.rows} pool bytes {dp.pages_bytes}")
    _check(dp, tier_of, lengths, 1)


def test_device_plan_follows_allocate_order_at_reference_defaults(gpu):
    # the reference orders a head's tiers by first appearance in allocate()'s
    # sinks + recents + rest list (SINK_TOKENS=4, RECENT_WINDOW=256,
    # config.py:14-15); the device planner by smallest token index.  With
    # the sinks and recents at the protected tier (token 0 is a sink) the
    # two orders agree: checked against the list order itself, on heads
    # shorter than, equal to and longer than sink + recent tokens
    rng = np.random.default_rng(12)
    num_kv, dh = 4, 128
    lengths = [3, 260, 261, 700, 2500]
    tier_of = []
    for L in lengths:
        for h in range(num_kv):
            t = rng.choice(np.array([0, 1, 2, 3]), size=L, p=[.2, .3, .3, .2]).astype(np.int32)
            prot = [fmt.DENSE_TIER_ID, 3][h % 2]                   # the protected tier of this head
            t[:4] = prot
            t[max(0, L - 256):] = prot
            tier_of.append(t)
    t, lens, _ = _device_inputs(tier_of, lengths, num_kv, gpu)
    base = _row_base(lengths, num_kv)
    dp = ops.plan_pages_gpu(t, lens, num_kv, dh, row_base=torch.from_numpy(base).to(gpu))
    log(f"sink 4 / recent 256: rows {dp.rows} pool bytes {dp.pages_bytes}")
    _check(dp, tier_of, lengths, num_kv, base, sink=4, recent=256)
