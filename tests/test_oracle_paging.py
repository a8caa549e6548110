"""Pins of oracle/paging.py, the restatement of _build_per_head_pages'
grouping, sort, chunking and offsets (spherical_kv_pipeline.py:1146-1228) and
of the order allocate() returns retained tokens in (allocation.py:28-37,
207-217).  Every expected value below is written by hand from those lines; the
planners of the package are then checked against the oracle.
"""
import numpy as np
import pytest

import oracle
from oracle import paging
import sphkv_format as fmt
import sphkv_synth as synth

R = paging.RetainedToken
D = paging.DENSE_TIER_ID


def test_tier_order_is_first_appearance_not_tier_id():
    # keys (0, 0, 2) then (0, 0, 1): tier 2's group comes first although its
    # id is larger; each group is sorted by token index
    ret = [R(0, 0, 2, 5), R(0, 0, 1, 3), R(0, 0, 2, 1), R(0, 0, 1, 0)]
    assert paging.group_pages(ret) == {(0, 0): [(2, [[1, 5]]), (1, [[0, 3]])]}


def test_heads_are_grouped_apart_even_when_interleaved():
    ret = [R(0, 1, 1, 0), R(0, 0, 3, 0), R(0, 1, 1, 2), R(0, 0, 1, 1), R(0, 1, 2, 1)]
    g = paging.group_pages(ret)
    assert g == {(0, 1): [(1, [[0, 2]]), (2, [[1]])], (0, 0): [(3, [[0]]), (1, [[1]])]}
    assert list(g) == [(0, 1), (0, 0)]              # (seq, head) order of first appearance


def test_partial_last_chunk():
    ret = [R(0, 0, 1, i) for i in reversed(range(37))]
    (tier, chunks), = paging.group_pages(ret)[(0, 0)]
    assert tier == 1 and [len(c) for c in chunks] == [16, 16, 5]
    assert chunks[0] == list(range(16)) and chunks[2] == [32, 33, 34, 35, 36]


def test_page_size_of_the_reference_config():
    # PAGE_SIZE = 128 (config.py:4): 300 tokens -> 128, 128, 44
    ret = [R(0, 0, 2, i) for i in range(300)]
    (_, chunks), = paging.group_pages(ret, page_size=128)[(0, 0)]
    assert [len(c) for c in chunks] == [128, 128, 44]


def test_dropped_tier_and_empty_head():
    # tier 0 is never retained; a head whose tokens are all dropped has no
    # entry (the reference's defaultdict is never touched for it)
    t = [np.array([0, 1, 0, 2, 1]), np.zeros(5, np.int64)]
    ret = paging.retained_tokens(t, num_seqs=1, num_kv=2)
    assert ret == [R(0, 0, 1, 1), R(0, 0, 2, 3), R(0, 0, 1, 4)]
    assert paging.group_pages(ret) == {(0, 0): [(1, [[1, 4]]), (2, [[3]])]}


def test_retained_order_is_sinks_recents_rest():
    # allocate() returns sinks + recents + ctrl: with a sink of 1 and a recent
    # window of 2, head 0's token 0 and tokens 4, 5 come before token 1..3
    t = [np.array([3, 1, 2, 1, 2, 3]), np.array([1, 1, 1, 1, 1, 1])]
    ret = paging.retained_tokens(t, num_seqs=1, num_kv=2, sink=1, recent=2)
    assert [(r.head, r.index) for r in ret] == [(0, 0), (1, 0), (0, 4), (0, 5), (1, 4), (1, 5),
                                                 (0, 1), (0, 2), (0, 3), (1, 1), (1, 2), (1, 3)]
    # tier order of head 0 follows that list: 3 (sink), 2 (recent), 1
    assert [tier for tier, _ in paging.group_pages(ret)[(0, 0)]] == [3, 2, 1]


def test_dense_tier_groups_like_any_tier():
    ret = [R(0, 0, D, 0), R(0, 0, 1, 1), R(0, 0, D, 2)]
    assert paging.group_pages(ret) == {(0, 0): [(D, [[0, 2]]), (1, [[1]])]}


def test_page_offsets_known_answers():
    # tier 1 at dh 128 (G = 8, b = 6): pages of 16, 16 and 5 tokens are 264,
    # 264 and 8 + 32 + 30 + 40 = 110 bytes, back to back
    pt = paging.page_offsets(1, [16, 16, 5], 128)
    assert pt.tolist() == [[0, 40, 136], [264, 304, 400], [528, 568, 598]]
    # tier 3 at dh 128 (G = 4, b = 3): 16 tokens -> 8 + 16 + 24 + 64 = 112
    assert paging.page_offsets(3, [16, 1], 128).tolist() == [[0, 24, 48], [112, 136, 138]]
    # tier 2 at dh 64 (G = 4, b = 4): 16 tokens -> 8 + 16 + 32 + 64 = 120
    assert paging.page_offsets(2, [16], 64).tolist() == [[0, 24, 56]]
    # dense (this build's tier): 8-byte header, 2 * N * dh K bytes
    assert paging.page_offsets(D, [2, 1], 64).tolist() == [[0, 8, 264], [264, 272, 400]]


def test_build_per_head_pages_tuples():
    rng = np.random.default_rng(0)
    dh, L = 64, 40
    t = np.array([1] * 20 + [2] * 10 + [0] * 5 + [3] * 5)
    rng.shuffle(t)
    cbs = synth.make_codebooks(rng, 1, dh, [1, 2])               # no tier-3 codebook
    K = {(0, 0): rng.standard_normal((L, dh)).astype(np.float16)}
    V = {(0, 0): rng.standard_normal((L, dh)).astype(np.float16)}
    ret = paging.retained_tokens([t], 1, 1)
    out = paging.build_per_head_pages(ret, K, V, cbs, dh)[(0, 0)]
    order = [tier for tier, _ in paging.group_pages(ret)[(0, 0)]]
    assert 3 in order and [e[2] for e in out] == [{1: 6, 2: 4}[x] for x in order if x != 3]   # tier 3 skipped
    for pages, ptable, b, n, v, (r, th), pos in out:
        tier = {6: 1, 4: 2}[b]
        idx = np.nonzero(t == tier)[0]
        assert n == idx.size and (pos == idx).all() and (v == V[(0, 0)][idx]).all()
        assert ptable.tolist() == paging.page_offsets(tier, [16] * (n // 16) + ([n % 16] if n % 16 else []),
                                                      dh).tolist()
        assert pages.size == int(ptable[-1, 2]) + (n - 16 * (ptable.shape[0] - 1)) * (dh // 16)
        # page bytes are the C oracle's page of the chunk
        p0 = oracle.build_page(*oracle.encode_groups(K[(0, 0)][idx[:16]].astype(np.float32), cbs[tier][0]),
                               tier, b)
        assert (pages[:p0.size] == p0).all()


@pytest.mark.parametrize("config,ctx", [(1, 300), (2, 2000), (4, 700), (5, 300)])
def test_host_planner_equals_the_reference_grouping(config, ctx):
    kw = {"num_seqs_override": 3} if config in (4, 5) else {}
    wl = synth.make_decode_workload(config, ctx_override=ctx, **kw)
    groups = paging.group_pages(paging.retained_tokens(wl.tier_of, wl.num_seqs, wl.num_kv))
    paging.check_plan(wl.plan, groups)


def test_check_plan_rejects_a_wrong_tier_order():
    # the planner's rows in tier-id order instead of first-appearance order
    # are caught
    t = [np.array([2, 1, 2, 1] * 10)]
    plan = fmt.plan_pages(t, None, 1, 1, 128, 16)
    ret = paging.retained_tokens(t, 1, 1)
    paging.check_plan(plan, paging.group_pages(ret))
    swapped = sorted(ret, key=lambda r: r.tier != 1)     # same tokens, tier 1 now appears first
    with pytest.raises(AssertionError, match="tier 2 != 1"):
        paging.check_plan(plan, paging.group_pages(swapped))


def test_host_planner_index_order_is_allocate_order_at_reference_defaults():
    # the planners order tiers by smallest token index; allocate() returns
    # sinks + recents + rest (SINK_TOKENS=4, RECENT_WINDOW=256).  They agree
    # when sinks and recents carry token 0's (protected) tier, and differ
    # when the recents carry a tier that first appears later in index order
    rng = np.random.default_rng(12)
    lengths, num_kv = [3, 260, 261, 700], 2
    tier_of = []
    for L in lengths:
        for h in range(num_kv):
            t = rng.choice(np.array([0, 1, 2, 3]), size=L, p=[.2, .3, .3, .2]).astype(np.int32)
            t[:4] = t[max(0, L - 256):] = [D, 3][h]
            tier_of.append(t)
    plan = fmt.plan_pages(tier_of, None, len(lengths), num_kv, 128)
    paging.check_plan(plan, paging.group_pages(paging.retained_tokens(tier_of, len(lengths), num_kv, 4, 256)))
    t = np.full(300, 1, np.int32)
    t[:4], t[100], t[-256:] = D, 2, 3                    # index order D, 1, 2, 3; list order D, 3, 1, 2
    plan = fmt.plan_pages([t], None, 1, 1, 128)
    with pytest.raises(AssertionError):
        paging.check_plan(plan, paging.group_pages(paging.retained_tokens([t], 1, 1, 4, 256)))
