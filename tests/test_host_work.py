"""Host-side decode work list (sphkv_ops.make_work): every row of every
(seq, head) is covered exactly once, items of one (seq, head) are contiguous
in the list, and interleaved items hold the same mix of rows."""
import numpy as np
import pytest

import sphkv_ops as ops


def _rows(item):
    sh, first, end, stride = (int(x) for x in item)
    return list(range(first, end, stride))


@pytest.mark.parametrize("interleave", [True, False])
@pytest.mark.parametrize("rpi", [1, 5, 64, 10 ** 6])
def test_make_work_covers_each_row_once(interleave, rpi):
    row_start = np.array([0, 0, 7, 200, 201, 330], np.int64)     # includes an empty head
    work, ws = ops.make_work(row_start, rpi, interleave=interleave)
    assert work.shape[1] == 4 and work.dtype == np.int32
    assert ws[0] == 0 and ws[-1] == len(work) and (np.diff(ws) >= 1).all()
    for sh in range(len(row_start) - 1):
        items = work[ws[sh]:ws[sh + 1]]
        assert (items[:, 0] == sh).all() and (items[:, 3] >= 1).all()
        rows = sorted(r for it in items for r in _rows(it))
        assert rows == list(range(row_start[sh], row_start[sh + 1]))
        assert all(len(_rows(it)) <= rpi for it in items)


def test_interleaved_items_spread_each_tier_run():
    # a head of 3 tier runs (rows 0-59 t1, 60-89 t2, 90-99 dense) over 5 items:
    # every item gets rows of every run
    work, ws = ops.make_work(np.array([0, 100]), 20, interleave=True)
    for it in work:
        r = np.array(_rows(it))
        assert ((r < 60).sum(), ((r >= 60) & (r < 90)).sum(), (r >= 90).sum()) == (12, 6, 2)


def test_auto_rows_per_item_fits_one_wave_of_workgroups():
    # one (seq, head) of 2049 rows x 8 heads on 256 CUs: 65 rows -> 256 items
    rs = np.arange(9, dtype=np.int64) * 2049
    r = ops.auto_rows_per_item(rs, 256)
    assert r == 65 and sum(-(-2049 // r) for _ in range(8)) == 256
    # the answer is the smallest fitting row count
    assert sum(-(-2049 // (r - 1)) for _ in range(8)) > 256


def test_auto_rows_per_item_with_more_ranges_than_cus_terminates():
    # 512 ranges of 128..2048 rows on 256 CUs: each range needs an item, so
    # about four smaller items per CU
    rng = np.random.default_rng(0)
    lens = rng.integers(128, 2049, size=512)
    rs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    r = ops.auto_rows_per_item(rs, 256)
    assert r == max(8, -(-int(lens.sum()) // 1024))
    work, ws = ops.make_work(rs, r)
    assert len(work) >= 512


def _items(lens, r):
    return sum(max(1, -(-int(n) // r)) for n in lens)


@pytest.mark.parametrize("seed", range(6))
def test_auto_rows_per_item_is_the_first_fitting_row_count(seed):
    # brute force over r: the smallest r >= max(8, ceil(total / target)) whose
    # item total fits the target, or the many-ranges rule when none does
    rng = np.random.default_rng(seed)
    num_sh = int(rng.integers(1, 40))
    lens = rng.integers(0, 3000, size=num_sh) * (rng.random(num_sh) < 0.9)
    rs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    cus, slots = int(rng.choice([4, 16, 256])), int(rng.integers(1, 3))
    target, total = cus * slots, int(lens.sum())
    got = ops.auto_rows_per_item(rs, cus, slots)
    if total == 0:
        assert got == 8
        return
    lo = max(8, -(-total // target))
    hi = max(lo, int(lens.max()))
    if _items(lens, hi) > target:
        assert got == max(8, -(-total // (4 * target)))
    else:
        want = next(r for r in range(lo, hi + 1) if _items(lens, r) <= target)
        assert got == want


@pytest.mark.parametrize("interleave", [True, False])
def test_make_work_matches_a_loop_restatement(interleave):
    rng = np.random.default_rng(7)
    lens = rng.integers(0, 500, size=33)
    rs = np.concatenate([[5], 5 + np.cumsum(lens)])
    for rpi in (1, 3, 16, 100, 499, 500, 10 ** 6):
        work, ws = ops.make_work(rs, rpi, interleave=interleave)
        want, want_ws = [], []
        for sh in range(len(lens)):
            b, e = int(rs[sh]), int(rs[sh + 1])
            n = max(1, -(-(e - b) // rpi))
            want_ws.append(len(want))
            for i in range(n):
                want.append((sh, b + i, e, n) if interleave else (sh, b + i * rpi, min(e, b + (i + 1) * rpi), 1))
        want_ws.append(len(want))
        np.testing.assert_array_equal(work, np.array(want, np.int32).reshape(-1, 4))
        np.testing.assert_array_equal(ws, np.array(want_ws, np.int32))


def test_work_helpers_reject_bad_row_starts():
    from sphkv_lib import SphkvError
    with pytest.raises(SphkvError, match="non-decreasing"):
        ops.make_work(np.array([0, 10, 4]), 8)
    with pytest.raises(SphkvError, match="non-decreasing"):
        ops.auto_rows_per_item(np.array([0, 10, 4]), 256)
    with pytest.raises(ValueError):
        ops.make_work(np.array([0, 10]), 0)
    with pytest.raises(ValueError):
        ops.make_work(np.array([0, 2 ** 31]), 8)
    work, ws = ops.make_work(np.array([3]), 8)                 # no ranges
    assert work.shape == (0, 4) and list(ws) == [0]
