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
