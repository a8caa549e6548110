"""Pins of oracle.layer_pool / layer_pool_page, the restatement of the
LayerPool constructor's page quantisation, page-id order and tables
(sphkv_lut.py:36-98).  Every expected value is written by hand from those
lines: pages are numbered kv head by kv head, run by run, page by page; a
head's block-table row lists its page ids in that order with the run's tier
index in the bits table; ctx_lens = pages * page_size; max_blocks = the
longest row + decode_capacity // num_kv + 2."""
import numpy as np

import oracle


def test_layer_pool_page_known_answer():
    # r_scale = per-group max (floored at 1e-8); codes = round-half-even(r / r_scale * 255)
    r = np.array([[1.0, 2.0, 0.0], [3.0, 0.5, 0.0]], np.float32)
    th = np.array([[5, 300, 7], [64, 1, 255]])
    t, rad, scl = oracle.layer_pool_page(r, th)
    assert scl.tolist() == [3.0, 2.0, np.float32(1e-8)]
    assert rad.tolist() == [[85, 255, 0], [255, 64, 0]]          # 0.5/2*255 = 63.75 -> 64
    assert t.tolist() == [[5, 44, 7], [64, 1, 255]]              # theta keeps the low byte (300 -> 44)


def test_layer_pool_half_even_rounding():
    # 1/2 * 255 = 127.5 -> 128 (even); 0.5/1 * 255 = 127.5 as well
    r = np.array([[1.0], [2.0]], np.float32)
    _, rad, _ = oracle.layer_pool_page(r, np.zeros((2, 1), np.int64))
    assert rad[:, 0].tolist() == [128, 255]


def test_layer_pool_tables_and_page_order():
    rng = np.random.default_rng(3)
    ps, dh, G_max, cap = 4, 16, 8, 4

    def run(b, n, G):
        return (b, n, rng.standard_normal((n, dh)).astype(np.float16),
                np.abs(rng.standard_normal((n, G))).astype(np.float32), rng.integers(0, 64, (n, G)))

    per_head = {0: [run(6, 5, 8), run(4, 2, 8)], 1: [run(3, 9, 4)]}
    tier = {6: (0, 8), 4: (1, 8), 3: (2, 4)}                     # b_theta -> (tier index, G)
    out = oracle.layer_pool(per_head, 2, ps, G_max, dh, cap, tier)
    # head 0: run of 5 -> pages 0 (4 tokens), 1 (1 token); run of 2 -> page 2;
    # head 1: run of 9 -> pages 3, 4 (4 each), 5 (1 token)
    assert out["num_pages_used"] == 6
    assert out["max_blocks"] == 3 + cap // 2 + 2
    assert out["block_table"].tolist() == [[0, 1, 2, -1, -1, -1, -1], [3, 4, 5, -1, -1, -1, -1]]
    assert out["bits_table"].tolist() == [[0, 0, 1, 0, 0, 0, 0], [2, 2, 2, 0, 0, 0, 0]]
    assert out["ctx_lens"].tolist() == [12, 12]
    assert out["theta"].shape == (6 + cap, ps, G_max)
    # V rows land page by page; unused slots and the capacity pages stay zero
    V0, V1 = per_head[0][0][2], per_head[1][0][2]
    assert (out["v_pool"][1, 0] == V0[4]).all() and (out["v_pool"][1, 1:] == 0).all()
    assert (out["v_pool"][4] == V1[4:8]).all() and (out["v_pool"][5, 0] == V1[8]).all()
    assert (out["v_pool"][6:] == 0).all()
    # page 5 holds head 1's last token in its first slot, G = 4 of G_max = 8 columns
    t, rad, scl = oracle.layer_pool_page(per_head[1][0][3][8:9], per_head[1][0][4][8:9])
    assert (out["radius"][5, 0, :4] == rad[0]).all() and (out["radius"][5, :, 4:] == 0).all()
    assert (out["r_scales"][5, :4] == scl).all() and (out["r_scales"][5, 4:] == 0).all()
    assert (out["theta"][5, 0, :4] == t[0]).all()
    # a page's r_scale is the max over its own tokens only (page 0: tokens 0..3 of the run)
    assert np.array_equal(out["r_scales"][0, :8], per_head[0][0][3][:4].max(0))


def test_layer_pool_empty_head():
    per_head = {0: [], 1: [(6, 3, np.ones((3, 16), np.float16), np.ones((3, 8), np.float32), np.zeros((3, 8)))]}
    out = oracle.layer_pool(per_head, 2, 16, 8, 16, 2, {6: (0, 8)})
    assert out["block_table"][0].tolist() == [-1] * out["max_blocks"]
    assert out["block_table"][1, 0] == 0 and out["ctx_lens"].tolist() == [0, 16]
    assert out["max_blocks"] == 1 + 2 // 2 + 2
