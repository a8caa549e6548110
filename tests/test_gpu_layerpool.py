"""GPU parity of the LayerPool drop-in (sphkv_lut.py:17-206): pools and
tables built by the constructor bit-exact with the oracle's restatement of
sphkv_lut.py:36-98, then a run of append_and_compute steps (crossing page
boundaries) against the oracle's append (decode_kernel.cu:10-84) and decode
(decode_kernel.cu:108-246): outputs within 2e-3, pools bit-exact."""
import numpy as np
import pytest
import torch

import oracle
import sphkv_format as fmt
from gpu_helpers import log, max_err

pytestmark = pytest.mark.gpu


class _Pipeline:
    def __init__(self, per_head_pages, codebooks):
        self.per_head_pages = per_head_pages
        self.codebooks = codebooks


def _unit(rng, shape):
    x = rng.standard_normal(shape)
    return (x / np.linalg.norm(x, axis=-1, keepdims=True)).astype(np.float32)


@pytest.mark.parametrize("page_size", [16, 128])
def test_layer_pool_build_and_steps(gpu, page_size):
    import sphkv_lut
    rng = np.random.default_rng(50 + page_size)
    num_kv, kvg, dh, layer = 4, 4, 128, 0
    tiers = fmt.build_tiers(dh)
    tmap = sphkv_lut.make_tier_idx_map(tiers)
    active = [t for t in tiers if t.tier_id != 0]
    G_max, cb_max, g_max = max(t.G for t in active), max(t.codebook_size for t in active), max(t.g for t in active)
    codebooks = {(layer, h, t.tier_id): _unit(rng, (t.G, t.codebook_size, t.g)) for h in range(num_kv) for t in active}
    per_head_pages, per_head_np = {}, {}
    for h in range(num_kv):
        tuples, nps = [], []
        for t in active:
            n = int(rng.integers(1, 3 * page_size))
            r = np.abs(rng.standard_normal((n, t.G)) * np.exp(rng.normal(0, 0.5, t.G))).astype(np.float32)
            th = rng.integers(0, t.codebook_size, size=(n, t.G)).astype(np.int64)
            V = rng.standard_normal((n, dh)).astype(np.float16)
            tuples.append((None, None, t.b_theta, n, torch.from_numpy(V), (torch.from_numpy(r), torch.from_numpy(th))))
            nps.append((t.b_theta, n, V, r, th))
        per_head_pages[(layer, h)] = tuples
        per_head_np[h] = nps
    pipe = _Pipeline(per_head_pages, {k: torch.from_numpy(v) for k, v in codebooks.items()})
    cap = 3 * num_kv
    pool = sphkv_lut.LayerPool(pipe, layer, page_size, G_max, cb_max, cap, gpu, tiers, tmap, num_kv * kvg, num_kv,
                               kvg, dh)
    torch.cuda.synchronize()
    want = oracle.layer_pool(per_head_np, num_kv, page_size, G_max, dh, cap,
                             {t.b_theta: (tmap[t.tier_id], t.G) for t in active})
    log(f"layer pool page_size={page_size} pages={want['num_pages_used']} max_blocks={want['max_blocks']}")
    assert pool.max_blocks == want["max_blocks"] and pool.num_pages_used == want["num_pages_used"]
    for name, t in (("theta", pool.theta_codes), ("radius", pool.radius_codes)):
        assert (t.cpu().numpy() == want[name]).all(), name
    assert (pool.r_scales.cpu().numpy().view(np.uint32) == want["r_scales"].view(np.uint32)).all()
    assert (pool.v_pool.cpu().numpy().view(np.uint16) == want["v_pool"].view(np.uint16)).all()
    assert (pool.block_table_gpu.cpu().numpy() == want["block_table"]).all()
    assert (pool.bits_table_gpu.cpu().numpy() == want["bits_table"]).all()
    assert (pool.ctx_lens_gpu.cpu().numpy() == want["ctx_lens"]).all()

    # decode steps: the oracle mirrors the bookkeeping of sphkv_lut.py:150-171
    cb_flat = np.zeros((num_kv, len(active), G_max, cb_max, g_max), np.float32)
    for t in active:
        for h in range(num_kv):
            cb_flat[h, tmap[t.tier_id], :t.G, :t.codebook_size, :t.g] = codebooks[(layer, h, t.tier_id)]
    dec = next(t for t in active if t.tier_id == 1)
    dec_cb = np.stack([codebooks[(layer, h, 1)] for h in range(num_kv)])
    tG = np.array([t.G for t in active], np.int32)
    tg = np.array([t.g for t in active], np.int32)
    th, rd, rs, vp = (want[k].copy() for k in ("theta", "radius", "r_scales", "v_pool"))
    bt, bits = want["block_table"].copy(), want["bits_table"].copy()
    ctx, n_used = int(want["ctx_lens"][0]), want["num_pages_used"]
    sm = 1.0 / np.sqrt(dh)
    pids = None
    worst = 0.0
    for step in range(page_size + 24):
        slot = ctx % page_size
        new = slot == 0
        if new:
            pg = ctx // page_size
            bt[:, pg] = n_used + np.arange(num_kv)
            bits[:, pg] = tmap[1]
            pids = (n_used + np.arange(num_kv)).astype(np.int64)
            n_used += num_kv
        ctx += 1
        q = rng.standard_normal((num_kv * kvg, dh)).astype(np.float32)
        k = (rng.standard_normal((num_kv, dh)) * np.exp(rng.normal(0, 0.5, (num_kv, dh)))).astype(np.float32)
        v = rng.standard_normal((num_kv, dh)).astype(np.float32)
        out = pool.append_and_compute(torch.from_numpy(q).to(gpu), torch.from_numpy(k).to(gpu),
                                      torch.from_numpy(v).to(gpu), tiers, sm)
        oracle.encode_append(k, v, dec_cb, th, rd, rs, vp, pids, slot, new)
        ref, _, _ = oracle.decode_mode_a(q, cb_flat, tG, tg, th, rd, rs, vp, bt, bits, kvg, sm)
        err = max_err(out.cpu().numpy(), ref)
        worst = max(worst, err)
        assert err <= 2e-3, (step, err)
    log(f"  {page_size + 24} steps, worst max abs err {worst:.3e}")
    assert (pool.theta_codes.cpu().numpy() == th).all() and (pool.radius_codes.cpu().numpy() == rd).all()
    assert (pool.r_scales.cpu().numpy().view(np.uint32) == rs.view(np.uint32)).all()
    assert (pool.v_pool.cpu().numpy().view(np.uint16) == vp.view(np.uint16)).all()
    assert (pool.block_table_gpu.cpu().numpy() == bt).all() and np.array_equal(pool.block_table_cpu, bt)
    assert (pool.ctx_lens_gpu.cpu().numpy() == want["ctx_lens"] + page_size + 24).all()
