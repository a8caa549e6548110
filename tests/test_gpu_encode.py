"""GPU parity of the fused encode kernel (bit-exact).

Pins: the committed torch fixtures (tests/golden/encode_golden.npz, torch CPU
running spherical_kv_pipeline.py:1136-1144 + pagebuilder.py:8-33) and the C
oracle on the full config-3 workload.
"""
import os

import numpy as np
import pytest
import torch

import oracle
import sphkv_format as fmt
import sphkv_ops as ops
import sphkv_synth as synth
from gpu_helpers import log, single_page_plan

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_encode_golden_fixtures(gpu):
    z = np.load(os.path.join(GOLD, "encode_golden.npz"))
    names = sorted({k.split("__")[0] for k in z.files if "__" in k})
    for name in names:
        N, tid, g, b, dh = (int(x) for x in z[name + "__meta"])
        log(f"encode fixture {name} N={N} tier={tid} dh={dh}")
        plan = single_page_plan(N, tid, dh)
        pool = ops.PagedPool.allocate(plan, {tid: z[name + "__cb"][None]}, gpu)
        K = torch.as_tensor(z[name + "__K"], device=gpu)
        V = torch.zeros_like(K)
        src = torch.as_tensor(np.where(plan.tokens >= 0, plan.tokens, -1), device=gpu)
        r_out = torch.zeros((1, 16, dh // 16), dtype=torch.float32, device=gpu)
        c_out = torch.zeros((1, 16, dh // 16), dtype=torch.int32, device=gpu)
        ops.encode_pages(pool, K, V, src, r_out, c_out)
        torch.cuda.synchronize()
        G = dh // g
        page = pool.pages.cpu().numpy()[: z[name + "__page"].size]
        r = r_out.cpu().numpy()[0, :N, :G]
        c = c_out.cpu().numpy()[0, :N, :G]
        assert (r.view(np.uint32) == z[name + "__r"].view(np.uint32)).all(), name
        assert (c == z[name + "__codes"]).all(), name
        assert (page == z[name + "__page"]).all(), name


def test_encode_fp32_input_matches_fp16(gpu):
    # the reference feeds K.float(); fp32 input of the same values is identical
    z = np.load(os.path.join(GOLD, "encode_golden.npz"))
    name = "t1_n16_c3"
    plan = single_page_plan(16, 1, 128)
    outs = []
    for dt in (torch.float16, torch.float32):
        pool = ops.PagedPool.allocate(plan, {1: z[name + "__cb"][None]}, gpu)
        K = torch.as_tensor(z[name + "__K"], device=gpu).to(dt)
        ops.encode_pages(pool, K, torch.zeros(K.shape, dtype=torch.float16, device=gpu),
                         torch.as_tensor(plan.tokens, device=gpu))
        outs.append(pool.pages.cpu().numpy())
    assert (outs[0] == outs[1]).all()
    assert (outs[0][: z[name + "__page"].size] == z[name + "__page"]).all()


@pytest.mark.parametrize("config", [3, 2, 1])
def test_encode_full_workload_vs_oracle(gpu, config):
    wl = synth.make_encode_workload() if config == 3 else synth.make_decode_workload(config)
    log(f"encode full config{config}: rows={wl.plan.num_rows}")
    pool, r_out, c_out = ops.build_pool_gpu(wl, gpu, with_codes=True)
    torch.cuda.synchronize()
    cpu = oracle.build_pool(wl, with_codes=True)
    pages = pool.pages.cpu().numpy()
    assert (pages == cpu["pages"]).all(), f"{int((pages != cpu['pages']).sum())} page bytes differ"
    assert (pool.v_pool.cpu().numpy().view(np.uint16) == cpu["v_pool"].view(np.uint16)).all()
    r, c = r_out.cpu().numpy(), c_out.cpu().numpy()
    comp = wl.plan.tier != fmt.DENSE_TIER_ID
    assert (c[comp] == cpu["codes"][comp]).all()
    assert (r[comp].view(np.uint32) == cpu["r"][comp].view(np.uint32)).all()


def test_encode_partial_and_edge_pages(gpu):
    # ragged tier lists: pages with 1..16 tokens, tier 3, dense, dh 64 and 128
    rng = np.random.default_rng(11)
    for dh in (64, 128):
        L = 173
        tier_of = [rng.choice(np.array([1, 2, 3, fmt.DENSE_TIER_ID], np.int32), size=L) for _ in range(3)]
        cbs = synth.make_codebooks(rng, 3, dh, [1, 2, 3])
        K = [(rng.standard_normal((3, L, dh)) * 3).astype(np.float16)]
        V = [rng.standard_normal((3, L, dh)).astype(np.float16)]
        plan = fmt.plan_pages(tier_of, None, 1, 3, dh, 16, rng=rng, num_vpages=None)
        wl = synth.Workload(name="edge", dh=dh, num_kv=3, gqa=1, num_seqs=1, lengths=[L], rope_theta=5e5,
                            codebooks=cbs, K=K, V=V, q=np.zeros((1, 3, dh), np.float16), tier_of=tier_of,
                            plan=plan)
        log(f"encode edge dh={dh} rows={plan.num_rows} counts={sorted(set(plan.count.tolist()))}")
        pool, r_out, c_out = ops.build_pool_gpu(wl, gpu, with_codes=True)
        torch.cuda.synchronize()
        cpu = oracle.build_pool(wl, with_codes=True)
        assert (pool.pages.cpu().numpy() == cpu["pages"]).all()
        assert (pool.v_pool.cpu().numpy().view(np.uint16) == cpu["v_pool"].view(np.uint16)).all()


def test_encode_near_ties_and_degenerate_groups(gpu):
    # Keys built to stress the nearest-centroid search: the sum of two
    # centroids of the group (an exact tie in real arithmetic, decided by the
    # rounding of the reference's fp32 dot products), a centroid itself at
    # several scales, a centroid plus a tiny share of another, and all-zero
    # groups.  Codes and radii must match the C oracle bit for bit.
    rng = np.random.default_rng(23)
    dh, H, L = 128, 2, 160
    tier_of = [np.array([[1, 2, 3][(i + h) % 3] for i in range(L)], np.int32) for h in range(H)]
    cbs = synth.make_codebooks(rng, H, dh, [1, 2, 3])
    K = np.zeros((H, L, dh), np.float32)
    for h in range(H):
        for t in range(L):
            tid = int(tier_of[h][t])
            cb = cbs[tid][h]                      # [G, C, g]
            G, C, g = cb.shape
            for j in range(G):
                a, b = rng.choice(C, size=2, replace=False)
                kind = (t + j) % 5
                if kind == 0:
                    v = cb[j, a] + cb[j, b]
                elif kind == 1:
                    v = cb[j, a] * np.float32(2.0 ** rng.integers(-6, 7))
                elif kind == 2:
                    v = cb[j, a] + np.float32(1e-3) * cb[j, b]
                elif kind == 3:
                    v = np.zeros(g, np.float32)
                else:
                    v = (cb[j, a] - cb[j, b]) * np.float32(0.5)
                K[h, t, j * g:(j + 1) * g] = v
    K16 = [K.astype(np.float16)]
    V = [rng.standard_normal((H, L, dh)).astype(np.float16)]
    plan = fmt.plan_pages(tier_of, None, 1, H, dh, 16, rng=rng, num_vpages=None)
    wl = synth.Workload(name="ties", dh=dh, num_kv=H, gqa=1, num_seqs=1, lengths=[L], rope_theta=5e5,
                        codebooks=cbs, K=K16, V=V, q=np.zeros((1, H, dh), np.float16), tier_of=tier_of,
                        plan=plan)
    log(f"encode near-ties dh={dh} rows={plan.num_rows}")
    pool, r_out, c_out = ops.build_pool_gpu(wl, gpu, with_codes=True)
    torch.cuda.synchronize()
    cpu = oracle.build_pool(wl, with_codes=True)
    r, c = r_out.cpu().numpy(), c_out.cpu().numpy()
    comp = wl.plan.tier != fmt.DENSE_TIER_ID
    assert (c[comp] == cpu["codes"][comp]).all(), f"{int((c[comp] != cpu['codes'][comp]).sum())} codes differ"
    assert (r[comp].view(np.uint32) == cpu["r"][comp].view(np.uint32)).all()
    assert (pool.pages.cpu().numpy() == cpu["pages"]).all()


@pytest.mark.parametrize("kind", ["scaled", "raw", "near_unit"])
def test_encode_non_unit_codebooks_bit_exact(gpu, kind):
    # _encode_keys_with_codebooks (spherical_kv_pipeline.py:1130-1144) takes
    # any codebook; only codebook_loader.py:43-44 normalises the rows.  Rows
    # scaled by 0.5..3, raw N(0,1) rows, and rows 1% off unit length (inside
    # the pre-ranking bound) must all give the oracle's codes, radii and pages.
    rng = np.random.default_rng({"scaled": 31, "raw": 32, "near_unit": 33}[kind])
    dh, H, L = 128, 2, 200
    tier_of = [rng.choice(np.array([1, 2, 3], np.int32), size=L) for _ in range(H)]
    cbs = synth.make_codebooks(rng, H, dh, [1, 2, 3])
    for tid, cb in cbs.items():
        if kind == "scaled":
            cb *= rng.uniform(0.5, 3.0, size=cb.shape[:-1] + (1,)).astype(np.float32)
        elif kind == "raw":
            cb[:] = rng.standard_normal(cb.shape).astype(np.float32)
        else:
            cb *= np.float32(1.01)
    # keys on near-ties of the scaled rows: c_a + c_b and c_a + 1e-3 c_b, plus plain ones
    K = np.zeros((H, L, dh), np.float32)
    for h in range(H):
        for t in range(L):
            cb = cbs[int(tier_of[h][t])][h]
            G, C, g = cb.shape
            for j in range(G):
                a, b = rng.choice(C, size=2, replace=False)
                m = (t + j) % 3
                v = cb[j, a] + cb[j, b] if m == 0 else (cb[j, a] + np.float32(1e-3) * cb[j, b] if m == 1
                                                         else rng.standard_normal(g).astype(np.float32))
                K[h, t, j * g:(j + 1) * g] = v
    V = [rng.standard_normal((H, L, dh)).astype(np.float16)]
    plan = fmt.plan_pages(tier_of, None, 1, H, dh, 16, rng=rng, num_vpages=None)
    wl = synth.Workload(name=f"nonunit_{kind}", dh=dh, num_kv=H, gqa=1, num_seqs=1, lengths=[L], rope_theta=5e5,
                        codebooks=cbs, K=[K.astype(np.float16)], V=V, q=np.zeros((1, H, dh), np.float16),
                        tier_of=tier_of, plan=plan)
    log(f"encode non-unit codebooks ({kind}) rows={plan.num_rows}")
    pool, r_out, c_out = ops.build_pool_gpu(wl, gpu, with_codes=True)
    torch.cuda.synchronize()
    cpu = oracle.build_pool(wl, with_codes=True)
    r, c = r_out.cpu().numpy(), c_out.cpu().numpy()
    comp = wl.plan.tier != fmt.DENSE_TIER_ID
    assert (c[comp] == cpu["codes"][comp]).all(), f"{int((c[comp] != cpu['codes'][comp]).sum())} codes differ"
    assert (r[comp].view(np.uint32) == cpu["r"][comp].view(np.uint32)).all()
    assert (pool.pages.cpu().numpy() == cpu["pages"]).all()
