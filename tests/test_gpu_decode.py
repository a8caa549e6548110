"""GPU parity of the paged angle-domain decode and the ragged logits kernel.

Tolerance (north star): max-abs error <= 2e-3 of the fp16 decode output
against the fp64 oracle evaluated on the page-decoded radius
r_hat = int8 / 127 * scale, the same centroids, positions and fp16 V.
"""
import numpy as np
import pytest
import torch

import oracle
import sphkv_format as fmt
import sphkv_ops as ops
import sphkv_synth as synth
from gpu_helpers import log, max_err, pool_from_oracle

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _decode(pool, wl, gpu):
    q = torch.as_tensor(wl.q, device=gpu)
    out = ops.decode_paged(pool, q, wl.gqa, wl.rope_theta, check=True)     # raises on a skipped page
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


@pytest.mark.parametrize("config,ctx", [(1, None), (2, 4096), (2, None), (5, 4096), (4, 3000)])
def test_decode_matches_oracle(gpu, config, ctx):
    kw = {"num_seqs_override": 6} if config == 4 else ({"num_seqs_override": 2} if config == 5 else {})
    wl = synth.make_decode_workload(config, ctx_override=ctx, **kw)
    log(f"decode config{config} ctx={ctx} seqs={wl.num_seqs} rows={wl.plan.num_rows} gqa={wl.gqa}")
    pool, cpu = pool_from_oracle(wl, gpu)
    got = _decode(pool, wl, gpu)
    want = oracle.decode_mode_b(cpu, wl.plan, wl.codebooks, wl.q, wl.gqa, wl.rope_theta)
    err = max_err(got, want)
    log(f"  max abs err {err:.3e}")
    assert err <= TOL


def test_decode_gpu_encoded_pool_matches_oracle_pool(gpu):
    # end to end: GPU encode then GPU decode equals decode of the oracle pool
    wl = synth.make_decode_workload(2, ctx_override=6000)
    pool_g, _, _ = ops.build_pool_gpu(wl, gpu)
    pool_c, cpu = pool_from_oracle(wl, gpu)
    a, b = _decode(pool_g, wl, gpu), _decode(pool_c, wl, gpu)
    assert (a == b).all()


def test_decode_work_split_invariance(gpu):
    # splitting the context into more / fewer work items only reorders the
    # log-sum-exp merge
    wl = synth.make_decode_workload(2, ctx_override=5000)
    outs = []
    for rpi in (4, 32, 4096):
        pool, cpu = pool_from_oracle(wl, gpu, rows_per_item=rpi)
        outs.append(_decode(pool, wl, gpu))
    assert max_err(outs[0], outs[1]) < 2e-3 * 0.25 and max_err(outs[1], outs[2]) < 2e-3 * 0.25


def test_decode_long_items_matches_oracle(gpu):
    # one work item per (seq, head): ~1,300 pages per item, over 100 per wave,
    # so each wave's page table is reloaded (and rechecked) past its 64th page
    wl = synth.make_decode_workload(2, ctx_override=20000)
    pool, cpu = pool_from_oracle(wl, gpu, rows_per_item=1 << 20)
    per_item = np.diff(pool.work_start.cpu().numpy())
    assert per_item.max() == 1 and pool.num_items == wl.num_kv
    got = _decode(pool, wl, gpu)
    want = oracle.decode_mode_b(cpu, wl.plan, wl.codebooks, wl.q, wl.gqa, wl.rope_theta)
    err = max_err(got, want)
    log(f"long items: {pool.num_items} items, rows {wl.plan.tokens.shape[0]}, max abs err {err:.3e}")
    assert err <= TOL


def test_decode_interleaved_and_contiguous_items_agree(gpu):
    # the same pool decoded with interleaved (strided) and contiguous work
    # items: only the order of the log-sum-exp merge differs
    wl = synth.make_decode_workload(2, ctx_override=6000)
    pool, cpu = pool_from_oracle(wl, gpu, rows_per_item=32)
    w, ws = ops.make_work(wl.plan.row_start, 32, interleave=False)
    pool2 = ops.PagedPool(**{**pool.__dict__, "work": torch.as_tensor(w, device=gpu),
                             "work_start": torch.as_tensor(ws, device=gpu)})
    a, b = _decode(pool, wl, gpu), _decode(pool2, wl, gpu)
    want = oracle.decode_mode_b(cpu, wl.plan, wl.codebooks, wl.q, wl.gqa, wl.rope_theta)
    assert max_err(a, want) <= 2e-3 and max_err(b, want) <= 2e-3
    assert max_err(a, b) < 2e-3 * 0.25


def test_decode_malformed_work_items_stay_in_bounds(gpu):
    # work items naming no (seq, head), negative or past-the-end rows and
    # absurd strides are clamped by the kernels: the call completes and the
    # well-formed items' heads are decoded as before
    wl = synth.make_decode_workload(2, ctx_override=3000)
    pool, cpu = pool_from_oracle(wl, gpu)
    ref = _decode(pool, wl, gpu)
    w = pool.work.cpu().numpy().copy()
    ws = pool.work_start.cpu().numpy()
    bad = w.copy()
    last = ws[-2]                                     # first item of the last (seq, head)
    bad[last:, 0] = 1 << 30                           # names no (seq, head)
    bad[last:, 1] = -(1 << 30)
    bad[last:, 2] = 1 << 30
    bad[last:, 3] = 1 << 30
    p2 = ops.PagedPool(**{**pool.__dict__, "work": torch.as_tensor(bad, device=gpu)})
    got = _decode(p2, wl, gpu)
    gqa = wl.gqa
    h_last = wl.plan.num_kv - 1
    keep = np.ones(got.shape[1], bool)
    keep[h_last * gqa:(h_last + 1) * gqa] = False
    assert (got[:, keep] == ref[:, keep]).all()
    assert np.isfinite(got).all()


def test_decode_edge_cases(gpu):
    rng = np.random.default_rng(3)
    dh, num_kv, gqa = 128, 4, 4
    # head 0: 1 token; head 1: empty; head 2: 17 tokens mixed tiers; head 3: all dense 33
    Ls = [1, 0, 17, 33]
    L = 40
    tier_of = []
    for h, n in enumerate(Ls):
        t = np.zeros(L, np.int32)
        if h == 2:
            t[:n] = rng.choice(np.array([1, 2, 3, fmt.DENSE_TIER_ID], np.int32), size=n)
        elif h == 3:
            t[:n] = fmt.DENSE_TIER_ID
        else:
            t[:n] = 1
        tier_of.append(t)
    cbs = synth.make_codebooks(rng, num_kv, dh, [1, 2, 3])
    K = [(rng.standard_normal((num_kv, L, dh)) * 2).astype(np.float16)]
    V = [rng.standard_normal((num_kv, L, dh)).astype(np.float16)]
    q = (rng.standard_normal((1, num_kv * gqa, dh)) * 2).astype(np.float16)
    pos = [np.sort(rng.choice(120000, size=L, replace=False))]
    plan = fmt.plan_pages(tier_of, pos, 1, num_kv, dh, 16, rng=rng)
    wl = synth.Workload(name="edge", dh=dh, num_kv=num_kv, gqa=gqa, num_seqs=1, lengths=[L],
                        rope_theta=5e5, codebooks=cbs, K=K, V=V, q=q, tier_of=tier_of, plan=plan, positions=pos)
    pool, cpu = pool_from_oracle(wl, gpu)
    got = _decode(pool, wl, gpu)
    want = oracle.decode_mode_b(cpu, plan, cbs, q, gqa, 5e5)
    assert max_err(got, want) <= TOL
    assert (got[0, gqa:2 * gqa] == 0).all()             # empty head -> zeros
    # single token -> exactly its V row (fp16)
    assert max_err(got[0, :gqa], np.broadcast_to(V[0][0, 0].astype(np.float32), (gqa, dh))) == 0.0


@pytest.mark.parametrize("dh,gqa", [(128, 4), (64, 1), (128, 2), (128, 8), (128, 1), (64, 2), (64, 4), (64, 8)])
def test_decode_partial_and_far_pages(gpu, dh, gqa):
    # Every tier with a partial last page (250 tokens: 15 full pages + 10);
    # pages whose tokens lie 10 positions apart (|pos - centre| up to 75: the
    # far rows of the phasor table); and pages whose tokens lie 14 positions
    # apart (page span > the phasor table, so the direct phasors run), full
    # and partial.  Logits span several units, so a token's weight depends on
    # its own logit.
    rng = np.random.default_rng(19)
    H = 2
    cases = [("dense", 250, lambda i: fmt.DENSE_TIER_ID), ("t1", 250, lambda i: 1), ("t2", 250, lambda i: 2),
             ("t3", 250, lambda i: 3), ("wide", 1600, lambda i: 1 if i % 10 == 0 else fmt.DENSE_TIER_ID),
             ("far", 2240, lambda i: 1 if i % 14 == 0 else fmt.DENSE_TIER_ID),
             ("far-partial", 2100, lambda i: 1 if i % 14 == 0 else 2)]
    for name, L, tier in cases:
        tier_of = [np.array([tier(i) for i in range(L)], np.int32) for _ in range(H)]
        cbs = synth.make_codebooks(rng, H, dh, [1, 2, 3])
        K = [rng.standard_normal((H, L, dh)).astype(np.float16)]
        V = [rng.standard_normal((H, L, dh)).astype(np.float16)]
        q = (rng.standard_normal((1, H * gqa, dh)) * 2).astype(np.float16)
        plan = fmt.plan_pages(tier_of, None, 1, H, dh, 16, rng=rng)
        wl = synth.Workload(name=name, dh=dh, num_kv=H, gqa=gqa, num_seqs=1, lengths=[L], rope_theta=5e5,
                            codebooks=cbs, K=K, V=V, q=q, tier_of=tier_of, plan=plan)
        log(f"decode partial/far {name} dh={dh} gqa={gqa} counts={sorted(set(plan.count.tolist()))}")
        pool, cpu = pool_from_oracle(wl, gpu)
        err = max_err(_decode(pool, wl, gpu), oracle.decode_mode_b(cpu, plan, cbs, q, gqa, 5e5))
        log(f"  max abs err {err:.3e}")
        assert err <= TOL, name


def test_decode_masked_positions(gpu):
    # slots with position -1 are excluded even inside full pages
    wl = synth.make_decode_workload(1, ctx_override=512)
    pool, cpu = pool_from_oracle(wl, gpu)
    pos = wl.plan.positions.copy()
    rng = np.random.default_rng(5)
    drop = rng.random(pos.shape) < 0.3
    pos[drop] = -1
    pool.positions.copy_(torch.from_numpy(pos))
    got = _decode(pool, wl, gpu)
    plan2 = fmt.PagePlan(**{**wl.plan.__dict__, "positions": pos})
    # oracle: rebuild the token lists without the dropped slots
    want = np.zeros_like(got, np.float64)
    inv = oracle.rope_inv_freq(wl.dh, wl.rope_theta)
    for h in range(wl.num_kv):
        lg, vs = [], []
        qh = wl.q[0, h * wl.gqa:(h + 1) * wl.gqa].astype(np.float64)
        for p in range(int(plan2.row_start[h]), int(plan2.row_start[h + 1])):
            n = int(plan2.count[p])
            keep = np.nonzero(pos[p, :n] >= 0)[0]
            if keep.size == 0:
                continue
            codes, r_hat = oracle.unpack_page(cpu["pages"], plan2.ptable[p], 1, n, wl.dh)
            cb = wl.codebooks[1][h].astype(np.float64)
            cw = cb[np.arange(4)[None, :], codes[keep]]
            ang = pos[p, keep][:, None].astype(np.float64) * inv[None]
            ang = np.concatenate([ang, ang], 1)
            lg.append(oracle.mode_b_logits(qh, None, np.cos(ang), np.sin(ang), cw, r_hat[keep], None, 4, 16))
            vs.append(oracle.v_page_rows(cpu["v_pool"], plan2.vslot[p], n, wl.dh)[keep].astype(np.float64))
        lgc = np.concatenate(lg, 1)
        e = np.exp(lgc - lgc.max(1, keepdims=True))
        want[0, h * wl.gqa:(h + 1) * wl.gqa] = (e / e.sum(1, keepdims=True)) @ np.concatenate(vs, 0)
    assert max_err(got, want) <= TOL


@pytest.mark.parametrize("ctx", [3000, 8192, 32768])
def test_ragged_logits_matches_oracle(gpu, ctx):
    # 8192 tokens: > 2048 tier-1 chunks, so the pipelined kernel runs its full
    # grid with the XCD-aware work split; 32768: config 2 at full size (the
    # bench line's workload)
    import fused_decode
    wl = synth.make_decode_workload(2, ctx_override=ctx)
    cpu = oracle.build_pool(wl)
    plan = wl.plan
    for tid, (g, b) in ((1, (16, 6)), (2, (16, 4))):
        rows = [p for p in range(plan.num_rows) if plan.tier[p] == tid]
        heads = (plan.seq_head[rows] % plan.num_kv).astype(np.int32)
        G = wl.dh // g
        max_pos = ctx + 100
        cos_t, sin_t = fmt.rope_tables(max_pos, wl.dh, wl.rope_theta)
        pos = plan.positions[rows].reshape(-1).astype(np.int32)
        q = wl.q[0].astype(np.float32)
        cb = wl.codebooks[tid].reshape(plan.num_kv * G, 2 ** b, g)
        log(f"ragged tier {tid}: pages={len(rows)}")
        got = fused_decode.fused_decode_ragged(
            torch.as_tensor(cpu["pages"], device=gpu), torch.as_tensor(plan.ptable[rows], device=gpu),
            torch.as_tensor(heads, device=gpu), torch.as_tensor(pos, device=gpu),
            torch.as_tensor(cos_t, device=gpu), torch.as_tensor(sin_t, device=gpu),
            torch.as_tensor(q, device=gpu), wl.gqa, plan.num_kv, torch.as_tensor(cb, device=gpu),
            wl.dh, G, g, b, 16)
        torch.cuda.synchronize()
        want = oracle.ragged_logits(cpu["pages"], plan.ptable[rows], heads, pos, cos_t, sin_t, q, wl.gqa,
                                    cb, wl.dh, G, g, b, 16)
        got = got.cpu().numpy()
        fin = np.isfinite(want)
        assert (np.isneginf(got) == ~fin).all()
        assert max_err(got[fin], want[fin]) < 2e-4


def _reference_layout_case(tid, page_size, dh, grp, num_kv, L=300):
    """Pages of num_kv heads laid out back to back as _build_per_head_pages
    does (spherical_kv_pipeline.py:1198-1213), one masked token in each head's
    first page; returns the fused_decode_ragged inputs as numpy arrays."""
    from oracle import paging
    rng = np.random.default_rng(700 + tid + page_size + dh + grp + num_kv)
    g, b = fmt.TIER_GEOMETRY[tid]
    G = dh // g
    cbs = synth.make_codebooks(rng, num_kv, dh, [tid])[tid]
    buf, ptab, heads, pos = [], [], [], []
    base = 0
    for h in range(num_kv):
        K = (rng.standard_normal((L, dh)) * np.exp(rng.normal(0, 0.5, dh))).astype(np.float16)
        idx = np.sort(rng.choice(4000, size=L, replace=False))
        counts = [min(page_size, L - s) for s in range(0, L, page_size)]
        rows = paging.page_offsets(tid, counts, dh).astype(np.int64) + base
        for ci, s0 in enumerate(range(0, L, page_size)):
            n = counts[ci]
            r, codes = oracle.encode_groups(K[s0:s0 + n].astype(np.float32), cbs[h])
            buf.append(oracle.build_page(r, codes, tid, b))
            pp = np.full(page_size, -1, np.int32)
            pp[:n] = idx[s0:s0 + n]
            if ci == 0:
                pp[3] = -1                                   # a masked token inside the page
            pos.append(pp)
            heads.append(h)
        ptab.append(rows)
        base += sum(x.size for x in buf[len(buf) - len(counts):])
    cos_t, sin_t = fmt.rope_tables(4100, dh, 500000.0)
    return dict(pages=np.concatenate(buf), ptable=np.concatenate(ptab).astype(np.int32),
                heads=np.asarray(heads, np.int32), pos=np.concatenate(pos).astype(np.int32), cos_t=cos_t,
                sin_t=sin_t, q=rng.standard_normal((num_kv * grp, dh)).astype(np.float32),
                cb=cbs.reshape(num_kv * G, 2 ** b, g), G=G, g=g, b=b)


def _ragged_gpu(c, gpu, grp, num_kv, dh, page_size):
    import fused_decode
    got = fused_decode.fused_decode_ragged(
        torch.as_tensor(c["pages"], device=gpu), torch.as_tensor(c["ptable"], device=gpu),
        torch.as_tensor(c["heads"], device=gpu), torch.as_tensor(c["pos"], device=gpu),
        torch.as_tensor(c["cos_t"], device=gpu), torch.as_tensor(c["sin_t"], device=gpu),
        torch.as_tensor(c["q"], device=gpu), grp, num_kv, torch.as_tensor(c["cb"], device=gpu), dh, c["G"], c["g"],
        c["b"], page_size)
    torch.cuda.synchronize()
    return got.cpu().numpy()


@pytest.mark.parametrize("tid,page_size,dh,grp,num_kv", [
    (1, 128, 128, 4, 2), (3, 128, 128, 4, 2), (3, 16, 128, 4, 2), (2, 128, 64, 4, 2), (1, 16, 128, 8, 2),
    (3, 32, 64, 6, 2), (2, 48, 128, 1, 2), (1, 16, 64, 3, 2), (1, 24, 128, 4, 2), (2, 128, 128, 9, 2),
    (1, 16, 128, 8, 9), (2, 32, 64, 5, 11)])
def test_ragged_logits_reference_page_size_and_tier3(gpu, tid, page_size, dh, grp, num_kv):
    # the reference's call shape: PAGE_SIZE = 128 pages (config.py:4,
    # spherical_kv_pipeline.py:1109-1125) and tier-3 decode pages (:1900-1910);
    # page_size 24 and grp 9 take the general kernel; 9 heads x grp 8 at dh
    # 128 (q 36 KB, over the LDS budget) the one-chunk-per-wave form; the rest
    # the pipeline (11 heads: codebooks restaged at each head change).  The
    # pools' byte sizes are not multiples of 4 (the last dword is partial).
    L = 300
    c = _reference_layout_case(tid, page_size, dh, grp, num_kv, L)
    log(f"ragged tier {tid}, page_size {page_size}, dh {dh}, grp {grp}: {c['ptable'].shape[0]} pages, "
        f"pool {c['pages'].size} bytes")
    got = _ragged_gpu(c, gpu, grp, num_kv, dh, page_size)
    want = oracle.ragged_logits(c["pages"], c["ptable"], c["heads"], c["pos"], c["cos_t"], c["sin_t"], c["q"], grp,
                                c["cb"], dh, c["G"], c["g"], c["b"], page_size)
    fin = np.isfinite(want)
    assert fin.sum() == num_kv * (L - 1) * grp                  # every token but the masked ones
    assert (np.isneginf(got) == ~fin).all()
    assert max_err(got[fin], want[fin]) < 2e-4


@pytest.mark.parametrize("tid,page_size,dh,grp,num_kv", [(1, 16, 128, 4, 2), (2, 16, 64, 4, 3), (3, 128, 128, 4, 2),
                                                          (1, 24, 128, 4, 2)])
def test_ragged_logits_malformed_rows_contribute_nothing(gpu, tid, page_size, dh, grp, num_kv):
    # pointer-table rows with a negative offset, a page past the pool's end,
    # sections past it, or a head id out of range: every slot of such a page
    # is -inf and every other page's logits are unchanged
    c = _reference_layout_case(tid, page_size, dh, grp, num_kv)
    P = c["ptable"].shape[0]
    bad = {1: "neg_page", 2: "neg_theta", P // 2: "page_past_end", P // 2 + 1: "sections_past_end",
           P - 2: "head_out_of_range"}
    want = oracle.ragged_logits(c["pages"], c["ptable"], c["heads"], c["pos"], c["cos_t"], c["sin_t"], c["q"], grp,
                                c["cb"], dh, c["G"], c["g"], c["b"], page_size)
    pt, hd = c["ptable"].copy(), c["heads"].copy()
    nb = c["pages"].size
    for p, kind in bad.items():
        if kind == "neg_page":
            pt[p, 0] = -16
        elif kind == "neg_theta":
            pt[p, 1] = -1
        elif kind == "page_past_end":
            pt[p] = (nb + 64, nb + 64 + 8 + 4 * c["G"], nb + 64 + 200)
        elif kind == "sections_past_end":
            pt[p, 1:] = (nb + 8, nb + 400)
        else:
            hd[p] = num_kv + 3
        want[:, p * page_size:(p + 1) * page_size] = -np.inf
    log(f"ragged malformed rows: tier {tid}, page_size {page_size}, dh {dh}, {P} pages, bad {sorted(bad)}")
    got = _ragged_gpu(dict(c, ptable=pt, heads=hd), gpu, grp, num_kv, dh, page_size)
    fin = np.isfinite(want)
    assert (np.isneginf(got) == ~fin).all()
    assert max_err(got[fin], want[fin]) < 2e-4


def test_decode_split_phases_equal_fused_call(gpu):
    # partials + merge as two calls give exactly the one-call result, and the
    # partials merge (fp64, on the host) to the same output
    wl = synth.make_decode_workload(2, ctx_override=3000)
    pool, _ = pool_from_oracle(wl, gpu, rows_per_item=24)
    q = torch.as_tensor(wl.q, device=gpu)
    ref = ops.decode_paged(pool, q, wl.gqa, wl.rope_theta)
    ws = torch.zeros(pool.workspace_bytes(wl.gqa), dtype=torch.uint8, device=gpu)
    part = ops.decode_paged_partials(pool, q, wl.gqa, wl.rope_theta, ws)
    out = ops.merge_partials(pool, ws, wl.gqa, torch.empty_like(q))
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    P = part.double().cpu().numpy()
    ws_h = pool.work_start.cpu().numpy()
    G, DH = wl.gqa, wl.dh
    host = np.zeros((wl.num_kv * G, DH))
    for sh in range(wl.num_kv):
        rows = P[ws_h[sh]:ws_h[sh + 1]]
        m, l, acc = rows[:, :G], rows[:, G:2 * G], rows[:, 16:].reshape(-1, G, DH)
        M = m.max(0)
        f = np.where(np.isfinite(m), np.exp2(m - M), 0.0)
        host[sh * G:(sh + 1) * G] = (f[:, :, None] * acc).sum(0) / (f * l).sum(0)[:, None]
    assert max_err(out[0].float().cpu().numpy(), host) < 1e-3


def _drop_rows(plan, drop):
    """The plan without the given rows (page bytes stay where they are)."""
    keep = np.setdiff1d(np.arange(plan.num_rows), np.asarray(sorted(drop)))
    sh = plan.seq_head[keep]
    rs = np.searchsorted(sh, np.arange(plan.num_seqs * plan.num_kv + 1), side="left").astype(np.int32)
    return fmt.PagePlan(dh=plan.dh, page_size=plan.page_size, num_seqs=plan.num_seqs, num_kv=plan.num_kv,
                        tier=plan.tier[keep], count=plan.count[keep], tokens=plan.tokens[keep],
                        positions=plan.positions[keep], seq_head=sh, row_start=rs, ptable=plan.ptable[keep],
                        vslot=plan.vslot[keep], pages_bytes=plan.pages_bytes, num_vpages=plan.num_vpages)


def test_decode_v_slots_beyond_2_pow_20(gpu):
    # regression of the 64-bit V-page offset: every row's V page sits at a
    # slot >= 2^20 (element offset >= 2^31 at dh 128) in a 1.31M-page pool;
    # the decode must equal the same pool with compact slots, bit for bit,
    # and the oracle within 2e-3
    wl = synth.make_decode_workload(2, ctx_override=4096)
    P = wl.plan.num_rows
    rng = np.random.default_rng(21)
    hi_slots = ((1 << 20) + rng.choice(1 << 18, size=P, replace=False)).astype(np.int32)
    plan_hi = fmt.PagePlan(**{**wl.plan.__dict__, "vslot": hi_slots, "num_vpages": (1 << 20) + (1 << 18)})
    log(f"vslots in [{int(hi_slots.min())}, {int(hi_slots.max())}], pool {plan_hi.num_vpages} pages")
    pool_hi, _, _ = ops.build_pool_gpu(synth.Workload(**{**wl.__dict__, "plan": plan_hi}), gpu)
    pool_lo, cpu = pool_from_oracle(wl, gpu)
    q = torch.as_tensor(wl.q, device=gpu)
    a = ops.decode_paged(pool_hi, q, wl.gqa, wl.rope_theta, check=True)
    b = ops.decode_paged(pool_lo, q, wl.gqa, wl.rope_theta, check=True)
    assert torch.equal(a, b)
    want = oracle.decode_mode_b(cpu, wl.plan, wl.codebooks, wl.q, wl.gqa, wl.rope_theta)
    assert max_err(a.float().cpu().numpy(), want) <= TOL
    del pool_hi


def test_decode_malformed_rows_past_the_first_page_table(gpu):
    # one work item per (seq, head), so wave w's page k is the head's row
    # w + 12 k: rows past 12 * 64 = 768 sit in a wave's second page table
    # (loaded and checked after its 64th page); four malformed rows there are
    # skipped and counted like the others (this layout puts every dense page,
    # the sink tokens' tier, in the first table)
    wl = synth.make_decode_workload(2, ctx_override=20000)
    pool, cpu = pool_from_oracle(wl, gpu, rows_per_item=1 << 20)
    plan = wl.plan
    rs = plan.row_start
    assert pool.num_items == wl.num_kv and min(np.diff(rs)) > 900
    comp = [p for p in range(rs[2] + 800, rs[3]) if plan.tier[p] == 1]
    r_off, r_vs, r_tier, r_sec = int(rs[1]) + 801, int(rs[4]) + 870, int(rs[5]) + 900, comp[4]
    assert min(r - rs[h] for r, h in [(r_off, 1), (r_vs, 4), (r_tier, 5), (r_sec, 2)]) >= 12 * 64
    pt = plan.ptable.copy()
    vs = plan.vslot.copy()
    pt[r_off, 0] = -16                                 # page offset outside the pool
    vs[r_vs] = plan.num_vpages + 5                     # V slot outside the V pool
    pt[r_sec, 2] += 600                                # radius section beyond the 512-byte window
    pages = pool.pages.clone()
    pages[int(plan.ptable[r_tier, 0])] = 7             # unknown tier id
    bad = ops.PagedPool(**{**pool.__dict__, "ptable": torch.as_tensor(pt, device=gpu),
                           "vslot": torch.as_tensor(vs, device=gpu), "pages": pages})
    q = torch.as_tensor(wl.q, device=gpu)
    ws = torch.zeros(pool.workspace_bytes(wl.gqa), dtype=torch.uint8, device=gpu)
    out = ops.decode_paged(bad, q, wl.gqa, wl.rope_theta, workspace=ws)
    assert ops.decode_status(bad, ws, wl.gqa) == 4
    want = oracle.decode_mode_b(cpu, _drop_rows(plan, [r_off, r_vs, r_tier, r_sec]), wl.codebooks,
                                wl.q, wl.gqa, wl.rope_theta)
    err = max_err(out.float().cpu().numpy(), want)
    log(f"  malformed rows past the first page table skipped: max abs err {err:.3e}")
    assert err <= TOL and torch.isfinite(out).all()


def test_decode_malformed_rows_are_skipped_and_counted(gpu):
    # five malformed rows of different kinds: each contributes no token, the
    # checked entry reports all five, the output equals the oracle over the
    # other rows, and a clean decode on the same workspace reports zero again.
    # An empty dense page (count 0, radius offset = theta offset) is well
    # formed: no token, not counted
    wl = synth.make_decode_workload(2, ctx_override=3000)
    pool, cpu = pool_from_oracle(wl, gpu)
    plan = wl.plan
    rs = plan.row_start
    dense = [p for p in range(rs[0], rs[1]) if plan.tier[p] == fmt.DENSE_TIER_ID]
    comp = [p for p in range(rs[2], rs[3]) if plan.tier[p] == 1]
    r_off, r_vs, r_tier, r_dense, r_sec = int(rs[1]) + 3, int(rs[4]) + 1, int(rs[5]) + 2, dense[1], comp[4]
    r_empty = dense[2]
    pt = plan.ptable.copy()
    vs = plan.vslot.copy()
    pt[r_off, 0] = -16                                 # page offset outside the pool
    vs[r_vs] = plan.num_vpages + 5                     # V slot outside the V pool
    pt[r_dense, 1] += 2                                # dense K rows not 16-byte aligned
    pt[r_sec, 2] += 600                                # radius section beyond the 512-byte window
    pt[r_empty, 2] = pt[r_empty, 1]                    # empty dense page: no K rows
    pages = pool.pages.clone()
    pages[int(plan.ptable[r_tier, 0])] = 7             # unknown tier id
    pages[int(plan.ptable[r_empty, 0]) + 1] = 0        # its count byte
    bad = ops.PagedPool(**{**pool.__dict__, "ptable": torch.as_tensor(pt, device=gpu),
                           "vslot": torch.as_tensor(vs, device=gpu), "pages": pages})
    q = torch.as_tensor(wl.q, device=gpu)
    ws = torch.zeros(pool.workspace_bytes(wl.gqa), dtype=torch.uint8, device=gpu)
    out = ops.decode_paged(bad, q, wl.gqa, wl.rope_theta, workspace=ws)
    assert ops.decode_status(bad, ws, wl.gqa) == 5
    with pytest.raises(Exception, match="5 malformed"):
        ops.decode_paged(bad, q, wl.gqa, wl.rope_theta, workspace=ws, check=True)
    want = oracle.decode_mode_b(cpu, _drop_rows(plan, [r_off, r_vs, r_tier, r_dense, r_sec, r_empty]),
                                wl.codebooks, wl.q, wl.gqa, wl.rope_theta)
    err = max_err(out.float().cpu().numpy(), want)
    log(f"  malformed rows skipped: max abs err {err:.3e} against the oracle without them")
    assert err <= TOL and torch.isfinite(out).all()
    ops.decode_paged(pool, q, wl.gqa, wl.rope_theta, workspace=ws)
    assert ops.decode_status(pool, ws, wl.gqa) == 0


@pytest.mark.parametrize("config,heads", [(2, None), (5, 2)])
def test_decode_peaked_softmax_with_sink(gpu, config, heads):
    # One dense sink token (position 0) 25 log2 units above a long, quiet
    # tail, with one work item per (seq, head): at config 5 every wave then
    # walks ~680 pages whose weights sit 2^-25 below the running maximum
    # (the sink's); the tail still carries 2^17 * 2^-25 of the mass.  The
    # output must match the fp64 oracle within the north-star tolerance.
    from gpu_helpers import check_sampled_heads
    wl = synth.make_decode_workload(config, num_seqs_override=1 if config == 5 else None)
    D = fmt.DENSE_TIER_ID
    q = wl.q[0].astype(np.float64)
    for h in range(wl.num_kv):
        K = wl.K[0][h].astype(np.float32)
        K[1:] *= 0.02                                          # a quiet tail
        qs = q[h * wl.gqa:(h + 1) * wl.gqa]
        u = qs.sum(axis=0)
        u /= np.linalg.norm(u)
        gap = (qs @ u) / np.sqrt(wl.dh)                        # natural-log logit per unit of sink norm
        K[0] = (25.0 * np.log(2.0) / gap.min()) * u           # every q head >= 25 log2 units above
        wl.K[0][h] = K.astype(np.float16)
        wl.tier_of[h][0] = D
    wl.plan = fmt.plan_pages(wl.tier_of, None, 1, wl.num_kv, wl.dh, 16, rng=np.random.default_rng(7))
    log(f"peaked softmax config{config}: rows={wl.plan.num_rows}, one item per head")
    pool, _, _ = ops.build_pool_gpu(wl, gpu, rows_per_item=1 << 22)
    assert pool.num_items == wl.num_kv
    out = ops.decode_paged(pool, torch.as_tensor(wl.q, device=gpu), wl.gqa, wl.rope_theta, check=True)
    torch.cuda.synchronize()
    if heads is None:
        cpu = oracle.build_pool(wl)
        want = oracle.decode_mode_b(cpu, wl.plan, wl.codebooks, wl.q, wl.gqa, wl.rope_theta)
        err = max_err(out.float().cpu().numpy(), want)
        log(f"  all heads: max abs err {err:.3e}")
        assert err <= TOL
    else:
        check_sampled_heads(wl, pool, out, heads, seed=55, tol=TOL)


@pytest.mark.parametrize("config,ctx", [(2, 4096), (1, None)])
def test_decode_runner_equals_decode_paged(gpu, config, ctx):
    # the bound call (sphkv_decode_plan) launches the same kernels as
    # decode_paged: bit-identical output, in both of its forms, over two
    # calls with different q
    wl = synth.make_decode_workload(config, ctx_override=ctx)
    pool, cpu = pool_from_oracle(wl, gpu)
    run = ops.DecodeRunner(pool, wl.gqa, wl.rope_theta)
    fn = run.raw()
    rng = np.random.default_rng(30)
    for k in range(2):
        qh = wl.q if k == 0 else (rng.standard_normal(wl.q.shape) * 0.5).astype(np.float16)
        q = torch.as_tensor(qh, device=gpu)
        a = ops.decode_paged(pool, q, wl.gqa, wl.rope_theta)
        b = run(q)
        c = torch.empty_like(q)
        fn(q.data_ptr(), c.data_ptr())
        torch.cuda.synchronize()
        assert torch.equal(a, b) and torch.equal(a, c)
    want = oracle.decode_mode_b(cpu, wl.plan, wl.codebooks, qh, wl.gqa, wl.rope_theta)
    assert max_err(c.float().cpu().numpy(), want) <= TOL
    # regression: a runner dropped right after raw() (the closure keeps it and
    # its plan alive)
    import gc
    fn2 = ops.DecodeRunner(pool, wl.gqa, wl.rope_theta).raw()
    gc.collect()
    d = torch.empty_like(q)
    fn2(q.data_ptr(), d.data_ptr())
    torch.cuda.synchronize()
    assert torch.equal(a, d)
