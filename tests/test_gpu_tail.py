"""GPU parity of the decode-time tail (sphkv_decode_step / sphkv_decode_append):
a full reference decode step scores the page context, the flushed decode
pages, the staged tokens and the new token in one softmax, then stages the
new token and flushes full pages (spherical_kv_pipeline.py:2248-2342,
2389-2475).

Tolerance: the decode output within max-abs 2e-3 of the fp64 oracle
(oracle.decode_mode_b with oracle/tail.py's TailOracle).  Staged radii, codes,
V, positions and the flushed pages' bytes are bit-exact.
"""
import numpy as np
import pytest
import torch

import oracle
import sphkv_format as fmt
import sphkv_ops as ops
import sphkv_synth as synth
from gpu_helpers import log, max_err, pool_from_oracle
from oracle.tail import TailOracle, step_with_context

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _setup(gpu, config=2, ctx=4096, steps=40, capacity=4, seqs=None):
    kw = {"num_seqs_override": seqs} if seqs else {}
    wl = synth.make_decode_workload(config, ctx_override=ctx, **kw)
    st = synth.make_tail_steps(wl, steps)
    wl.codebooks[3] = st.cb3
    pool, cpu = pool_from_oracle(wl, gpu)
    tail = ops.DecodeTail(pool, wl.gqa, wl.rope_theta, capacity=capacity)
    orc = TailOracle(wl.num_seqs, wl.num_kv, wl.dh, st.cb3)
    return wl, st, pool, cpu, tail, orc


def _dev(x, gpu):
    return torch.as_tensor(np.ascontiguousarray(x), device=gpu)


def _check_state(wl, pool, tail, orc):
    """Staging and flushed pages on the GPU equal the oracle's, bit for bit."""
    h = tail.state_host()
    plan = wl.plan
    cap, G3, dh = tail.capacity, wl.dh // 32, wl.dh
    pages = pool.pages.cpu().numpy()
    vpool = pool.v_pool.cpu().numpy()
    pos_d = tail.positions.cpu().numpy()
    ws = tail.work_start.cpu().numpy()
    for sh in range(wl.num_seqs * wl.num_kv):
        st = orc.staged[sh]
        n = len(st)
        assert h["state"][sh, 0] == n and h["state"][sh, 1] == len(orc.pages[sh]) and h["state"][sh, 2] == 0, sh
        for i, (r, c, v, p) in enumerate(st):
            assert (h["stg_r"][sh, i].view(np.uint32) == r.view(np.uint32)).all(), (sh, i)
            assert (h["stg_code"][sh, i] == c).all(), (sh, i)
            assert (h["stg_v"][sh, i].view(np.uint16) == v.view(np.uint16)).all(), (sh, i)
            assert h["stg_pos"][sh, i] == p
        base = int(plan.row_start[sh + 1]) + sh * cap          # sh's first reserved row
        for k, (page, pos, V) in enumerate(orc.pages[sh]):
            off = tail.dec_byte0 + (sh * cap + k) * ops.tail_slot_bytes(dh)
            assert (pages[off:off + page.size] == page).all(), f"sh {sh} decode page {k}: bytes differ"
            vp = vpool[tail.dec_vpage0 + sh * cap + k].view(np.uint16).reshape(dh, 16)
            assert (vp.T == V.view(np.uint16)).all(), f"sh {sh} decode page {k}: V differs"
            assert (pos_d[base + k] == pos).all()
        # every work item of sh ends after its flushed rows
        ends = h["work"][ws[sh]:ws[sh + 1], 2]
        assert (ends == base + len(orc.pages[sh])).all(), sh
    assert G3 == orc.G


def test_append_stages_and_flushes_bit_exact(gpu):
    # 37 appends per (seq, head): two flushed pages and 5 staged tokens, with
    # checks before, across and after each flush
    wl, st, pool, cpu, tail, orc = _setup(gpu, steps=37, capacity=3)
    log(f"tail append: {wl.num_seqs * wl.num_kv} heads, capacity {tail.capacity}")
    for t in range(37):
        ops.decode_append(pool, tail, _dev(st.k[t], gpu), _dev(st.v[t], gpu), _dev(st.pos[t], gpu))
        for s in range(wl.num_seqs):
            for h in range(wl.num_kv):
                orc.append(s, h, st.k[t, s, h], st.v[t, s, h], int(st.pos[t, s]))
        if t in (0, 14, 15, 16, 31, 36):
            torch.cuda.synchronize()
            _check_state(wl, pool, tail, orc)
    assert tail.flushed == 2 and tail.staged == 5


def test_append_fp32_keys_bit_exact(gpu):
    # fp32 keys that fp16 cannot hold: the encode reads them as given
    wl, st, pool, cpu, tail, orc = _setup(gpu, config=1, ctx=512, steps=17, capacity=2)
    rng = np.random.default_rng(3)
    for t in range(17):
        k32 = (st.k[t].astype(np.float32) * (1 + 1e-3 * rng.standard_normal(st.k[t].shape))).astype(np.float32)
        ops.decode_append(pool, tail, _dev(k32, gpu), _dev(st.v[t], gpu), _dev(st.pos[t], gpu))
        for s in range(wl.num_seqs):
            for h in range(wl.num_kv):
                orc.append(s, h, k32[s, h], st.v[t, s, h], int(st.pos[t, s]))
    torch.cuda.synchronize()
    _check_state(wl, pool, tail, orc)


@pytest.mark.parametrize("config,ctx,seqs", [(2, 4096, None), (1, 4096, None), (4, 2500, 3), (5, 3000, 1)])
def test_decode_step_matches_oracle(gpu, config, ctx, seqs):
    # steps with 0, 1, 2, 14 and 15 staged tokens, across the flush and after
    # it (a decode page in the context), and after a second flush
    steps = 34
    wl, st, pool, cpu, tail, orc = _setup(gpu, config=config, ctx=ctx, steps=steps, capacity=3, seqs=seqs)
    log(f"decode step config{config} ctx={ctx} seqs={wl.num_seqs} gqa={wl.gqa} rows={wl.plan.num_rows}")
    worst = 0.0
    for t in range(steps):
        q, k, v, p = st.q[t], st.k[t], st.v[t], st.pos[t]
        out = ops.decode_step(pool, tail, _dev(q, gpu), _dev(k, gpu), _dev(v, gpu), _dev(p, gpu))
        if t in (0, 1, 2, 14, 15, 16, 17, 31, 32, 33):
            got = out.float().cpu().numpy()
            want = oracle.decode_mode_b(cpu, wl.plan, wl.codebooks, q, wl.gqa, wl.rope_theta, tail=orc,
                                        k_new=k, v_new=v, cur_pos=p)
            err = max_err(got, want)
            worst = max(worst, err)
            log(f"  step {t}: staged {len(orc.staged[0])}, decode pages {len(orc.pages[0])}, max abs err {err:.3e}")
            assert err <= TOL
        for s in range(wl.num_seqs):
            for h in range(wl.num_kv):
                orc.append(s, h, k[s, h], v[s, h], int(p[s]))
    torch.cuda.synchronize()
    _check_state(wl, pool, tail, orc)
    log(f"  worst {worst:.3e}")


@pytest.mark.parametrize("dh,gqa", [(128, 4), (64, 2), (128, 1), (64, 8)])
def test_decode_step_empty_head_and_shapes(gpu, dh, gqa):
    # Head 1 has no context pages: its one work item is empty (its partial
    # holds no token); head 0 holds one token, head 2 a mix of every tier,
    # head 3 dense tokens.  Steps cross a flush, so the decode page joins
    # head 1's empty item.
    rng = np.random.default_rng(5)
    num_kv, L, steps = 4, 40, 18
    Ls = [1, 0, 17, 33]
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
    st = synth.make_tail_steps(wl, steps)
    wl.codebooks[3] = st.cb3
    pool, cpu = pool_from_oracle(wl, gpu)
    tail = ops.DecodeTail(pool, wl.gqa, wl.rope_theta, capacity=2)
    orc = TailOracle(wl.num_seqs, wl.num_kv, wl.dh, st.cb3)
    ws, w = tail.work_start.cpu().numpy(), tail.work.cpu().numpy()
    assert ws[2] - ws[1] == 1 and w[ws[1], 1] == w[ws[1], 2], "head 1: one empty work item"
    log(f"decode step, empty head: dh={dh} gqa={gqa} items={tail.num_items}")
    for t in range(steps):
        qt, k, v, p = st.q[t], st.k[t], st.v[t], st.pos[t]
        out = ops.decode_step(pool, tail, _dev(qt, gpu), _dev(k, gpu), _dev(v, gpu), _dev(p, gpu))
        if t in (0, 1, 15, 16, 17):
            got = out.float().cpu().numpy()
            want = oracle.decode_mode_b(cpu, wl.plan, wl.codebooks, qt, wl.gqa, wl.rope_theta, tail=orc,
                                        k_new=k, v_new=v, cur_pos=p)
            err = max_err(got, want)
            log(f"  step {t}: staged {len(orc.staged[0])}, decode pages {len(orc.pages[0])}, max abs err {err:.3e}")
            assert err <= TOL
        for h in range(wl.num_kv):
            orc.append(0, h, k[0, h], v[0, h], int(p[0]))
    torch.cuda.synchronize()
    _check_state(wl, pool, tail, orc)


def test_decode_step_caller_list_without_item(gpu):
    # A caller's work list may give a (seq, head) no item at all: head 0's
    # output is then its staged tokens and new token alone (the tail kernel's
    # merge has no item partial for it), the other heads see their context as
    # well.  Unbound sphkv_decode_step, no append.
    import ctypes
    wl, st, pool, cpu, tail, orc = _setup(gpu, config=1, ctx=256, steps=6, capacity=1)
    for t in range(5):
        ops.decode_append(pool, tail, _dev(st.k[t], gpu), _dev(st.v[t], gpu), _dev(st.pos[t], gpu))
        for h in range(wl.num_kv):
            orc.append(0, h, st.k[t][0, h], st.v[t][0, h], int(st.pos[t][0]))
    torch.cuda.synchronize()
    ws, w = tail.work_start.cpu().numpy(), tail.work.cpu().numpy()
    w2 = np.ascontiguousarray(w[ws[1]:])                  # sh 0's items removed
    ws2 = np.concatenate([[0], ws[1:] - ws[1]]).astype(np.int32)
    w2d, ws2d = _dev(w2, gpu), _dev(ws2, gpu)
    n2 = int(w2.shape[0])
    lib = ops.load()
    nbytes = int(lib.sphkv_decode_paged_workspace_bytes(n2, wl.gqa, wl.dh))
    wsp = torch.zeros(nbytes, dtype=torch.uint8, device=gpu)
    q, k, v, p = st.q[5], st.k[5], st.v[5], st.pos[5]
    qd, kd, vd, pd = (_dev(x, gpu) for x in (q, k, v, p))
    out = torch.empty_like(qd)
    c1, c2, c3 = pool.cb_ptrs()
    parity = tail.counts()[2]
    rc = lib.sphkv_decode_step(
        pool.pages.data_ptr(), tail.pages_bytes, tail.ptable.data_ptr(), tail.vslot.data_ptr(),
        tail.positions.data_ptr(), tail.num_rows, pool.v_pool.data_ptr(), tail.num_vpages, c1, c2, c3,
        w2d.data_ptr(), n2, ws2d.data_ptr(), wl.num_seqs, wl.num_kv, wl.gqa, qd.data_ptr(), kd.data_ptr(), 0,
        vd.data_ptr(), pd.data_ptr(), tail.stg_r.data_ptr(), tail.stg_code.data_ptr(), tail.stg_v.data_ptr(),
        tail.stg_pos.data_ptr(), tail.state.data_ptr(), tail.dec_byte0, tail.dec_vpage0, tail.capacity, 0, parity,
        out.data_ptr(), wsp.data_ptr(), nbytes, wl.dh, 16, ctypes.c_float(tail.sm_scale), wl.rope_theta,
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    ops.check(rc, "sphkv_decode_step")
    got = out.float().cpu().numpy()
    ctx_out, ctx_lse = oracle.decode_mode_b(cpu, wl.plan, wl.codebooks, q, wl.gqa, wl.rope_theta, return_lse=True)
    ctx_lse[:, :wl.gqa] = -np.inf                         # head 0: no context
    want = step_with_context(ctx_out, ctx_lse, orc, q, wl.gqa, wl.rope_theta, k, v, p)
    err = max_err(got, want)
    log(f"caller list without sh 0's item: max abs err {err:.3e}")
    assert err <= TOL


def test_decode_step_full_config2(gpu):
    # BASELINE config 2 at full size (32,768 tokens): tails of 0, 1 and 15
    # tokens and the step after the flush; the page context is evaluated once
    # by the oracle (same q every step) and merged with each tail
    steps = 17
    wl, st, pool, cpu, tail, orc = _setup(gpu, config=2, ctx=None, steps=steps, capacity=2)
    q = wl.q
    ctx_out, ctx_lse = oracle.decode_mode_b(cpu, wl.plan, wl.codebooks, q, wl.gqa, wl.rope_theta, return_lse=True)
    qd = _dev(q, gpu)
    for t in range(steps):
        k, v, p = st.k[t], st.v[t], st.pos[t]
        out = ops.decode_step(pool, tail, qd, _dev(k, gpu), _dev(v, gpu), _dev(p, gpu))
        if t in (0, 1, 15, 16):
            got = out.float().cpu().numpy()
            want = step_with_context(ctx_out, ctx_lse, orc, q, wl.gqa, wl.rope_theta, k, v, p)
            err = max_err(got, want)
            log(f"  config2 full, step {t}: staged {len(orc.staged[0])}, pages {len(orc.pages[0])}, err {err:.3e}")
            assert err <= TOL
        for h in range(wl.num_kv):
            orc.append(0, h, k[0, h], v[0, h], int(p[0]))
    torch.cuda.synchronize()
    _check_state(wl, pool, tail, orc)


def test_decode_step_without_append_leaves_state(gpu):
    wl, st, pool, cpu, tail, orc = _setup(gpu, config=2, ctx=2000, steps=8, capacity=2)
    for t in range(5):
        ops.decode_append(pool, tail, _dev(st.k[t], gpu), _dev(st.v[t], gpu), _dev(st.pos[t], gpu))
    before = tail.state_host()
    args = [_dev(x, gpu) for x in (st.q[5], st.k[5], st.v[5], st.pos[5])]
    a = ops.decode_step(pool, tail, *args, append=False).cpu().numpy()
    b = ops.decode_step(pool, tail, *args, append=False).cpu().numpy()
    after = tail.state_host()
    assert (a.view(np.uint16) == b.view(np.uint16)).all()
    for key in before:
        assert (before[key] == after[key]).all(), key
    assert tail.staged == 5


def test_decode_step_capacity_is_enforced(gpu):
    # capacity 0: the 16th token would need a decode page; the host refuses
    wl, st, pool, cpu, tail, orc = _setup(gpu, config=1, ctx=256, steps=16, capacity=0)
    for t in range(15):
        ops.decode_append(pool, tail, _dev(st.k[t], gpu), _dev(st.v[t], gpu), _dev(st.pos[t], gpu))
    with pytest.raises(ValueError, match="no decode-page slot"):
        ops.decode_append(pool, tail, _dev(st.k[15], gpu), _dev(st.v[15], gpu), _dev(st.pos[15], gpu))
    torch.cuda.synchronize()
    assert int(tail.state_host()["state"][:, 0].min()) == 15


def test_second_tail_on_a_pool_is_refused(gpu):
    # two tails would share one decode-page region (or reallocate the pool
    # under the first tail's bound plan)
    wl, st, pool, cpu, tail, orc = _setup(gpu, config=1, ctx=256, steps=1, capacity=1)
    with pytest.raises(ValueError, match="already has a DecodeTail"):
        ops.DecodeTail(pool, wl.gqa, wl.rope_theta, capacity=1)
