"""GPU parity of the Mode-A (LayerPool) path through the reference-named
Python entry points (fused_decode.sphkv_decode / sphkv_encode_append,
new_fused_decode.sphkv_logits / build_q_lut) and the C ABI behind them.

Bars: encode_append bit-exact with the oracle's restatement of
decode_kernel.cu:10-84 (codes, radius codes, radius scales, fp16 V) over a
sequence of appends that opens pages and rescales earlier radius codes;
decode output within max-abs 2e-3 of the fp64 oracle, per-page (m, l) within
1e-4 abs / 1e-4 relative; LUT and logits within 1e-4 (fp32 sums of at most
G_max terms), -inf exactly where the oracle has it.
"""
import numpy as np
import pytest
import torch

import fused_decode
import new_fused_decode
import oracle
import sphkv_synth as synth
from gpu_helpers import log, max_err

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("page_size,G,g,C,dup", [(16, 8, 16, 64, False), (128, 8, 16, 64, False),
                                                  (16, 4, 32, 100, True)])
def test_encode_append_bitexact_over_a_sequence(gpu, page_size, G, g, C, dup):
    # g 16: centroid rows as 16-byte loads; g 32 with C 100: one element at a
    # time, two codes per lane in the argmax, and (dup) every row c equal to
    # row c + 50, so every argmax is a tie that the first maximum settles
    rng = np.random.default_rng(21 + page_size + C)
    num_kv, dh, G_max = 8, 128, 8
    x = rng.standard_normal((num_kv, G, C, g))
    if dup:
        x[:, :, C // 2:] = x[:, :, :C // 2]
    cb = (x / np.linalg.norm(x, axis=-1, keepdims=True)).astype(np.float32)
    n_pages = 3 * num_kv
    th = np.zeros((n_pages, page_size, G_max), np.uint8)
    rd = np.zeros_like(th)
    rs = np.zeros((n_pages, G_max), np.float32)
    vp = np.zeros((n_pages, page_size, dh), np.float16)
    d_th, d_rd, d_rs, d_vp, d_cb = _t(th, gpu), _t(rd, gpu), _t(rs, gpu), _t(vp, gpu), _t(cb, gpu)
    steps = page_size + 5                               # opens a second page per head
    scale = np.exp(rng.normal(0, 0.7, size=(steps, num_kv, dh)))
    for step in range(steps):
        slot = step % page_size
        pg = step // page_size
        pids = np.arange(num_kv, dtype=np.int64) + pg * num_kv
        k = (rng.standard_normal((num_kv, dh)) * scale[step]).astype(np.float32)
        v = rng.standard_normal((num_kv, dh)).astype(np.float32)
        oracle.encode_append(k, v, cb, th, rd, rs, vp, pids, slot, slot == 0)
        fused_decode.sphkv_encode_append(_t(k, gpu), _t(v, gpu), d_cb, d_th, d_rd, d_rs, d_vp, _t(pids, gpu),
                                         slot, G, g, C, G_max, dh, page_size, slot == 0)
    torch.cuda.synchronize()
    log(f"append page_size={page_size} steps={steps}")
    assert (d_th.cpu().numpy() == th).all()
    assert (d_rd.cpu().numpy() == rd).all()
    assert (d_rs.cpu().numpy().view(np.uint32) == rs.view(np.uint32)).all()
    assert (d_vp.cpu().numpy().view(np.uint16) == vp.view(np.uint16)).all()
    if dup:
        assert th.max() < C // 2                        # the ties went to the first maximum


CASES = [
    dict(dh=128, kv_groups=4, page_size=16, ctx=2000, tiers=(1, 2), holes=0.0),
    dict(dh=128, kv_groups=4, page_size=128, ctx=3001, tiers=(1, 2, 3), holes=0.1),
    dict(dh=64, kv_groups=8, page_size=32, ctx=777, tiers=(1, 3), holes=0.05),
    dict(dh=128, kv_groups=1, page_size=16, ctx=17, tiers=(2,), holes=0.0),
    dict(dh=64, kv_groups=2, page_size=64, ctx=5000, tiers=(1, 2), holes=0.3),
    # G_max outside {4, 8}: the general kernel
    dict(dh=64, kv_groups=4, page_size=16, ctx=1500, tiers=(1, 3), holes=0.1, G_pad=6),
    dict(dh=128, kv_groups=8, page_size=48, ctx=2000, tiers=(1, 2, 3), holes=0.0, G_pad=12),
]


def _modea_call(w, gpu):
    dev = {k: _t(w[k], gpu) for k in ("q", "cb_flat", "tier_G", "tier_g", "theta", "radius", "r_scales",
                                       "v_pool", "block_table", "bits_table", "ctx_lens")}
    nq = w["q"].shape[0]
    out = torch.empty((nq, w["dh"]), dtype=torch.float32, device=gpu)
    part = torch.zeros((nq, w["max_blocks"], w["dh"] + 2), dtype=torch.float32, device=gpu)
    r = fused_decode.sphkv_decode(dev["q"], dev["cb_flat"], dev["tier_G"], dev["tier_g"], dev["theta"],
                                  dev["radius"], dev["r_scales"], dev["v_pool"], dev["block_table"],
                                  dev["bits_table"], dev["ctx_lens"], out, part, nq, w["num_kv"], w["kv_groups"],
                                  w["num_tiers"], w["max_blocks"], w["page_size"], w["dh"], w["G_max"],
                                  w["cb_max"], w["g_max"], w["sm_scale"], w["max_ctx"])
    assert r is out
    torch.cuda.synchronize()
    return out.cpu().numpy(), part.cpu().numpy(), dev


@pytest.mark.parametrize("case", CASES, ids=[f"dh{c['dh']}-g{c['kv_groups']}-p{c['page_size']}-G{c.get('G_pad', 0)}" for c in CASES])
def test_decode_modea_matches_oracle(gpu, case):
    w = synth.make_modea_workload(seed=31, num_kv=4, **case)
    log(f"modea {case} max_blocks={w['max_blocks']}")
    got, part, _ = _modea_call(w, gpu)
    want, M, L = oracle.decode_mode_a(w["q"], w["cb_flat"], w["tier_G"], w["tier_g"], w["theta"], w["radius"],
                                      w["r_scales"], w["v_pool"], w["block_table"], w["bits_table"],
                                      w["kv_groups"], w["sm_scale"])
    err = max_err(got, want)
    log(f"  out max abs err {err:.3e}")
    assert err <= TOL
    gm, gl = part[:, :, 0], part[:, :, 1]
    absent = np.isinf(M)
    assert (np.isinf(gm) == absent).all() and (gl[absent] == 0).all()
    np.testing.assert_allclose(gm[~absent], M[~absent], atol=1e-4, rtol=1e-4)
    np.testing.assert_allclose(gl[~absent], L[~absent], rtol=1e-4)


@pytest.mark.parametrize("G_pad", [0, 12])
def test_lut_and_logits_match_oracle(gpu, G_pad):
    # G_max 8: the grouped kernel (one thread per kv head and token); G_max
    # 12: the general one
    w = synth.make_modea_workload(seed=41, num_kv=4, kv_groups=4, dh=128, page_size=16, ctx=1000,
                                  tiers=(1, 2, 3), fracs=(1, 1, 1), holes=0.1, G_pad=G_pad)
    dev = {k: _t(w[k], gpu) for k in ("q", "cb_flat", "tier_G", "tier_g", "theta", "radius", "r_scales",
                                       "block_table", "bits_table")}
    lut = new_fused_decode.build_q_lut(dev["q"], dev["cb_flat"], dev["tier_G"], dev["tier_g"], w["num_kv"],
                                       w["kv_groups"], w["num_tiers"], w["G_max"], w["cb_max"], w["g_max"])
    want_lut = oracle.q_lut(w["q"], w["cb_flat"], w["tier_G"], w["tier_g"], w["kv_groups"])
    assert max_err(lut.cpu().numpy(), want_lut) <= 1e-4
    ctx = np.array([1000, 999, 600, 1], np.int32)
    max_ctx = 1024
    nq = w["q"].shape[0]
    logits = torch.empty((nq, max_ctx), dtype=torch.float32, device=gpu)
    r = new_fused_decode.sphkv_logits(lut, dev["theta"], dev["radius"], dev["r_scales"], dev["block_table"],
                                      dev["bits_table"], _t(ctx, gpu), logits, nq, w["num_kv"], w["kv_groups"],
                                      w["num_tiers"], w["max_blocks"], w["page_size"], w["G_max"], w["cb_max"],
                                      w["sm_scale"], max_ctx)
    assert r is logits
    got = logits.cpu().numpy()
    want = oracle.lut_logits(want_lut, w["theta"], w["radius"], w["r_scales"], w["block_table"],
                             w["bits_table"], ctx, w["kv_groups"], w["sm_scale"], max_ctx)
    inf = np.isinf(want)
    assert (np.isinf(got) == inf).all()
    err = max_err(got[~inf], want[~inf])
    log(f"lut logits max abs err {err:.3e}")
    assert err <= 1e-4


def test_q_lut_row_load_forms_agree(gpu):
    # 16-dim groups read as 16-byte loads when q and the centroid rows are
    # 16-byte aligned, else one float at a time: same fma order, same bits
    w = synth.make_modea_workload(seed=43, num_kv=2, kv_groups=4, dh=128, page_size=16, ctx=300,
                                  tiers=(1, 2, 3), fracs=(1, 1, 1))
    q = _t(w["q"], gpu)
    qbuf = torch.empty(q.numel() + 1, dtype=torch.float32, device=gpu)
    q_odd = qbuf[1:].view(q.shape)                    # data 4 bytes past a 16-byte boundary
    q_odd.copy_(q)
    assert q_odd.data_ptr() % 16 == 4
    args = (_t(w["cb_flat"], gpu), _t(w["tier_G"], gpu), _t(w["tier_g"], gpu), w["num_kv"], w["kv_groups"],
            w["num_tiers"], w["G_max"], w["cb_max"], w["g_max"])
    a = new_fused_decode.build_q_lut(q, *args)
    b = new_fused_decode.build_q_lut(q_odd, *args)
    assert torch.equal(a, b)
    want = oracle.q_lut(w["q"], w["cb_flat"], w["tier_G"], w["tier_g"], w["kv_groups"])
    assert max_err(a.cpu().numpy(), want) <= 1e-4


def test_modea_single_range_and_empty_tables(gpu):
    """max_blocks 1 (one range writes out directly) and a head whose pages are all absent."""
    w = synth.make_modea_workload(seed=5, num_kv=2, kv_groups=4, dh=128, page_size=16, ctx=9, tiers=(1,), fracs=(1,))
    w["block_table"] = w["block_table"].copy()
    w["block_table"][1, :] = -1
    got, part, _ = _modea_call(w, gpu)
    want, M, L = oracle.decode_mode_a(w["q"], w["cb_flat"], w["tier_G"], w["tier_g"], w["theta"], w["radius"],
                                      w["r_scales"], w["v_pool"], w["block_table"], w["bits_table"], 4, w["sm_scale"])
    assert max_err(got, want) <= TOL
    assert (got[4:] == 0).all()                       # acc 0 / (0 + 1e-8)


def test_omega_ema_after_decode_matches_oracle(gpu):
    """The decode's partial_scratch (m, l) views feed the omega update in place
    (spherical_kv_pipeline.py:1690-1701), with absent pages and a head whose
    pages are all absent."""
    import omega_ema
    w = synth.make_modea_workload(seed=17, num_kv=4, kv_groups=4, dh=128, page_size=16, ctx=3000,
                                  tiers=(1, 2), holes=0.2)
    w["block_table"] = w["block_table"].copy()
    w["block_table"][3, :] = -1
    _, part, _ = _modea_call(w, gpu)
    rng = np.random.default_rng(2)
    prev = rng.random((w["num_kv"], w["max_blocks"])).astype(np.float32)
    scratch = torch.from_numpy(part).to(gpu)
    ml = scratch[:, :, :2]
    for beta in (0.9, 0.0):
        got = omega_ema.omega_ema(ml[..., 0], ml[..., 1], _t(prev, gpu), w["num_kv"], 4, w["max_blocks"], beta)
        want = oracle.omega_ema(part[:, :, 0], part[:, :, 1], prev, w["num_kv"], 4, beta)
        err = np.abs(got.cpu().numpy() - want).max()
        log(f"omega beta={beta} max abs err {err:.3e}")
        np.testing.assert_allclose(got.cpu().numpy(), want, rtol=1e-5, atol=1e-7)
    # in place, and a pool-like object through update_omega_gpu
    om = _t(prev, gpu)
    omega_ema.omega_ema(ml[..., 0], ml[..., 1], om, w["num_kv"], 4, w["max_blocks"], 0.9, out=om)
    np.testing.assert_allclose(om.cpu().numpy(), oracle.omega_ema(part[:, :, 0], part[:, :, 1], prev, 4, 4, 0.9),
                               rtol=1e-5, atol=1e-7)
    pool = type("P", (), dict(num_kv=w["num_kv"], kv_groups=4, max_blocks=w["max_blocks"], device=gpu,
                              _partial_scratch=scratch))()
    d = {}
    first = omega_ema.update_omega_gpu(d, 0, pool)
    want1 = oracle.omega_ema(part[:, :, 0], part[:, :, 1], np.ones_like(prev), 4, 4, 0.9)
    np.testing.assert_allclose(first.cpu().numpy(), want1, rtol=1e-5, atol=1e-7)
    assert (first.cpu().numpy()[3] == np.float32(0.9)).all()   # head without pages: mass 0


@pytest.mark.parametrize("num_kv,kv_groups,max_blocks,adjacent", [
    (3, 4, 300, False), (2, 8, 3000, True), (2, 12, 100, True), (1, 2, 5000, True), (2, 1, 2048, False),
    (2, 6, 1500, False), (3, 3, 4096, True)])
def test_omega_ema_kernel_forms(gpu, num_kv, kv_groups, max_blocks, adjacent):
    # the single-pass kernel (kv_groups <= 4 or <= 8, max_blocks <= 4096; (m, l) read
    # as one 8-byte word when l follows m, else separately) and the general one
    import omega_ema
    rng = np.random.default_rng(num_kv * 1000 + kv_groups * 10 + max_blocks)
    nq = num_kv * kv_groups
    m = (rng.standard_normal((nq, max_blocks)) * 4).astype(np.float32)
    l = np.where(rng.random((nq, max_blocks)) < 0.8, rng.random((nq, max_blocks)) * 3, 0.0).astype(np.float32)
    m[0, :] += 100.0                                  # exp arguments clamp at -60 for the others
    prev = rng.random((num_kv, max_blocks)).astype(np.float32)
    if adjacent:
        ml = torch.from_numpy(np.stack([m, l], axis=-1)).to(gpu)
        mt, lt = ml[..., 0], ml[..., 1]
    else:
        mt, lt = _t(m, gpu), _t(l, gpu)
    got = omega_ema.omega_ema(mt, lt, _t(prev, gpu), num_kv, kv_groups, max_blocks, 0.9).cpu().numpy()
    want = oracle.omega_ema(m, l, prev, num_kv, kv_groups, 0.9)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-7)
