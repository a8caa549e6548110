"""CPU pins of the Mode-A oracle (no GPU).

The reference's Mode-A kernels (decode_kernel.cu:10-289) cannot run here (CUDA
only) and ship no fixtures, so the restatements are pinned by what the
mathematics fixes:
  * encode_append: a key that is a scaled codebook row encodes to that row and
    its norm; the running-max radius scale follows hand-computed closed forms
    (new page, a smaller norm, a larger norm that rescales earlier codes);
    argmax agrees with an fp64 brute force wherever the top-2 margin is clear.
  * decode_mode_a: equals textbook attention softmax(q K_hat^T * sm_scale) V
    over keys rebuilt as r_hat * centroid (a formulation that never forms the
    LUT); a page holding one token returns that token's V row and (m, l) =
    (its logit, 1); unwritten slots (zero radius) carry no weight.
  * lut_logits: equals q . K_hat over the rebuilt keys; -inf past ctx_lens.
"""
import numpy as np
import pytest

import oracle
import sphkv_synth as synth


def _fresh_pools(n_pages=2, page_size=16, G_max=8, dh=128):
    return (np.zeros((n_pages, page_size, G_max), np.uint8), np.zeros((n_pages, page_size, G_max), np.uint8),
            np.zeros((n_pages, G_max), np.float32), np.zeros((n_pages, page_size, dh), np.float16))


def _codebook(rng, num_kv=1, G=8, C=64, g=16):
    x = rng.standard_normal((num_kv, G, C, g))
    return (x / np.linalg.norm(x, axis=-1, keepdims=True)).astype(np.float32)


def test_append_scaled_centroid_encodes_to_itself():
    rng = np.random.default_rng(0)
    cb = _codebook(rng)
    codes = rng.integers(0, 64, size=8)
    norms = np.exp(rng.normal(0, 0.5, size=8)).astype(np.float32)
    k = np.concatenate([norms[gi] * cb[0, gi, codes[gi]] for gi in range(8)])[None, :].astype(np.float32)
    v = rng.standard_normal((1, 128)).astype(np.float32)
    th, rd, rs, vp = _fresh_pools()
    oracle.encode_append(k, v, cb, th, rd, rs, vp, np.array([1]), 0, True)
    assert (th[1, 0] == codes).all()
    np.testing.assert_allclose(rs[1], norms, rtol=1e-5)
    assert (rd[1, 0] == 255).all()                      # norm / (norm + 1e-8) * 255 rounds to 255
    assert (vp[1, 0] == v[0].astype(np.float16)).all()
    assert not th[0].any() and not rd[0].any()         # other pages untouched


def test_append_running_max_scale_closed_forms():
    """slot 0 (new page) norm a, slot 1 norm b < a, slot 2 norm c > a:
    codes 255, round(255 b / a), then the earlier codes scale by a / c."""
    rng = np.random.default_rng(1)
    cb = _codebook(rng, G=1, C=16, g=16)
    d = cb[0, 0, 3]
    a, b, c = 2.0, 0.75, 4.0
    th, rd, rs, vp = _fresh_pools(n_pages=1, G_max=1, dh=16)
    z = np.zeros((1, 16), np.float32)
    oracle.encode_append((a * d)[None, :].astype(np.float32), z, cb, th, rd, rs, vp, np.array([0]), 0, True)
    oracle.encode_append((b * d)[None, :].astype(np.float32), z, cb, th, rd, rs, vp, np.array([0]), 1, False)
    assert rd[0, 0, 0] == 255 and rd[0, 1, 0] == round(255 * b / a)      # 95.625 -> 96
    assert abs(rs[0, 0] - a) < 1e-5
    oracle.encode_append((c * d)[None, :].astype(np.float32), z, cb, th, rd, rs, vp, np.array([0]), 2, False)
    assert abs(rs[0, 0] - c) < 1e-5
    assert rd[0, 0, 0] == round(255 * a / c)            # 127.5 in fp32 rounds half away -> 128
    assert rd[0, 1, 0] == round(96 * a / c)             # 48
    assert rd[0, 2, 0] == 255
    assert (th[0, :3, 0] == 3).all()


def test_append_argmax_matches_fp64_brute_force():
    rng = np.random.default_rng(2)
    G, C, g = 8, 64, 16
    cb = _codebook(rng, num_kv=3, G=G, C=C, g=g)
    checked = 0
    for trial in range(20):
        k = (rng.standard_normal((3, G * g)) * np.exp(rng.normal(0, 1, size=(3, G * g)))).astype(np.float32)
        v = np.zeros((3, G * g), np.float32)
        th, rd, rs, vp = _fresh_pools(n_pages=3, G_max=G, dh=G * g)
        oracle.encode_append(k, v, cb, th, rd, rs, vp, np.array([0, 1, 2]), 5, True)
        for h in range(3):
            for gi in range(G):
                kg = k[h, gi * g:(gi + 1) * g].astype(np.float64)
                sims = cb[h, gi].astype(np.float64) @ (kg / np.linalg.norm(kg))
                top = np.sort(sims)[-2:]
                if top[1] - top[0] > 1e-5:
                    assert th[h, 5, gi] == int(np.argmax(sims))
                    checked += 1
    assert checked > 400


def _rebuilt_keys(w, hkv, p):
    """r_hat * centroid per token of logical page p of kv head hkv, [page_size, dh] fp64."""
    phys, t = int(w["block_table"][hkv, p]), int(w["bits_table"][hkv, p])
    G, g = int(w["tier_G"][t]), int(w["tier_g"][t])
    K = np.zeros((w["page_size"], w["dh"]))
    for s in range(w["page_size"]):
        for gi in range(G):
            rh = float(w["r_scales"][phys, gi]) * float(w["radius"][phys, s, gi]) / 255.0
            K[s, gi * g:(gi + 1) * g] = rh * w["cb_flat"][hkv, t, gi, int(w["theta"][phys, s, gi]), :g].astype(np.float64)
    return K


@pytest.mark.parametrize("tiers,page_size,kv_groups", [((1, 2), 16, 4), ((1, 2, 3), 32, 2), ((3,), 16, 8)])
def test_decode_mode_a_equals_textbook_attention(tiers, page_size, kv_groups):
    w = synth.make_modea_workload(seed=7, num_kv=2, kv_groups=kv_groups, dh=64, page_size=page_size, ctx=90,
                                  tiers=tiers, fracs=[1.0] * len(tiers), holes=0.15)
    out, M, L = oracle.decode_mode_a(w["q"], w["cb_flat"], w["tier_G"], w["tier_g"], w["theta"], w["radius"],
                                     w["r_scales"], w["v_pool"], w["block_table"], w["bits_table"], kv_groups,
                                     w["sm_scale"])
    for hq in range(w["q"].shape[0]):
        hkv = hq // kv_groups
        Ks, Vs = [], []
        for p in range(w["max_blocks"]):
            if w["block_table"][hkv, p] < 0:
                assert M[hq, p] == -np.inf and L[hq, p] == 0
                continue
            K = _rebuilt_keys(w, hkv, p)
            live = np.abs(K).sum(1) > 0                  # unwritten slots have zero radius
            Ks.append(K[live])
            Vs.append(w["v_pool"][w["block_table"][hkv, p]][live].astype(np.float64))
            s = K[live] @ w["q"][hq].astype(np.float64) * w["sm_scale"]
            assert abs(M[hq, p] - s.max()) < 1e-9
            assert abs(L[hq, p] - np.exp(s - s.max()).sum()) < 1e-9
        K, V = np.concatenate(Ks), np.concatenate(Vs)
        s = K @ w["q"][hq].astype(np.float64) * w["sm_scale"]
        pr = np.exp(s - s.max())
        np.testing.assert_allclose(out[hq], pr @ V / pr.sum(), atol=1e-7)


def test_decode_mode_a_single_token_page():
    w = synth.make_modea_workload(seed=3, num_kv=1, kv_groups=1, dh=64, page_size=16, ctx=1, tiers=(1,), fracs=(1,))
    out, M, L = oracle.decode_mode_a(w["q"], w["cb_flat"], w["tier_G"], w["tier_g"], w["theta"], w["radius"],
                                     w["r_scales"], w["v_pool"], w["block_table"], w["bits_table"], 1, w["sm_scale"])
    ph = w["block_table"][0, 0]
    np.testing.assert_allclose(out[0], w["v_pool"][ph, 0].astype(np.float64), atol=1e-6)
    assert abs(L[0, 0] - 1.0) < 1e-12


def test_lut_logits_equal_rebuilt_key_dot_products():
    w = synth.make_modea_workload(seed=5, num_kv=2, kv_groups=2, dh=64, page_size=16, ctx=40, tiers=(1, 2, 3),
                                  fracs=(1, 1, 1), holes=0.2)
    lut = oracle.q_lut(w["q"], w["cb_flat"], w["tier_G"], w["tier_g"], 2)
    ctx = np.array([40, 23], np.int32)
    lg = oracle.lut_logits(lut, w["theta"], w["radius"], w["r_scales"], w["block_table"], w["bits_table"], ctx, 2,
                           w["sm_scale"], 48)
    for hq in range(4):
        hkv = hq // 2
        assert np.isinf(lg[hq, ctx[hkv]:]).all()
        for p in range(w["max_blocks"]):
            n0 = p * 16
            if n0 >= ctx[hkv]:
                break
            n1 = min(n0 + 16, ctx[hkv])
            if w["block_table"][hkv, p] < 0:
                assert np.isinf(lg[hq, n0:n1]).all()
                continue
            K = _rebuilt_keys(w, hkv, p)
            want = K @ w["q"][hq].astype(np.float64) * w["sm_scale"]
            np.testing.assert_allclose(lg[hq, n0:n1], want[:n1 - n0], atol=1e-9)


def test_layer_pool_page_closed_forms():
    r = np.array([[2.0, 0.0, 1.0], [1.0, 0.0, 3.0], [0.5, 0.0, 3.0]], np.float32)
    th, rad, rs = oracle.layer_pool_page(r, np.array([[1, 2, 300], [4, 5, 6], [7, 8, 9]]))
    np.testing.assert_array_equal(rs, np.array([2.0, 1e-8, 3.0], np.float32))
    assert rad[0, 0] == 255 and rad[1, 0] == 128 and rad[2, 0] == 64   # 127.5 -> 128 (even), 63.75 -> 64
    assert (rad[:, 1] == 0).all()                                       # all-zero group
    assert rad[1, 2] == 255 and rad[2, 2] == 255 and rad[0, 2] == 85
    assert th[0, 2] == 300 & 0xFF                                       # .to(torch.uint8) keeps the low byte


def test_layer_pool_page_rounding_bound_and_monotone():
    rng = np.random.default_rng(4)
    r = np.abs(rng.standard_normal((128, 8))).astype(np.float32)
    _, rad, rs = oracle.layer_pool_page(r, np.zeros((128, 8), np.int32))
    exact = r.astype(np.float64) / rs.astype(np.float64) * 255.0
    assert np.abs(rad - exact).max() <= 0.5 + 1e-4
    for g in range(8):
        o = np.argsort(r[:, g], kind="stable")
        assert (np.diff(rad[o, g].astype(int)) >= 0).all()
