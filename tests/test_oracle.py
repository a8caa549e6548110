"""CPU tests that pin the oracle (no GPU).

Each pin is chosen so that a plausible mistake in the oracle (dropped term,
wrong sign or index, transposed operand, wrong rounding) fails one of them:
hand-written known answers, committed torch fixtures, brute force in fp64, and
closed forms that take an independent route (complex-number RoPE, textbook
attention).
"""
import math
import os

import numpy as np
import pytest

import oracle
import sphkv_format as fmt
import sphkv_synth as synth

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ---------------------------------------------------------------- pack_bits --
def test_pack_bits_known_answers():
    # bitpacking.py:5-29, LSB-first: value i bit j -> global bit i*b + j
    assert oracle.pack_bits(np.array([1, 2, 3]), 6).tolist() == [0x81, 0x30, 0x00]
    assert oracle.pack_bits(np.array([0xF, 0x1]), 4).tolist() == [0x1F]
    assert oracle.pack_bits(np.array([7, 0, 5]), 3).tolist() == [0x47, 0x01]
    # only the low b bits of a value are stored
    assert oracle.pack_bits(np.array([0x41]), 6).tolist() == [0x01]
    assert oracle.pack_bits(np.array([], np.int32), 6).tolist() == []


@pytest.mark.parametrize("bits", [3, 4, 6])
def test_pack_bits_round_trip(bits):
    rng = np.random.default_rng(bits)
    for n in (1, 2, 5, 16, 127, 128):
        v = rng.integers(0, 2 ** bits, size=n).astype(np.int32)
        buf = oracle.pack_bits(v, bits)
        assert buf.size == (n * bits + 7) // 8
        assert (oracle.unpack_bits(buf, n, bits) == v).all()


def test_pack_bits_single_bit_positions():
    # a single set bit in value i lands exactly at global bit i*b + j
    for bits in (3, 4, 6):
        for i in range(5):
            for j in range(bits):
                v = np.zeros(5, np.int32)
                v[i] = 1 << j
                buf = oracle.pack_bits(v, bits)
                gb = i * bits + j
                want = np.zeros_like(buf)
                want[gb >> 3] = 1 << (gb & 7)
                assert (buf == want).all()


# ------------------------------------------------------------ page / header --
def test_page_header_and_sections():
    r = np.array([[1.0, 0.0], [2.0, 0.0], [0.5, 0.0]], np.float32)     # N=3, G=2
    codes = np.array([[5, 1], [63, 0], [0, 2]], np.int32)
    page = oracle.build_page(r, codes, tier_id=1, b_theta=6)
    assert page.size == 8 + 4 * 2 + (3 * 2 * 6 + 7) // 8 + 3 * 2
    assert page[0] == 1 and page[1] == 3 and (page[2:8] == 0).all()
    scales = np.frombuffer(page[8:16].tobytes(), "<f4")
    assert scales.tolist() == [2.0, 0.0]                     # max |r| per group, unclamped
    th = page[16:16 + 5]
    assert (oracle.unpack_bits(th, 6, 6) == codes.reshape(-1)).all()
    rc = page[21:].view(np.int8).reshape(3, 2)
    # group 0: r/2*127 = 63.5 -> 64 (half to even), 127, 31.75 -> 32; group 1: scale 0 -> 1e-8 -> 0
    assert rc[:, 0].tolist() == [64, 127, 32]
    assert rc[:, 1].tolist() == [0, 0, 0]


def test_page_sizes_match_the_pagebuilder_layout():
    # header 8 B + G fp32 scales + ceil(16 G b / 8) code bytes + 16 G int8 radii
    # (pagebuilder.py:8-33): tier 1 at dh 128 is 8 + 32 + 96 + 128 = 264
    assert fmt.page_nbytes(1, 16, 128) == 264
    assert fmt.page_nbytes(2, 16, 128) == 232
    assert fmt.page_nbytes(3, 16, 128) == 112
    assert fmt.page_nbytes(1, 16, 64) == 136
    assert fmt.page_nbytes(fmt.DENSE_TIER_ID, 16, 128) == 8 + 4096
    assert fmt.ptable_row(100, 1, 16, 128) == (100, 140, 236)


def test_radius_round_half_even_against_torch_rounding():
    # r/scale*127 landing on .5 exactly: scale 2, r = 1 -> 63.5 -> 64; r = 3/127*... use powers of two
    r = np.array([[2.0], [1.0], [0.0]], np.float32)
    scale, rc = oracle.radius_codes(r)
    assert scale.tolist() == [2.0]
    assert rc[:, 0].tolist() == [127, 64, 0]


# ------------------------------------------------------------ encode codes --
def _golden_cases():
    z = np.load(os.path.join(GOLD, "encode_golden.npz"))
    names = sorted({k.split("__")[0] for k in z.files if "__" in k})
    return z, names


def test_encode_matches_torch_fixtures_bit_exact():
    z, names = _golden_cases()
    assert len(names) >= 20
    for n in names:
        N, tid, g, b, dh = (int(x) for x in z[n + "__meta"])
        r, c = oracle.encode_groups(z[n + "__K"].astype(np.float32), z[n + "__cb"])
        assert (r.view(np.uint32) == z[n + "__r"].view(np.uint32)).all(), n
        assert (c == z[n + "__codes"]).all(), n
        page = oracle.build_page(r, c, tid, b)
        assert (page == z[n + "__page"]).all(), n


def test_encode_single_token_near_ties_pin_the_m1_order():
    # Single-token tier-1 pages on near-ties (fp64 top-2 margins ~1e-7): the
    # oracle's N = 1 order (MKL's M = 1 kernel) reproduces torch on every one
    # of them, while the fmaf chain of the N >= 2 path -- the same token
    # encoded as the first row of a two-token call -- picks a different code
    # on some, so these fixtures pin the order and not just the argmax.
    z, names = _golden_cases()
    ties = [n for n in names if n.startswith("t1_n1_tie")]
    assert len(ties) >= 48
    chain_diff = 0
    for n in ties:
        K = z[n + "__K"].astype(np.float32)
        assert K.shape[0] == 1
        _, c1 = oracle.encode_groups(K, z[n + "__cb"])
        assert (c1 == z[n + "__codes"]).all(), n
        _, c2 = oracle.encode_groups(np.vstack([K, np.zeros_like(K)]), z[n + "__cb"])
        chain_diff += int((c2[0] != z[n + "__codes"][0]).sum())
    assert chain_diff >= 1


def test_encode_argmax_brute_force_fp64():
    # Independent of summation order: where the fp64 top-2 margin is clear,
    # the oracle's code is the fp64 argmax; the radius is the fp64 norm.
    rng = np.random.default_rng(7)
    for (G, C, g) in ((8, 64, 16), (8, 16, 16), (4, 8, 32)):
        cb = rng.standard_normal((G, C, g))
        cb = (cb / np.linalg.norm(cb, axis=-1, keepdims=True)).astype(np.float32)
        K = rng.standard_normal((64, G * g)).astype(np.float16).astype(np.float32)
        r, c = oracle.encode_groups(K, cb)
        Kg = K.astype(np.float64).reshape(64, G, g)
        s = np.einsum("ngi,gci->ngc", Kg / np.linalg.norm(Kg, axis=-1, keepdims=True), cb.astype(np.float64))
        srt = np.sort(s, axis=-1)
        clear = (srt[..., -1] - srt[..., -2]) > 1e-5
        assert clear.mean() > 0.95
        assert (c[clear] == s.argmax(-1)[clear]).all()
        assert np.allclose(r, np.linalg.norm(Kg, axis=-1), rtol=3e-7, atol=0)


def test_encode_zero_group():
    cb = np.eye(16, dtype=np.float32)[None].repeat(8, 0)[:, :16]      # [8, 16, 16]
    K = np.zeros((2, 128), np.float32)
    r, c = oracle.encode_groups(K, cb)
    assert (r == 0).all() and (c == 0).all()                        # 0/(0+EPS)=0, argmax -> first


# ------------------------------------------------------------------ decode --
def _complex_rope_logits(q, k, pos, theta):
    """<q, R(pos) k> / sqrt(dh) via complex multiplication (independent of
    rotate_half): k_j + i k_{j+h} times exp(i pos f_j)."""
    dh = q.shape[-1]
    h = dh // 2
    f = theta ** (-2.0 * np.arange(h) / dh)
    kc = (k[:, :h] + 1j * k[:, h:]) * np.exp(1j * pos[:, None] * f[None, :])
    kr = np.concatenate([kc.real, kc.imag], axis=1)
    return q @ kr.T / math.sqrt(dh)


def _textbook(wl, pool):
    """Reconstruct every token's key in fp64 from the pool and run textbook
    attention with complex-number RoPE."""
    plan = wl.plan
    out = np.zeros((plan.num_seqs, wl.num_q, wl.dh))
    for sh in range(plan.num_seqs * plan.num_kv):
        s, h = divmod(sh, plan.num_kv)
        keys, vals, poss = [], [], []
        for p in range(int(plan.row_start[sh]), int(plan.row_start[sh + 1])):
            tid, n = int(plan.tier[p]), int(plan.count[p])
            if tid == fmt.DENSE_TIER_ID:
                k = oracle.unpack_page(pool["pages"], plan.ptable[p], tid, n, wl.dh).astype(np.float64)
            else:
                g, _ = fmt.TIER_GEOMETRY[tid]
                G = wl.dh // g
                codes, r_hat = oracle.unpack_page(pool["pages"], plan.ptable[p], tid, n, wl.dh)
                cb = wl.codebooks[tid][h].astype(np.float64)
                k = (cb[np.arange(G)[None, :], codes] * r_hat[..., None]).reshape(n, wl.dh)
            keys.append(k)
            vals.append(oracle.v_page_rows(pool["v_pool"], plan.vslot[p], n, wl.dh).astype(np.float64))
            poss.append(plan.positions[p, :n].astype(np.float64))
        K, V, pos = np.concatenate(keys), np.concatenate(vals), np.concatenate(poss)
        q = wl.q[s, h * wl.gqa:(h + 1) * wl.gqa].astype(np.float64)
        lg = _complex_rope_logits(q, K, pos, wl.rope_theta)
        e = np.exp(lg - lg.max(1, keepdims=True))
        out[s, h * wl.gqa:(h + 1) * wl.gqa] = (e / e.sum(1, keepdims=True)) @ V
    return out


def test_decode_oracle_matches_textbook_attention():
    wl = synth.make_decode_workload(2, ctx_override=700)
    pool = oracle.build_pool(wl)
    a = oracle.decode_mode_b(pool, wl.plan, wl.codebooks, wl.q, wl.gqa, wl.rope_theta)
    b = _textbook(wl, pool)
    assert np.abs(a - b).max() < 1e-10


def test_decode_oracle_single_token_and_uniform():
    wl = synth.make_decode_workload(1, ctx_override=1)
    pool = oracle.build_pool(wl)
    out = oracle.decode_mode_b(pool, wl.plan, wl.codebooks, wl.q, wl.gqa, wl.rope_theta)
    for h in range(wl.num_kv):                       # one token: softmax = 1, out = V row
        v = wl.V[0][h, 0].astype(np.float64)
        assert np.abs(out[0, h * wl.gqa:(h + 1) * wl.gqa] - v[None]).max() < 1e-12
    wl = synth.make_decode_workload(1, ctx_override=50)
    pool = oracle.build_pool(wl)
    q0 = np.zeros_like(wl.q)                         # all logits 0 -> mean of V
    out = oracle.decode_mode_b(pool, wl.plan, wl.codebooks, q0, wl.gqa, wl.rope_theta)
    for h in range(wl.num_kv):
        mean = wl.V[0][h].astype(np.float64).mean(0)
        assert np.abs(out[0, h * wl.gqa] - mean).max() < 1e-12


def test_decode_oracle_matches_torch_golden():
    z = np.load(os.path.join(GOLD, "decode_golden.npz"))
    for name in ("d128_g4", "d64_g4", "d128_g8"):
        n_tok, gqa, dh = (int(x) for x in z[name + "__meta"])
        G, g = dh // 16, 16
        cb = z[name + "__cb"].astype(np.float64)
        codes, r_hat, pos = z[name + "__codes"], z[name + "__r_hat"].astype(np.float64), z[name + "__pos"]
        q = z[name + "__q"].astype(np.float64)
        inv = oracle.rope_inv_freq(dh, 500000.0)
        ang = pos[:, None].astype(np.float64) * inv[None]
        ang = np.concatenate([ang, ang], 1)
        cw = cb[np.arange(G)[None, :], codes]
        lg = oracle.mode_b_logits(q, pos, np.cos(ang), np.sin(ang), cw, r_hat, None, G, g)
        assert np.abs(lg - z[name + "__logits"]).max() < 2e-5
        e = np.exp(lg - lg.max(1, keepdims=True))
        out = (e / e.sum(1, keepdims=True)) @ z[name + "__V"].astype(np.float64)
        assert np.abs(out - z[name + "__out"]).max() < 2e-5


@pytest.mark.parametrize("config, ctx", [(1, 4096), (2, 4096)])
def test_radius_format_error(config, ctx):
    # The parity definition scores compressed pages on the page-decoded radius
    # r_hat = code / 127 * r_scale; the reference's torch path scores its
    # fp32 radii (spherical_kv_pipeline.py:2137, 2175-2176).  Their gap is the
    # format's error, reported here apart from any kernel's error.
    wl = synth.make_decode_workload(config, ctx_override=ctx)
    pool = oracle.build_pool(wl, with_codes=True)
    plan, dh = wl.plan, wl.dh
    args = (pool, plan, wl.codebooks, wl.q, wl.gqa, wl.rope_theta)
    o_hat = oracle.decode_mode_b(*args)
    o_r = oracle.decode_mode_b(*args, r_exact=pool["r"])
    # r_exact replaces r_hat: passing r_hat itself reproduces the default
    r_hat_all = np.zeros(pool["r"].shape, np.float64)
    for p in range(plan.num_rows):
        tid, n = int(plan.tier[p]), int(plan.count[p])
        if tid != fmt.DENSE_TIER_ID:
            G = dh // fmt.TIER_GEOMETRY[tid][0]
            r_hat_all[p, :n, :G] = oracle.unpack_page(pool["pages"], plan.ptable[p], tid, n, dh)[1]
    assert np.array_equal(oracle.decode_mode_b(*args, r_exact=r_hat_all), o_hat)
    gap = np.abs(o_r - o_hat).max()
    assert gap > 0
    # bound: |r - r_hat| <= scale / 254 per group, and |<q_g, c>| <= ||q_g||
    # for unit centroids (sum over groups <= sqrt(G) ||q||), so every logit
    # moves by at most delta; softmax weights then move by a factor within
    # e^(+-2 delta), so |d out| <= (e^(2 delta) - 1) max |V|
    scale_max = max(float(np.abs(pool["r"][p]).max()) for p in range(plan.num_rows))
    qn = np.linalg.norm(wl.q.astype(np.float64), axis=-1).max()
    delta = math.sqrt(dh // 16) * qn * scale_max / 254 / math.sqrt(dh)
    vmax = max(float(np.abs(v.astype(np.float64)).max()) for v in wl.V)
    assert gap <= (math.exp(2 * delta) - 1) * vmax
    print(f"config {config} ctx {ctx}: max |out(r) - out(r_hat)| = {gap:.3e} "
          f"(mean {np.abs(o_r - o_hat).mean():.3e}; bound {(math.exp(2 * delta) - 1) * vmax:.3e})")


def test_unpack_page_round_trip():
    wl = synth.make_decode_workload(2, ctx_override=400)
    pool = oracle.build_pool(wl, with_codes=True)
    plan = wl.plan
    for p in range(plan.num_rows):
        tid, n = int(plan.tier[p]), int(plan.count[p])
        if tid == fmt.DENSE_TIER_ID:
            continue
        g, _ = fmt.TIER_GEOMETRY[tid]
        G = wl.dh // g
        codes, r_hat = oracle.unpack_page(pool["pages"], plan.ptable[p], tid, n, wl.dh)
        assert (codes == pool["codes"][p, :n, :G]).all()
        r = pool["r"][p, :n, :G]
        scale, rc = oracle.radius_codes(r)
        assert np.allclose(r_hat, rc / 127.0 * scale.astype(np.float64)[None], rtol=0, atol=0)
        # format error of the int8 radius: at most half a step
        assert (np.abs(r_hat - r) <= 0.5 / 127 * scale[None] * (1 + 1e-6) + 1e-30).all()


def test_ragged_oracle_matches_mode_b():
    # the logits-only contract equals the full decode's logits with exact tables
    wl = synth.make_decode_workload(2, ctx_override=1200)
    pool = oracle.build_pool(wl)
    plan = wl.plan
    rows = [p for p in range(plan.num_rows) if plan.tier[p] == 1 and plan.seq_head[p] == 0]
    cos_t, sin_t = fmt.rope_tables(1300, wl.dh, wl.rope_theta)
    pos = plan.positions[rows].reshape(-1)
    lg = oracle.ragged_logits(pool["pages"], plan.ptable[rows], np.zeros(len(rows), np.int32), pos,
                              cos_t, sin_t, wl.q[0, :wl.gqa].astype(np.float32), wl.gqa,
                              wl.codebooks[1][0].reshape(-1, 64, 16), wl.dh, 8, 16, 6, 16)
    keys = []
    for p in rows:
        n = int(plan.count[p])
        codes, r_hat = oracle.unpack_page(pool["pages"], plan.ptable[p], 1, n, wl.dh)
        keys.append((wl.codebooks[1][0].astype(np.float64)[np.arange(8)[None], codes] * r_hat[..., None]).reshape(n, -1))
    K = np.concatenate(keys)
    valid = pos >= 0
    ref = _complex_rope_logits(wl.q[0, :wl.gqa].astype(np.float64), K, pos[valid].astype(np.float64), wl.rope_theta)
    assert np.abs(lg[:, valid] - ref).max() < 1e-5       # fp32 cos/sin tables
    assert np.isneginf(lg[:, ~valid]).all()
