"""Pins of the decode-time tail oracle (oracle/tail.py): the tier-3
single-token encode against torch CPU fixtures and fp64 brute force, the
flushed page's layout, and closed forms of a decode step's tail terms."""
import math
import os

import numpy as np

import oracle
import sphkv_format as fmt
from oracle.tail import TailOracle, run_steps

HERE = os.path.dirname(os.path.abspath(__file__))


def _cb3(rng, num_kv, dh):
    cb = rng.standard_normal((num_kv, dh // 32, 8, 32))
    return (cb / np.linalg.norm(cb, axis=-1, keepdims=True)).astype(np.float32)


def test_tail_encode_matches_torch_fixtures():
    # bit-exact against torch CPU running the reference's op sequence on one
    # token (tests/golden/make_golden.py: near-ties and ordinary tokens)
    d = np.load(os.path.join(HERE, "golden", "tail_golden.npz"))
    names = sorted({k.split("__")[0] for k in d.keys() if "__" in k})
    assert len(names) == 68
    for n in names:
        K, cb = d[n + "__K"], d[n + "__cb"]
        dh = K.shape[1]
        t = TailOracle(1, 1, dh, cb[None])
        r, codes = t.encode(0, K[0])
        assert (codes == d[n + "__codes"][0]).all(), n
        assert (r.view(np.uint32) == d[n + "__r"][0].view(np.uint32)).all(), n


def test_tail_encode_matches_fp64_bruteforce():
    rng = np.random.default_rng(5)
    for dh in (64, 128):
        cb = _cb3(rng, 1, dh)
        t = TailOracle(1, 1, dh, cb)
        for _ in range(200):
            k = (rng.standard_normal(dh) * np.exp(rng.normal(0, 0.5, dh))).astype(np.float16)
            r, codes = t.encode(0, k)
            kg = k.astype(np.float64).reshape(-1, 32)
            rn = np.linalg.norm(kg, axis=-1)
            s = np.einsum("gi,gci->gc", kg / (rn[:, None] + 1e-8), cb[0].astype(np.float64))
            top = np.sort(s, axis=-1)
            ok = top[:, -1] - top[:, -2] > 1e-5
            assert (codes[ok] == s.argmax(-1)[ok]).all()
            assert np.allclose(r, rn, rtol=1e-6, atol=0)


def test_flush_builds_tier3_page():
    # 16 appends: staging empties and one page holds the 16 tokens, laid out
    # as pagebuilder.py:8-33 (header, max-radius scales, 3-bit LSB-first
    # codes, int8 radius codes)
    rng = np.random.default_rng(6)
    dh, G = 128, 4
    t = TailOracle(1, 2, dh, _cb3(rng, 2, dh))
    ks = rng.standard_normal((16, dh)).astype(np.float16)
    vs = rng.standard_normal((16, dh)).astype(np.float16)
    enc = [t.encode(1, k) for k in ks]
    for i in range(16):
        t.append(0, 1, ks[i], vs[i], 1000 + i)
        assert len(t.staged[1]) == (i + 1) % 16
    assert len(t.pages[1]) == 1 and not t.pages[0]
    page, pos, V = t.pages[1][0]
    r = np.stack([e[0] for e in enc])
    codes = np.stack([e[1] for e in enc])
    assert page.size == fmt.page_nbytes(3, 16, dh) == 112
    assert page[0] == 3 and page[1] == 16 and not page[2:8].any()
    scale = np.frombuffer(page[8:8 + 4 * G].tobytes(), "<f4")
    assert (scale == r.max(axis=0)).all()
    got = oracle.unpack_bits(page[8 + 4 * G:8 + 4 * G + 24], 16 * G, 3).reshape(16, G)
    assert (got == codes).all()
    rc = page[8 + 4 * G + 24:].view(np.int8).reshape(16, G)
    want = np.clip(np.rint((r / scale[None, :]).astype(np.float32) * np.float32(127)), -127, 127)
    assert (rc == want).all()
    assert (pos == 1000 + np.arange(16)).all() and (V.view(np.uint16) == vs.view(np.uint16)).all()


def _empty_plan(num_seqs, num_kv, dh):
    return fmt.plan_pages([np.zeros(0, np.int32)] * (num_seqs * num_kv), None, num_seqs, num_kv, dh, 16)


def _step(plan, tail, q, gqa, k_new, v_new, cur_pos, theta=500000.0):
    pool = {"pages": np.zeros(16, np.uint8), "v_pool": np.zeros((0, 16 * plan.dh), np.float16)}
    return oracle.decode_mode_b(pool, plan, {}, q, gqa, theta, tail=tail, k_new=k_new, v_new=v_new,
                                cur_pos=cur_pos)


def test_new_token_alone_returns_its_v():
    # no context, nothing staged: the softmax has one term
    rng = np.random.default_rng(7)
    dh, gqa, nkv = 128, 4, 2
    plan = _empty_plan(1, nkv, dh)
    t = TailOracle(1, nkv, dh, _cb3(rng, nkv, dh))
    q = rng.standard_normal((1, nkv * gqa, dh)).astype(np.float16)
    k = rng.standard_normal((1, nkv, dh)).astype(np.float16)
    v = rng.standard_normal((1, nkv, dh)).astype(np.float16)
    out = _step(plan, t, q, gqa, k, v, np.array([777]))
    for h in range(nkv):
        assert (out[0, h * gqa:(h + 1) * gqa] == v[0, h].astype(np.float64)[None]).all()


def test_equal_tail_tokens_average_v():
    # staged tokens and the new token with the same key at the same position
    # have equal logits: the output is the mean of their V rows
    rng = np.random.default_rng(8)
    dh, gqa = 64, 2
    plan = _empty_plan(1, 1, dh)
    t = TailOracle(1, 1, dh, _cb3(rng, 1, dh))
    k = rng.standard_normal(dh).astype(np.float16)
    vs = rng.standard_normal((6, dh)).astype(np.float16)
    for i in range(5):
        t.append(0, 0, k, vs[i], 4321)
    q = rng.standard_normal((1, gqa, dh)).astype(np.float16)
    out = _step(plan, t, q, gqa, k[None, None], vs[5][None, None], np.array([4321]))
    want = vs.astype(np.float64).mean(axis=0)
    assert np.abs(out[0] - want[None]).max() < 1e-12


def test_tail_logits_equal_textbook_attention():
    # staged token and new token logits: <R(-t) q, k_hat> / sqrt(dh) with
    # k_hat = concat_g r_g c_g, through the dense (textbook) path
    rng = np.random.default_rng(9)
    dh, gqa = 128, 4
    cb3 = _cb3(rng, 1, dh)
    t = TailOracle(1, 1, dh, cb3)
    ks = rng.standard_normal((4, dh)).astype(np.float16)
    pos = np.array([5, 90000, 123456, 7])
    for i in range(3):
        t.append(0, 0, ks[i], np.zeros(dh, np.float16), pos[i])
    q = rng.standard_normal((gqa, dh)).astype(np.float16)
    inv = oracle.rope_inv_freq(dh, 500000.0)
    lg, V = t.terms(0, 0, q, inv, ks[3], np.zeros(dh, np.float16), pos[3])
    assert lg.shape == (gqa, 4) and V.shape == (4, dh)
    for i in range(4):
        r, codes = t.encode(0, ks[i])
        khat = np.concatenate([r[g] * cb3[0, g, codes[g]].astype(np.float64) for g in range(dh // 32)])
        ang = pos[i] * inv
        ang = np.concatenate([ang, ang])
        want = oracle.mode_b_logits(q.astype(np.float64), None, np.cos(ang)[None], np.sin(ang)[None], None, None,
                                    khat[None], 0, 0)[:, 0]
        assert np.abs(lg[:, i] - want).max() < 1e-9 * max(1.0, np.abs(want).max())


def test_flush_changes_logits_by_radius_rounding_only():
    # a token scored from the flushed page (r_hat = int8 / 127 * scale) and
    # from staging (fp32 r) differ by at most sum_g |q_g| scale_g / 254 / sqrt(dh)
    rng = np.random.default_rng(10)
    dh, gqa, G = 128, 4, 4
    t = TailOracle(1, 1, dh, _cb3(rng, 1, dh))
    ks = (rng.standard_normal((16, dh)) * np.exp(rng.normal(0, 0.5, dh))).astype(np.float16)
    pos = np.arange(16) + 3000
    q = rng.standard_normal((gqa, dh)).astype(np.float16)
    inv = oracle.rope_inv_freq(dh, 500000.0)
    for i in range(15):
        t.append(0, 0, ks[i], np.zeros(dh, np.float16), pos[i])
    before, _ = t.terms(0, 0, q, inv, ks[15], np.zeros(dh, np.float16), pos[15])
    t.append(0, 0, ks[15], np.zeros(dh, np.float16), pos[15])
    after, _ = t.terms(0, 0, q, inv)
    scale = np.frombuffer(t.pages[0][0][0][8:8 + 4 * G].tobytes(), "<f4").astype(np.float64)
    # |<R(-t) q, c>_g| <= |(R(-t) q)_g|: the rotation mixes group g with its
    # RoPE partner group g + G/2, so |(R(-t) q)_g| <= sqrt(2) max(|q_g|, |q_g'|)
    qn = np.linalg.norm(q.astype(np.float64).reshape(gqa, G, 32), axis=-1)
    qn2 = np.maximum(qn, qn[:, (np.arange(G) + G // 2) % G])
    bound = (np.sqrt(2.0) * qn2 * scale[None, :] / 254.0).sum(axis=1) / math.sqrt(dh) + 1e-9
    diff = np.abs(after - before)
    assert (diff <= bound[:, None]).all()
    assert diff.max() > 0                                  # the rounding is visible


def test_run_steps_multi_head_order():
    # every (seq, head) stages its own tokens; flushes happen per (seq, head)
    rng = np.random.default_rng(11)
    dh, nkv, ns = 64, 2, 2
    t = TailOracle(ns, nkv, dh, _cb3(rng, nkv, dh))
    T = 19
    ks = rng.standard_normal((T, ns, nkv, dh)).astype(np.float16)
    vs = rng.standard_normal((T, ns, nkv, dh)).astype(np.float16)
    pos = np.arange(T)[:, None] + np.array([100, 200])[None, :]
    run_steps(t, ks, vs, pos)
    for sh in range(ns * nkv):
        assert len(t.pages[sh]) == 1 and len(t.staged[sh]) == 3
        s, h = divmod(sh, nkv)
        assert (t.pages[sh][0][1] == pos[:16, s]).all()
        assert [x[3] for x in t.staged[sh]] == list(pos[16:, s])


def test_step_with_context_equals_full_decode():
    # the log-sum-exp merge of the context's (out, lse) with the tail terms is
    # the one-softmax decode over both
    import sphkv_synth as synth
    from oracle.tail import step_with_context
    wl = synth.make_decode_workload(2, ctx_override=700)
    st = synth.make_tail_steps(wl, 20)
    cpu = oracle.build_pool(wl)
    t = TailOracle(wl.num_seqs, wl.num_kv, wl.dh, st.cb3)
    run_steps(t, st.k[:18], st.v[:18], st.pos[:18])         # one flushed page + 2 staged per head
    q = st.q[18]
    full = oracle.decode_mode_b(cpu, wl.plan, wl.codebooks, q, wl.gqa, wl.rope_theta, tail=t,
                                k_new=st.k[18], v_new=st.v[18], cur_pos=st.pos[18])
    ctx_out, ctx_lse = oracle.decode_mode_b(cpu, wl.plan, wl.codebooks, q, wl.gqa, wl.rope_theta, return_lse=True)
    got = step_with_context(ctx_out, ctx_lse, t, q, wl.gqa, wl.rope_theta, st.k[18], st.v[18], st.pos[18])
    assert np.abs(got - full).max() < 1e-12
    # and the tail moves the output (it is not a no-op)
    assert np.abs(ctx_out - full).max() > 1e-3
