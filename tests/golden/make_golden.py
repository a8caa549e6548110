"""Writes the committed golden fixtures under tests/golden/.

The reference has no tests, fixtures or golden vectors for this path, so these
fixtures are the pins.  They are produced by torch on the CPU executing the
reference's own op sequence, restated here op for op (the reference module is
not imported):

* encode:  spherical_kv_pipeline.py:1136-1144
           K.view(N,G,g); r = K.norm(dim=-1); dir = K / (r[...,None] + EPS);
           sims = einsum('ngi,gci->ngc', dir, cb); codes = sims.argmax(-1)
* page:    pagebuilder.py:17-33, paging.py:20-31, bitpacking.py:5-29
* decode:  spherical_kv_pipeline.py:2143-2177 (logits), 2348 (softmax),
           2367 (attn @ V), in torch fp32, with fp32 cos/sin tables built from
           fp64 angles (the documented RoPE convention of this build).

Recorded with every encode case: torch version and the fp64 top-2 similarity
margin of every group (a margin of a few 1e-7 is where summation order decides
the argmax).  The t1_n1_tie* cases are single-token tier-1 pages built on
near-ties: they pin the summation order of torch's N = 1 path (MKL M = 1).
tail_golden.npz holds single-token tier-3 encodes (near-ties and ordinary
tokens): the decode-time tail's encode of each new key.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import torch_port  # noqa: E402  (the torch restatements of the reference's ops)

EPS = torch_port.EPS
HEADER_BYTES = torch_port.HEADER_BYTES


def t_encode(K: torch.Tensor, cb: torch.Tensor, g: int, G: int):
    return torch_port.encode_chunk(K, cb, g, G)


def t_pack_bits(values: torch.Tensor, bits: int) -> torch.Tensor:
    return torch_port.pack_bits(values, bits)


def t_build_page(r: torch.Tensor, codes: torch.Tensor, tier_id: int, b_theta: int) -> torch.Tensor:
    return torch_port.build_page(r, codes, tier_id, b_theta)


def margins(K: np.ndarray, cb: np.ndarray, g: int, G: int) -> np.ndarray:
    Kg = K.astype(np.float64).reshape(-1, G, g)
    d = Kg / (np.linalg.norm(Kg, axis=-1, keepdims=True) + EPS)
    s = np.einsum('ngi,gci->ngc', d, cb.astype(np.float64))
    s.sort(axis=-1)
    return s[..., -1] - s[..., -2]


def encode_case(name, rng, N, tier_id, g, b, dh=128, kind="normal"):
    G, C = dh // g, 2 ** b
    cb = rng.standard_normal((G, C, g))
    cb = (cb / np.linalg.norm(cb, axis=-1, keepdims=True)).astype(np.float32)
    if kind == "normal":
        K = rng.standard_normal((N, dh)).astype(np.float16)
    else:  # config-3 style: lognormal channel scale, 1% outlier channels x8
        sc = np.exp(rng.normal(0, 0.5, size=dh))
        sc[rng.choice(dh, size=max(1, dh // 100), replace=False)] *= 8
        K = (rng.standard_normal((N, dh)) * sc).astype(np.float16)
    if kind == "zeros":
        K[:] = 0
    Kt = torch.from_numpy(K.astype(np.float32))
    r, codes = t_encode(Kt, torch.from_numpy(cb), g, G)
    page = t_build_page(r, codes, tier_id, b)
    return {f"{name}__K": K, f"{name}__cb": cb, f"{name}__r": r.numpy(), f"{name}__codes": codes.numpy(),
            f"{name}__page": page.numpy(), f"{name}__margin": margins(K, cb, g, G).astype(np.float64),
            f"{name}__meta": np.array([N, tier_id, g, b, dh], np.int64)}


def tie_case(name, rng, dh=128, tries=4096):
    """One single-token tier-1 page (N = 1, g = 16, C = 64: the only encode
    that reaches MKL's M = 1 sgemm) whose every group sits on a near-tie:
    K_g ~ r * (c_a + c_b) for two random centroids a < b, rounded to fp16, and
    of `tries` fp16 roundings of randomly perturbed copies the one with the
    smallest fp64 top-2 margin is kept (margins of a few 1e-8 to 1e-7, where
    the fp32 summation order decides the argmax)."""
    g, b = 16, 6
    G, C = dh // g, 2 ** b
    cb = rng.standard_normal((G, C, g))
    cb = (cb / np.linalg.norm(cb, axis=-1, keepdims=True)).astype(np.float32)
    K = np.zeros((1, dh), np.float16)
    for gi in range(G):
        a, bb = rng.choice(C, size=2, replace=False)
        base = cb[gi, a].astype(np.float64) + cb[gi, bb].astype(np.float64)
        base *= rng.uniform(1.0, 8.0) / np.linalg.norm(base)
        cand = (base[None, :] * (1.0 + 2e-3 * rng.standard_normal((tries, g)))).astype(np.float16)
        d = cand.astype(np.float64)
        d /= np.linalg.norm(d, axis=-1, keepdims=True) + EPS
        s = d @ cb[gi].astype(np.float64).T                          # [tries, C]
        top = np.sort(s, axis=-1)
        pick = int(np.argmin(top[:, -1] - top[:, -2]))
        K[0, gi * g:(gi + 1) * g] = cand[pick]
    Kt = torch.from_numpy(K.astype(np.float32))
    r, codes = t_encode(Kt, torch.from_numpy(cb), g, G)
    page = t_build_page(r, codes, 1, b)
    return {f"{name}__K": K, f"{name}__cb": cb, f"{name}__r": r.numpy(), f"{name}__codes": codes.numpy(),
            f"{name}__page": page.numpy(), f"{name}__margin": margins(K, cb, g, G).astype(np.float64),
            f"{name}__meta": np.array([1, 1, g, b, dh], np.int64)}


def tie3_case(name, rng, dh=128, tries=4096):
    """One single-token tier-3 encode (N = 1, g = 32, C = 8: the decode-time
    encode of _append_decode_kv / the new token, spherical_kv_pipeline.py:
    2311-2313, 2423-2425; N*g*C = 256 < 400 takes torch's naive bmm loop)
    whose every group sits on a near-tie between two centroids, built as
    tie_case builds the tier-1 ones."""
    g, b = 32, 3
    G, C = dh // g, 2 ** b
    cb = rng.standard_normal((G, C, g))
    cb = (cb / np.linalg.norm(cb, axis=-1, keepdims=True)).astype(np.float32)
    K = np.zeros((1, dh), np.float16)
    for gi in range(G):
        a, bb = rng.choice(C, size=2, replace=False)
        base = cb[gi, a].astype(np.float64) + cb[gi, bb].astype(np.float64)
        base *= rng.uniform(1.0, 8.0) / np.linalg.norm(base)
        cand = (base[None, :] * (1.0 + 2e-3 * rng.standard_normal((tries, g)))).astype(np.float16)
        d = cand.astype(np.float64)
        d /= np.linalg.norm(d, axis=-1, keepdims=True) + EPS
        s = d @ cb[gi].astype(np.float64).T
        top = np.sort(s, axis=-1)
        pick = int(np.argmin(top[:, -1] - top[:, -2]))
        K[0, gi * g:(gi + 1) * g] = cand[pick]
    Kt = torch.from_numpy(K.astype(np.float32))
    r, codes = t_encode(Kt, torch.from_numpy(cb), g, G)
    return {f"{name}__K": K, f"{name}__cb": cb, f"{name}__r": r.numpy(), f"{name}__codes": codes.numpy(),
            f"{name}__margin": margins(K, cb, g, G).astype(np.float64),
            f"{name}__meta": np.array([1, 3, g, b, dh], np.int64)}


def tail_fixtures():
    """Single-token tier-3 encodes (the decode-time tail's), tails_golden.npz:
    24 near-tie tokens at dh 128 and 12 at dh 64, plus 32 ordinary tokens."""
    rng = np.random.default_rng(20261203)
    out = {}
    for i in range(24):
        out.update(tie3_case(f"t3_n1_tie{i}", rng, dh=128))
    for i in range(12):
        out.update(tie3_case(f"t3_n1_tie_dh64_{i}", rng, dh=64))
    for i in range(32):
        out.update(encode_case(f"t3_n1_plain{i}", rng, 1, 3, 32, 3, dh=128 if i % 4 else 64,
                               kind="config3" if i % 2 else "normal"))
    out["torch_version"] = np.array(torch.__version__)
    return out


def decode_case(name, rng, n_tok, gqa, dh, theta=500000.0):
    """Torch fp32 restatement of the Mode-B reference decode on one KV head
    with one tier-1 block, positions spread over [0, 40000)."""
    g, b = 16, 6
    G, C = dh // g, 2 ** b
    cb = rng.standard_normal((G, C, g))
    cb = (cb / np.linalg.norm(cb, axis=-1, keepdims=True)).astype(np.float32)
    codes = rng.integers(0, C, size=(n_tok, G)).astype(np.int32)
    r_hat = np.abs(rng.standard_normal((n_tok, G)) * 4).astype(np.float32)
    pos = np.sort(rng.choice(40000, size=n_tok, replace=False)).astype(np.int64)
    q = rng.standard_normal((gqa, dh)).astype(np.float16)
    V = rng.standard_normal((n_tok, dh)).astype(np.float16)
    j = np.arange(dh // 2, dtype=np.float64)
    ang = pos[:, None].astype(np.float64) * (theta ** (-2.0 * j / dh))[None, :]
    ang = np.concatenate([ang, ang], axis=1)
    cos_i, sin_i = torch.from_numpy(np.cos(ang).astype(np.float32)), torch.from_numpy(np.sin(ang).astype(np.float32))
    qt = torch.from_numpy(q.astype(np.float32))
    qe = qt.unsqueeze(1)
    half = dh // 2
    qh = torch.cat([-qe[..., half:], qe[..., :half]], dim=-1)
    q_rot = qe * cos_i.unsqueeze(0) - qh * sin_i.unsqueeze(0)
    q_rot_g = q_rot.view(gqa, n_tok, G, g)
    q_norms = q_rot_g.norm(dim=-1, keepdim=True).clamp(min=1e-6)
    q_normed = q_rot_g / q_norms
    cbt = torch.from_numpy(cb)
    cw = cbt[torch.arange(G).unsqueeze(1), torch.from_numpy(codes).long().T].permute(1, 0, 2)
    cos_pg = (q_normed * cw.unsqueeze(0)).sum(-1).clamp(-1.0, 1.0)
    logits = (q_norms.squeeze(-1) * cos_pg * torch.from_numpy(r_hat).unsqueeze(0)).sum(-1) / math.sqrt(dh)
    attn = torch.softmax(logits, dim=1)
    out = attn @ torch.from_numpy(V.astype(np.float32))
    return {f"{name}__cb": cb, f"{name}__codes": codes, f"{name}__r_hat": r_hat, f"{name}__pos": pos,
            f"{name}__q": q, f"{name}__V": V, f"{name}__logits": logits.numpy(), f"{name}__out": out.numpy(),
            f"{name}__meta": np.array([n_tok, gqa, dh], np.int64)}


def main():
    torch.set_num_threads(1)
    rng = np.random.default_rng(20260101)
    enc = {}
    enc.update(encode_case("t1_n16", rng, 16, 1, 16, 6))
    enc.update(encode_case("t1_n16_c3", rng, 16, 1, 16, 6, kind="config3"))
    enc.update(encode_case("t2_n16", rng, 16, 2, 16, 4))
    enc.update(encode_case("t3_n16", rng, 16, 3, 32, 3))
    enc.update(encode_case("t1_n7", rng, 7, 1, 16, 6))
    enc.update(encode_case("t2_n2", rng, 2, 2, 16, 4))
    enc.update(encode_case("t2_n1", rng, 1, 2, 16, 4))       # torch naive bmm path
    enc.update(encode_case("t3_n1", rng, 1, 3, 32, 3))       # torch naive bmm path
    enc.update(encode_case("t1_n16_dh64", rng, 16, 1, 16, 6, dh=64))
    enc.update(encode_case("t1_zero", rng, 16, 1, 16, 6, kind="zeros"))
    for i in range(24):                                        # 384 more tier-1 tokens, config-3 data
        enc.update(encode_case(f"t1_bulk{i}", rng, 16, 1 + (i % 2), 16, 6 - 2 * (i % 2), kind="config3"))
    # single-token tier-1 pages on near-ties (MKL's M = 1 order decides the
    # codes); their own generator, so the cases above are unchanged
    rng_t = np.random.default_rng(20261202)
    for i in range(48):
        enc.update(tie_case(f"t1_n1_tie{i}", rng_t, dh=128))
    for i in range(16):
        enc.update(tie_case(f"t1_n1_tie_dh64_{i}", rng_t, dh=64))
    enc["torch_version"] = np.array(torch.__version__)
    enc["blas"] = np.array("oneMKL 2024.2 (torch CPU, AVX-512 host)")
    np.savez_compressed(os.path.join(HERE, "encode_golden.npz"), **enc)

    dec = {}
    dec.update(decode_case("d128_g4", rng, 300, 4, 128))
    dec.update(decode_case("d64_g4", rng, 200, 4, 64))
    dec.update(decode_case("d128_g8", rng, 100, 8, 128))
    dec["torch_version"] = np.array(torch.__version__)
    np.savez_compressed(os.path.join(HERE, "decode_golden.npz"), **dec)
    np.savez_compressed(os.path.join(HERE, "tail_golden.npz"), **tail_fixtures())
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
