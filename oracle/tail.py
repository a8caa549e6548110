"""Decode-time tail of the Mode-B path, restated on the CPU.  TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module, as the checker.  It restates, per (sequence, kv head):

* _append_decode_kv (spherical_kv_pipeline.py:2389-2448): the new pre-RoPE key
  is encoded through the tier-3 codebook as ONE token
  (_encode_keys_with_codebooks(kn, cb, g, G) with kn [1, dh], :2423-2425) and
  staged with its fp32 radii, codes, V (vn = v_new.float(), :2398) and
  position (:2428-2441); at PAGE_SIZE staged tokens it is flushed (:2443-2444);
* _flush_decode_page (:2449-2475): build_page_from_codes(r, theta, b3)
  (pagebuilder.py:36-42 -> build_page :8-33) over the staged tokens, kept with
  their positions and V as one decode page (:2487-2495);
* the decode terms of _compressed_head_attention_batched: decode pages scored
  like context pages (:2180-2246; the page bytes' r_hat, as the fused path
  reads them), staged tokens with their unquantised radii (:2248-2285), and
  the new token encoded through the tier-3 codebook and scored at current_pos
  (:2294-2342), all in one softmax with the context (:2347-2348) and
  attn @ V (:2364-2367, V of the new token = vn).

PAGE_SIZE is 16 here, as in every BASELINE configuration (the reference's
config.py:4 default is 128).
"""
from __future__ import annotations

from typing import Dict, List, Tuple

import numpy as np

from oracle import TIER_GEOMETRY, build_page, encode_groups, mode_b_logits, unpack_page

TAIL_TIER = 3                       # decode tokens are classified recent: tier b3 (:2415-2416)
PAGE_SIZE = 16


class TailOracle:
    """Staging buffers and flushed decode pages of every (sequence, kv head).

    cb3: fp32 [num_kv, G3, 8, 32] tier-3 codebooks (unit rows)."""

    def __init__(self, num_seqs: int, num_kv: int, dh: int, cb3: np.ndarray, page_size: int = PAGE_SIZE):
        g, b = TIER_GEOMETRY[TAIL_TIER]
        self.num_seqs, self.num_kv, self.dh, self.page_size = num_seqs, num_kv, dh, page_size
        self.G = dh // g
        self.b = b
        self.cb3 = np.ascontiguousarray(cb3, np.float32)
        assert self.cb3.shape == (num_kv, self.G, 2 ** b, g)
        n = num_seqs * num_kv
        # staged tokens: (r fp32 [G], codes int32 [G], v fp16 [dh], position)
        self.staged: List[List[Tuple[np.ndarray, np.ndarray, np.ndarray, int]]] = [[] for _ in range(n)]
        # flushed decode pages: (page bytes, positions int64 [n], V fp16 [n, dh])
        self.pages: List[List[Tuple[np.ndarray, np.ndarray, np.ndarray]]] = [[] for _ in range(n)]

    def encode(self, h: int, k: np.ndarray):
        """One token through the tier-3 codebook of kv head h (N = 1)."""
        r, codes = encode_groups(np.asarray(k, np.float32).reshape(1, self.dh), self.cb3[h])
        return r[0], codes[0]

    def append(self, s: int, h: int, k: np.ndarray, v: np.ndarray, pos: int) -> None:
        """_append_decode_kv: stage, and flush a full page."""
        sh = s * self.num_kv + h
        r, codes = self.encode(h, k)
        self.staged[sh].append((r, codes, np.asarray(v, np.float16).copy(), int(pos)))
        if len(self.staged[sh]) >= self.page_size:
            self.flush(sh)

    def flush(self, sh: int) -> None:
        """_flush_decode_page: the staged tokens become a tier-3 page."""
        st = self.staged[sh]
        r = np.stack([x[0] for x in st]).astype(np.float32)
        codes = np.stack([x[1] for x in st]).astype(np.int32)
        page = build_page(r, codes, TAIL_TIER, self.b)
        pos = np.array([x[3] for x in st], np.int64)
        V = np.stack([x[2] for x in st]).astype(np.float16)
        self.pages[sh].append((page, pos, V))
        self.staged[sh] = []

    def terms(self, s: int, h: int, q: np.ndarray, inv_freq: np.ndarray, k_new=None, v_new=None, cur_pos=None):
        """Logits [gqa, n] (fp64, / sqrt(dh) included) and V rows [n, dh] of
        sh's decode pages, staged tokens and (if given) the new token."""
        sh = s * self.num_kv + h
        dh, G, g = self.dh, self.G, 32
        cb = self.cb3[h].astype(np.float64)
        q = np.asarray(q, np.float64)
        logits, vs = [], []

        def rope(pos):
            ang = np.asarray(pos, np.float64)[:, None] * inv_freq[None, :]
            ang = np.concatenate([ang, ang], axis=1)
            return np.cos(ang), np.sin(ang)

        for page, pos, V in self.pages[sh]:
            n = len(pos)
            th = 8 + 4 * G
            row = np.array([0, th, th + (n * G * self.b + 7) // 8])
            codes, r_hat = unpack_page(page, row, TAIL_TIER, n, dh)
            cos_t, sin_t = rope(pos)
            logits.append(mode_b_logits(q, pos, cos_t, sin_t, cb[np.arange(G)[None, :], codes], r_hat, None, G, g))
            vs.append(V.astype(np.float64))
        toks = [(r, c, v, p) for (r, c, v, p) in self.staged[sh]]
        if k_new is not None:
            r, c = self.encode(h, k_new)
            toks.append((r, c, np.asarray(v_new, np.float16), int(cur_pos)))
        if toks:
            r = np.stack([x[0] for x in toks]).astype(np.float64)
            codes = np.stack([x[1] for x in toks])
            pos = np.array([x[3] for x in toks], np.int64)
            cos_t, sin_t = rope(pos)
            logits.append(mode_b_logits(q, pos, cos_t, sin_t, cb[np.arange(G)[None, :], codes], r, None, G, g))
            vs.append(np.stack([x[2] for x in toks]).astype(np.float64))
        if not logits:
            return np.zeros((q.shape[0], 0)), np.zeros((0, dh))
        return np.concatenate(logits, axis=1), np.concatenate(vs, axis=0)


def run_steps(tail: TailOracle, ks: np.ndarray, vs: np.ndarray, pos: np.ndarray) -> None:
    """Append T steps: ks / vs [T, num_seqs, num_kv, dh], pos [T, num_seqs]."""
    for t in range(ks.shape[0]):
        for s in range(tail.num_seqs):
            for h in range(tail.num_kv):
                tail.append(s, h, ks[t, s, h], vs[t, s, h], int(pos[t, s]))


def step_with_context(ctx_out: np.ndarray, ctx_lse: np.ndarray, tail: TailOracle, q: np.ndarray, gqa: int,
                      rope_theta: float, k_new: np.ndarray, v_new: np.ndarray, cur_pos: np.ndarray) -> np.ndarray:
    """A full decode step from the page context's fp64 (out, lse)
    (decode_mode_b(..., return_lse=True), logits / sqrt(dh) in natural units)
    and the tail's terms: the two parts of one softmax merged by log-sum-exp.
    Equal to decode_mode_b(..., tail=tail, k_new=..., ...) on the same inputs;
    lets a large context be evaluated once for several tail states."""
    from oracle import rope_inv_freq
    num_seqs, nq, dh = ctx_out.shape
    inv = rope_inv_freq(dh, rope_theta)
    out = np.zeros_like(ctx_out)
    for s in range(num_seqs):
        for h in range(nq // gqa):
            sl = slice(h * gqa, (h + 1) * gqa)
            lg, V = tail.terms(s, h, q[s, sl], inv, k_new[s, h], v_new[s, h], cur_pos[s])
            lse = ctx_lse[s, sl][:, None]
            m = np.maximum(lse, lg.max(axis=1, keepdims=True))
            w_ctx = np.exp(lse - m)
            e = np.exp(lg - m)
            den = w_ctx + e.sum(axis=1, keepdims=True)
            out[s, sl] = (w_ctx * ctx_out[s, sl] + e @ V) / den
    return out
