"""CPU oracle for the angle-domain compressed-KV path.  TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, and only as the checker.  The product path
(spherical-kv_amd/) never imports it and fails loudly when its HIP library is
missing.

Contents and the reference lines each part restates (reference repo paths):

* C part (sphkv_oracle.c, built into oracle/_build/libsphkv_oracle.so):
  pack_bits (bitpacking.py:5-29), encode_groups
  (spherical_kv_pipeline.py:1130-1144, torch-CPU operation order),
  radius codes / build_page (pagebuilder.py:8-33, paging.py:20-31).
* numpy part, fp64:
  unpack_page                 inverse of pagebuilder.py:8-33
  build_pool                  spherical_kv_pipeline.py:1187-1213 (encode +
                              page + pointer-table row per chunk), placed as the
                              plan says
  decode_mode_b               spherical_kv_pipeline.py:2143-2177 (back-rotated,
                              per-group-normalised q, clipped cosine, radius,
                              / sqrt(dh)), softmax :2347-2348, attn @ V :2364-2367;
                              rotate_half :1004-1007.  Dense fp16 K tokens use
                              textbook attention <R(-t) q, k> / sqrt(dh).
  ragged_logits               the logits-only contract of fused_decode_ragged
                              (call sites spherical_kv_pipeline.py:1102-1125,
                              1865-1870) evaluated with the caller's cos/sin
                              tables.

Pins (see tests/test_oracle.py): hand-written known answers for pack_bits and
the header, brute-force fp64 argmax on unambiguous groups, committed golden
fixtures produced by torch CPU running the reference's op sequence, closed
forms of the decode (single token, equal logits, t = 0, dense textbook
attention).
"""
from __future__ import annotations

import ctypes
import functools
import os
import subprocess
import sys
from typing import Dict, Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libsphkv_oracle.so")
_lib = None

HEADER_BYTES = 8
DENSE_TIER_ID = 0xFF
TIER_GEOMETRY = {1: (16, 6), 2: (16, 4), 3: (32, 3)}


def build(force: bool = False) -> str:
    """Compile the C restatement (gcc; no fast-math, no FP contraction)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.check_call(["make", "-s", "-C", _HERE])
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        lib.orc_pack_bits.argtypes = [P, ctypes.c_int64, ctypes.c_int, P]
        lib.orc_unpack_bits.argtypes = [P, ctypes.c_int64, ctypes.c_int, P]
        lib.orc_encode_groups.argtypes = [P, ctypes.c_int64, ctypes.c_int, ctypes.c_int, P, ctypes.c_int, P, P]
        lib.orc_radius_codes.argtypes = [P, ctypes.c_int, ctypes.c_int, P, P]
        lib.orc_page_bytes.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int]
        lib.orc_page_bytes.restype = ctypes.c_int64
        lib.orc_build_page.argtypes = [P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, P]
        lib.orc_build_page.restype = ctypes.c_int64
        _lib = lib
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


# ----------------------------------------------------------------- C part --
def pack_bits(values: np.ndarray, bits: int) -> np.ndarray:
    v = np.ascontiguousarray(values, dtype=np.int32).reshape(-1)
    out = np.zeros((v.size * bits + 7) // 8, np.uint8)
    _load().orc_pack_bits(_ptr(v), v.size, bits, _ptr(out))
    return out


def unpack_bits(buf: np.ndarray, n: int, bits: int) -> np.ndarray:
    b = np.ascontiguousarray(buf, dtype=np.uint8)
    out = np.zeros(n, np.int32)
    _load().orc_unpack_bits(_ptr(b), n, bits, _ptr(out))
    return out


def encode_groups(K: np.ndarray, cb: np.ndarray):
    """K [N, G*g] (fp16 or fp32 values) , cb [G, C, g] -> (r [N,G] fp32, codes [N,G] int32)."""
    K = np.ascontiguousarray(K, dtype=np.float32)
    cb = np.ascontiguousarray(cb, dtype=np.float32)
    G, C, g = cb.shape
    N = K.shape[0]
    assert K.shape[1] == G * g
    r = np.zeros((N, G), np.float32)
    codes = np.zeros((N, G), np.int32)
    _load().orc_encode_groups(_ptr(K), N, G, g, _ptr(cb), C, _ptr(r), _ptr(codes))
    return r, codes


def radius_codes(r: np.ndarray):
    r = np.ascontiguousarray(r, dtype=np.float32)
    N, G = r.shape
    scale = np.zeros(G, np.float32)
    codes = np.zeros((N, G), np.int8)
    _load().orc_radius_codes(_ptr(r), N, G, _ptr(scale), _ptr(codes))
    return scale, codes


def build_page(r: np.ndarray, codes: np.ndarray, tier_id: int, b_theta: int) -> np.ndarray:
    r = np.ascontiguousarray(r, dtype=np.float32)
    codes = np.ascontiguousarray(codes, dtype=np.int32)
    N, G = r.shape
    out = np.zeros(int(_load().orc_page_bytes(N, G, b_theta)), np.uint8)
    n = _load().orc_build_page(_ptr(r), _ptr(codes), N, G, b_theta, tier_id, _ptr(out))
    assert n == out.size
    return out


# ------------------------------------------------------------ numpy part --
def unpack_page(pages: np.ndarray, row: np.ndarray, tier_id: int, n: int, dh: int):
    """Read one page through its pointer-table row.
    Compressed: returns (codes [n,G] int32, r_hat [n,G] fp64 = int8/127*scale).
    Dense: returns K [n, dh] fp16."""
    off, th, rad = (int(x) for x in row)
    assert pages[off] == (tier_id & 0xFF) and pages[off + 1] == (n & 0xFF)
    if tier_id == DENSE_TIER_ID:
        return np.frombuffer(pages[th:th + n * dh * 2].tobytes(), np.float16).reshape(n, dh)
    g, b = TIER_GEOMETRY[tier_id]
    G = dh // g
    scale = np.frombuffer(pages[off + 8:off + 8 + 4 * G].tobytes(), "<f4").astype(np.float64)
    codes = unpack_bits(pages[th:rad], n * G, b).reshape(n, G)
    rc = pages[rad:rad + n * G].view(np.int8).reshape(n, G).astype(np.float64)
    return codes, rc / 127.0 * scale[None, :]


@functools.lru_cache(maxsize=None)
def v_page_index(dh: int) -> np.ndarray:
    """Position of element (token k, dim d) inside a V page of the decode pool
    (dim-major: the 16 tokens of one dim are contiguous): d * 16 + k."""
    out = np.zeros((16, dh), np.int64)
    for k in range(16):
        for d in range(dh):
            out[k, d] = d * 16 + k
    return out


def v_page_rows(v_pool: np.ndarray, vs: int, n: int, dh: int) -> np.ndarray:
    """The first n V rows [n, dh] of V page vs."""
    return v_pool[vs][v_page_index(dh)][:n]


def build_pool(wl, with_codes: bool = False):
    """Encode every page of a synthetic workload on the CPU and place it as the
    plan says.  Returns dict(pages uint8, v_pool fp16 [nv, 16*dh], and, if
    with_codes, r [P, ps, Gmax] fp32 / codes [P, ps, Gmax] int32)."""
    plan = wl.plan
    dh, ps = wl.dh, plan.page_size
    pages = np.zeros(plan.pages_bytes, np.uint8)
    v_pool = np.zeros((plan.num_vpages, ps * dh), np.float16)
    vidx = v_page_index(dh)
    krows = wl.k_rows()
    vrows = wl.v_rows()
    src = wl.src_rows()
    Gmax = dh // 16
    r_all = np.zeros((plan.num_rows, ps, Gmax), np.float32)
    c_all = np.zeros((plan.num_rows, ps, Gmax), np.int32)
    for p in range(plan.num_rows):
        tid, n = int(plan.tier[p]), int(plan.count[p])
        rows = src[p, :n]
        off, th, rad = (int(x) for x in plan.ptable[p])
        v_pool[plan.vslot[p], vidx[:n]] = vrows[rows]
        if tid == DENSE_TIER_ID:
            pages[off] = tid
            pages[off + 1] = n
            pages[th:th + n * dh * 2] = np.frombuffer(krows[rows].astype(np.float16).tobytes(), np.uint8)
            continue
        g, b = TIER_GEOMETRY[tid]
        h = int(plan.seq_head[p]) % plan.num_kv
        cb = wl.codebooks[tid][h]
        r, codes = encode_groups(krows[rows].astype(np.float32), cb)
        page = build_page(r, codes, tid, b)
        pages[off:off + page.size] = page
        G = dh // g
        r_all[p, :n, :G] = r
        c_all[p, :n, :G] = codes
    out = {"pages": pages, "v_pool": v_pool}
    if with_codes:
        out["r"] = r_all
        out["codes"] = c_all
    return out


def rope_inv_freq(dh: int, theta: float) -> np.ndarray:
    j = np.arange(dh // 2, dtype=np.float64)
    return theta ** (-2.0 * j / dh)


def _rotate_half(x):
    """spherical_kv_pipeline.py:1004-1007."""
    half = x.shape[-1] // 2
    return np.concatenate([-x[..., half:], x[..., :half]], axis=-1)


def mode_b_logits(q: np.ndarray, pos: np.ndarray, cos_t: np.ndarray, sin_t: np.ndarray,
                  cw: Optional[np.ndarray], r_hat: Optional[np.ndarray],
                  K_dense: Optional[np.ndarray], G: int, g: int) -> np.ndarray:
    """Logits [nq, n] of one tier block, fp64.
    q [nq, dh]; cos_t/sin_t [n, dh] (HF layout); compressed: cw [n, G, g]
    centroids, r_hat [n, G]; dense: K_dense [n, dh]."""
    dh = q.shape[1]
    qe = q[:, None, :]
    q_rot = qe * cos_t[None] - _rotate_half(qe) * sin_t[None]          # [nq, n, dh]
    if K_dense is not None:
        return (q_rot * K_dense[None]).sum(-1) / np.sqrt(dh)
    nq, n = q_rot.shape[:2]
    q_rot_g = q_rot.reshape(nq, n, G, g)
    q_norms = np.maximum(np.linalg.norm(q_rot_g, axis=-1, keepdims=True), 1e-6)
    q_normed = q_rot_g / q_norms
    cos_pg = np.clip((q_normed * cw[None]).sum(-1), -1.0, 1.0)
    return (q_norms[..., 0] * cos_pg * r_hat[None]).sum(-1) / np.sqrt(dh)


def decode_mode_b(pool: Dict[str, np.ndarray], plan, codebooks: Dict[int, np.ndarray],
                  q: np.ndarray, gqa: int, rope_theta: float, return_lse: bool = False):
    """fp64 Mode-B decode over a placed pool.  q [num_seqs, num_kv*gqa, dh]
    (fp16 values).  Returns out [num_seqs, num_kv*gqa, dh] fp64."""
    dh, ps, num_kv = plan.dh, plan.page_size, plan.num_kv
    pages, v_pool = pool["pages"], pool["v_pool"]
    inv_freq = rope_inv_freq(dh, rope_theta)
    num_seqs = plan.num_seqs
    out = np.zeros((num_seqs, num_kv * gqa, dh), np.float64)
    lse = np.zeros((num_seqs, num_kv * gqa), np.float64)
    for sh in range(num_seqs * num_kv):
        s, h = divmod(sh, num_kv)
        qh = q[s, h * gqa:(h + 1) * gqa].astype(np.float64)
        logits, vs = [], []
        for p in range(int(plan.row_start[sh]), int(plan.row_start[sh + 1])):
            tid, n = int(plan.tier[p]), int(plan.count[p])
            pos = plan.positions[p, :n].astype(np.float64)
            ang = pos[:, None] * inv_freq[None, :]
            ang = np.concatenate([ang, ang], axis=1)
            cos_t, sin_t = np.cos(ang), np.sin(ang)
            vs.append(v_page_rows(v_pool, plan.vslot[p], n, dh).astype(np.float64))
            if tid == DENSE_TIER_ID:
                Kd = unpack_page(pages, plan.ptable[p], tid, n, dh).astype(np.float64)
                logits.append(mode_b_logits(qh, pos, cos_t, sin_t, None, None, Kd, 0, 0))
            else:
                g, _ = TIER_GEOMETRY[tid]
                G = dh // g
                codes, r_hat = unpack_page(pages, plan.ptable[p], tid, n, dh)
                cb = codebooks[tid][h].astype(np.float64)                  # [G, C, g]
                cw = cb[np.arange(G)[None, :], codes]                       # [n, G, g]
                logits.append(mode_b_logits(qh, pos, cos_t, sin_t, cw, r_hat, None, G, g))
        if not logits:
            continue
        lg = np.concatenate(logits, axis=1)
        V = np.concatenate(vs, axis=0)
        m = lg.max(axis=1, keepdims=True)
        e = np.exp(lg - m)
        ssum = e.sum(axis=1, keepdims=True)
        out[s, h * gqa:(h + 1) * gqa] = (e / ssum) @ V
        lse[s, h * gqa:(h + 1) * gqa] = (m + np.log(ssum))[:, 0]
    return (out, lse) if return_lse else out


def ragged_logits(pages, ptable, head_ids, positions, cos_tbl, sin_tbl, q, grp, codebooks,
                  dh, G, g, b_theta, page_size):
    """fused_decode_ragged contract (logits only), fp64 evaluation of the
    reference torch formula with the caller's fp32 cos/sin tables.
    Returns [grp, P*page_size]; pad slots (position < 0 or beyond the page
    count) are -inf."""
    P = ptable.shape[0]
    out = np.full((grp, P * page_size), -np.inf)
    for p in range(P):
        off = int(ptable[p, 0])
        tid, n = int(pages[off]), int(pages[off + 1])
        pos = positions[p * page_size:(p + 1) * page_size]
        valid = [i for i in range(n) if pos[i] >= 0]
        if not valid:
            continue
        codes, r_hat = unpack_page(pages, ptable[p], tid, n, dh)
        hk = int(head_ids[p])
        cb = codebooks[hk * G:(hk + 1) * G].astype(np.float64)
        cw = cb[np.arange(G)[None, :], codes]
        pv = pos[valid].astype(np.int64)
        lg = mode_b_logits(q[hk * grp:(hk + 1) * grp].astype(np.float64), pv,
                           cos_tbl[pv].astype(np.float64), sin_tbl[pv].astype(np.float64),
                           cw[valid], r_hat[valid], None, G, g)
        for j, i in enumerate(valid):
            out[:, p * page_size + i] = lg[:, j]
    return out
