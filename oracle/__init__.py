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
                              page + pointer-table row per chunk) over the
                              chunks of oracle/paging.py's restatement of the
                              grouping (:1156-1163), placed as the plan says
* paging.py: retained_tokens, group_pages, page_offsets, build_per_head_pages,
  check_plan (spherical_kv_pipeline.py:1146-1228, allocation.py:28-37, 207-217)
  decode_mode_b               spherical_kv_pipeline.py:2143-2177 (back-rotated,
                              per-group-normalised q, clipped cosine, radius,
                              / sqrt(dh)), softmax :2347-2348, attn @ V :2364-2367;
                              rotate_half :1004-1007.  Dense fp16 K tokens use
                              textbook attention <R(-t) q, k> / sqrt(dh).
                              With a tail (oracle/tail.py) it also scores the
                              decode pages, staged tokens and the step's own
                              token (:2248-2342) in the same softmax.
  ragged_logits               the logits-only contract of fused_decode_ragged
                              (call sites spherical_kv_pipeline.py:1102-1125,
                              1865-1870) evaluated with the caller's cos/sin
                              tables.
* Mode-A (LayerPool) path:
  encode_append (C)           decode_kernel.cu:10-84, nvcc's FP contraction
                              written out (bit-exact target)
  decode_mode_a               decode_kernel.cu:108-246 in fp64: per (q head,
                              page) logits sum_g r_hat_g <q_g, c> * sm_scale
                              (-1e9 where the sum is 0, :183), page (m, l, acc),
                              merge out = acc / (l + 1e-8) (:244)
  q_lut, lut_logits           the per-query table and the logits of
                              new_fused_decode.py:22-43 (fp64)

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
        lib.orc_encode_append.argtypes = [P, P, P, P, P, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
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
    plan says.  The pages' token sets come from the oracle's own restatement
    of the reference grouping (oracle/paging.py: retained tokens -> groups by
    (seq, head, tier) -> sorted chunks); the plan's rows are first checked to
    be exactly those chunks (paging.check_plan), so only the placement (byte
    offsets, V slots) is taken from the plan.  Returns dict(pages uint8,
    v_pool fp16 [nv, 16*dh], and, if with_codes, r [P, ps, Gmax] fp32 /
    codes [P, ps, Gmax] int32)."""
    from oracle import paging
    plan = wl.plan
    dh, ps = wl.dh, plan.page_size
    groups = paging.group_pages(paging.retained_tokens(wl.tier_of, plan.num_seqs, plan.num_kv), ps)
    paging.check_plan(plan, groups, positions_of=getattr(wl, "positions", None))
    pages = np.zeros(plan.pages_bytes, np.uint8)
    v_pool = np.zeros((plan.num_vpages, ps * dh), np.float16)
    vidx = v_page_index(dh)
    krows = wl.k_rows()
    vrows = wl.v_rows()
    base = wl.row_base()
    Gmax = dh // 16
    r_all = np.zeros((plan.num_rows, ps, Gmax), np.float32)
    c_all = np.zeros((plan.num_rows, ps, Gmax), np.int32)
    for sh in range(plan.num_seqs * plan.num_kv):
        s, h = divmod(sh, plan.num_kv)
        p = int(plan.row_start[sh])
        for tid, chunks in groups.get((s, h), []):
            for chunk in chunks:
                n = len(chunk)
                rows = base[sh] + np.asarray(chunk, np.int64)
                off, th, rad = (int(x) for x in plan.ptable[p])
                v_pool[plan.vslot[p], vidx[:n]] = vrows[rows]
                if tid == DENSE_TIER_ID:
                    pages[off] = tid
                    pages[off + 1] = n
                    pages[th:th + n * dh * 2] = np.frombuffer(krows[rows].astype(np.float16).tobytes(), np.uint8)
                else:
                    g, b = TIER_GEOMETRY[tid]
                    r, codes = encode_groups(krows[rows].astype(np.float32), wl.codebooks[tid][h])
                    page = build_page(r, codes, tid, b)
                    pages[off:off + page.size] = page
                    G = dh // g
                    r_all[p, :n, :G] = r
                    c_all[p, :n, :G] = codes
                p += 1
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
                  q: np.ndarray, gqa: int, rope_theta: float, return_lse: bool = False,
                  tail=None, k_new=None, v_new=None, cur_pos=None, r_exact: Optional[np.ndarray] = None):
    """fp64 Mode-B decode over a placed pool.  q [num_seqs, num_kv*gqa, dh]
    (fp16 values).  Returns out [num_seqs, num_kv*gqa, dh] fp64.

    Compressed pages are scored on the page-decoded radius r_hat = code / 127
    * r_scale (the parity definition).  r_exact [P, ps, Gmax] (build_pool's
    "r": the encoder's fp32 radii) scores them on the unquantised radii
    instead, as the reference's torch path does (K_tier's fp32 radii,
    spherical_kv_pipeline.py:2137, 2175-2176): the gap between the two is the
    format's error, not a kernel's.

    tail (oracle.tail.TailOracle): adds each (seq, head)'s decode pages and
    staged tokens, and with k_new / v_new [num_seqs, num_kv, dh], cur_pos
    [num_seqs] the step's own token, to the same softmax (a full decode step
    of _compressed_head_attention_batched, spherical_kv_pipeline.py:2057-2369)."""
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
                if r_exact is not None:
                    r_hat = r_exact[p, :n, :G].astype(np.float64)
                cb = codebooks[tid][h].astype(np.float64)                  # [G, C, g]
                cw = cb[np.arange(G)[None, :], codes]                       # [n, G, g]
                logits.append(mode_b_logits(qh, pos, cos_t, sin_t, cw, r_hat, None, G, g))
        if tail is not None:
            step = (k_new[s, h], v_new[s, h], cur_pos[s]) if k_new is not None else (None, None, None)
            lt, vt = tail.terms(s, h, qh, inv_freq, *step)
            if lt.shape[1]:
                logits.append(lt)
                vs.append(vt)
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


# ------------------------------------------------------------- Mode A --
def encode_append(k_post: np.ndarray, v_new: np.ndarray, decode_cb: np.ndarray, theta: np.ndarray,
                  radius: np.ndarray, r_scales: np.ndarray, v_pool: np.ndarray, pids: np.ndarray,
                  slot: int, is_new_page: bool) -> None:
    """decode_kernel.cu:10-84 on numpy pools, in place.  k_post / v_new fp32
    [num_kv, dh]; decode_cb fp32 [num_kv, G, C, g]; theta / radius uint8
    [n_pages, page_size, G_max]; r_scales fp32 [n_pages, G_max]; v_pool fp16
    [n_pages, page_size, dh]; pids int64 [num_kv]."""
    lib = _load()
    num_kv, dh = k_post.shape
    _, G, C, g = decode_cb.shape
    n_pages, page_size, G_max = theta.shape
    for a in (theta, radius, r_scales, v_pool):
        assert a.flags.c_contiguous
    for h in range(num_kv):
        pid = int(pids[h])
        if pid < 0 or pid >= n_pages:
            continue
        v_pool[pid, slot] = v_new[h].astype(np.float16)
        k = np.ascontiguousarray(k_post[h], np.float32)
        cb = np.ascontiguousarray(decode_cb[h], np.float32)
        lib.orc_encode_append(_ptr(k), _ptr(cb), _ptr(theta), _ptr(radius), _ptr(r_scales), pid, int(slot), G, g, C,
                              G_max, page_size, 1 if is_new_page else 0)


def q_lut(q_all: np.ndarray, cb_flat: np.ndarray, tier_G, tier_g, kv_groups: int) -> np.ndarray:
    """[num_q, num_tiers, G_max, cb_max] fp64: <q_g, centroid> per tier, group, code."""
    num_q, dh = q_all.shape
    _, T, G_max, cb_max, g_max = cb_flat.shape
    out = np.zeros((num_q, T, G_max, cb_max))
    for hq in range(num_q):
        hkv = hq // kv_groups
        for t in range(T):
            Gt, gt = int(tier_G[t]), int(tier_g[t])
            for gi in range(Gt):
                qg = q_all[hq, gi * gt:(gi + 1) * gt].astype(np.float64)
                out[hq, t, gi] = cb_flat[hkv, t, gi, :, :gt].astype(np.float64) @ qg
    return out


def decode_mode_a(q_all, cb_flat, tier_G, tier_g, theta, radius, r_scales, v_pool, block_table, bits_table,
                  kv_groups: int, sm_scale: float):
    """decode_kernel.cu:108-246 in fp64.  Returns (out [num_q, dh], m [num_q,
    max_blocks], l [num_q, max_blocks]) with m = -inf, l = 0 for absent pages."""
    num_q, dh = q_all.shape
    num_kv, max_blocks = block_table.shape
    page_size = theta.shape[1]
    lut = q_lut(q_all, cb_flat, tier_G, tier_g, kv_groups)
    out = np.zeros((num_q, dh))
    M = np.full((num_q, max_blocks), -np.inf)
    Lp = np.zeros((num_q, max_blocks))
    for hq in range(num_q):
        hkv = hq // kv_groups
        accs, ms, ls = [], [], []
        for p in range(max_blocks):
            phys, t = int(block_table[hkv, p]), int(bits_table[hkv, p])
            if phys < 0 or phys >= theta.shape[0] or t < 0 or t >= cb_flat.shape[1]:
                continue
            Gt = int(tier_G[t])
            rh = r_scales[phys, :Gt].astype(np.float64)[None, :] * radius[phys, :, :Gt].astype(np.float64) / 255.0
            vals = lut[hq, t, np.arange(Gt)[None, :], theta[phys, :, :Gt].astype(np.int64)]
            s = (rh * vals).sum(axis=1)
            lg = np.where(s == 0.0, -1e9, s * sm_scale)
            m = lg.max()
            e = np.exp(lg - m)
            M[hq, p], Lp[hq, p] = m, e.sum()
            ms.append(m)
            ls.append(e.sum())
            accs.append(e @ v_pool[phys].astype(np.float64))
        if ms:
            Mx = max(ms)
            f = np.exp(np.array(ms) - Mx)
            out[hq] = (f[:, None] * np.array(accs)).sum(0) / ((f * np.array(ls)).sum() + 1e-8)
    return out, M, Lp


def lut_logits(lut, theta, radius, r_scales, block_table, bits_table, ctx_lens, kv_groups: int,
               sm_scale: float, max_ctx: int) -> np.ndarray:
    """new_fused_decode.py:22-43 contract in fp64: [num_q, max_ctx]."""
    num_q, T, G_max, cb_max = lut.shape
    num_kv, max_blocks = block_table.shape
    page_size = theta.shape[1]
    out = np.full((num_q, max_ctx), -np.inf)
    for hq in range(num_q):
        hkv = hq // kv_groups
        for n in range(min(max_ctx, int(ctx_lens[hkv]))):
            lb, s = divmod(n, page_size)
            if lb >= max_blocks:
                break
            phys, t = int(block_table[hkv, lb]), int(bits_table[hkv, lb])
            if phys < 0 or phys >= theta.shape[0] or t < 0 or t >= T:
                continue
            rh = r_scales[phys].astype(np.float64) * radius[phys, s].astype(np.float64) / 255.0
            codes = theta[phys, s].astype(np.int64)
            vals = np.where(codes < cb_max, lut[hq, t, np.arange(G_max), np.minimum(codes, cb_max - 1)], 0.0)
            out[hq, n] = (rh * vals).sum() * sm_scale
    return out


def omega_ema(m_q, l_q, omega_prev, num_kv: int, kv_groups: int, ema_beta: float) -> np.ndarray:
    """spherical_kv_pipeline.py:952-987 (_omega_ema_eager) in fp64: m_q, l_q
    [num_q, max_blocks]; omega_prev [num_kv, max_blocks]."""
    m = np.asarray(m_q, np.float64)
    l = np.asarray(l_q, np.float64)
    valid = l > 0
    m_safe = np.where(valid, m, -1e30)
    m_max = m_safe.max(axis=1, keepdims=True)
    w = np.exp(np.maximum(m_safe - m_max, -60.0)) * l
    z = np.maximum(w.sum(axis=1, keepdims=True), 1e-12)
    mass_kv = (w / z).reshape(num_kv, kv_groups, -1).mean(axis=1)
    return np.asarray(omega_prev, np.float64) * ema_beta + mass_kv * (1.0 - ema_beta)


def layer_pool_page(r_chunk: np.ndarray, theta_chunk: np.ndarray):
    """One LayerPool page's quantisation (sphkv_lut.py:56-61) in the
    reference's fp32 arithmetic: r_scale = max(max_n r, 1e-8); radius code =
    clamp(round_half_even(r / r_scale * 255), 0, 255); theta code = low byte.
    Returns (theta uint8 [npg, G_t], radius uint8 [npg, G_t], r_scale fp32 [G_t])."""
    r = np.asarray(r_chunk, np.float32)
    rscl = np.maximum(r.max(axis=0), np.float32(1e-8))
    q = np.rint((r / rscl) * np.float32(255.0))
    rad = np.clip(q, 0, 255).astype(np.uint8)
    th = (np.asarray(theta_chunk).astype(np.int64) & 0xFF).astype(np.uint8)
    return th, rad, rscl.astype(np.float32)


def layer_pool(per_head: dict, num_kv: int, page_size: int, G_max: int, dh: int, decode_capacity: int,
               tier_of_btheta: dict):
    """LayerPool.__init__ pools and tables (sphkv_lut.py:36-98) in numpy.
    per_head[h] = list of (b_theta, n_tokens, V fp16 [n, dh], r fp32 [n, G_t],
    theta int [n, G_t]); tier_of_btheta[b_theta] = (tier index, G_t).
    Returns dict(theta, radius, r_scales, v_pool, block_table, bits_table,
    ctx_lens, max_blocks, num_pages_used)."""
    pages, head_blocks, ctx = [], {h: [] for h in range(num_kv)}, [0] * num_kv
    for h in range(num_kv):
        for b_theta, n_tokens, V, r, th in per_head.get(h, []):
            t_idx, G_t = tier_of_btheta[b_theta]
            for pg in range(-(-n_tokens // page_size)):
                s, e = pg * page_size, min((pg + 1) * page_size, n_tokens)
                tpg, rpg, spg = layer_pool_page(r[s:e], th[s:e])
                head_blocks[h].append((len(pages), t_idx))
                pages.append((G_t, e - s, tpg, rpg, spg, np.asarray(V[s:e], np.float16)))
        ctx[h] = len(head_blocks[h]) * page_size
    n_used = len(pages)
    n_total = n_used + decode_capacity
    max_blk = max((len(v) for v in head_blocks.values()), default=0) + decode_capacity // max(num_kv, 1) + 2
    theta = np.zeros((n_total, page_size, G_max), np.uint8)
    radius = np.zeros_like(theta)
    r_scales = np.zeros((n_total, G_max), np.float32)
    v_pool = np.zeros((n_total, page_size, dh), np.float16)
    for pid, (G_t, n, tpg, rpg, spg, v) in enumerate(pages):
        theta[pid, :n, :G_t] = tpg
        radius[pid, :n, :G_t] = rpg
        r_scales[pid, :G_t] = spg
        v_pool[pid, :n] = v
    bt = np.full((num_kv, max_blk), -1, np.int32)
    bits = np.zeros((num_kv, max_blk), np.int32)
    for h, bl in head_blocks.items():
        for lb, (pid, ti) in enumerate(bl):
            bt[h, lb], bits[h, lb] = pid, ti
    return dict(theta=theta, radius=radius, r_scales=r_scales, v_pool=v_pool, block_table=bt, bits_table=bits,
                ctx_lens=np.asarray(ctx, np.int32), max_blocks=max_blk, num_pages_used=n_used)
