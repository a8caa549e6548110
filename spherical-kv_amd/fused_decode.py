"""Drop-in replacement of the reference's fused_decode.py on MI355X.

Same module name, function names and argument order as the reference
(fused_decode.py:12-41 and the fused_decode_ragged contract inferred from its
call sites spherical_kv_pipeline.py:1102-1125, 1865-1870, 1906-1910).  Instead
of JIT-compiling a CUDA extension at import (fused_decode.py:5-10) it binds the
prebuilt libsphkv.so through its C ABI; a missing library raises at import, so
the reference's availability probe (`from fused_decode import fused_decode`,
spherical_kv_pipeline.py:1053-1086) sees the failure.

Every call launches on torch.cuda.current_stream() (the reference used the
legacy default stream) and raises RuntimeError on a non-zero status.  Outputs
the reference writes through (out, partial_scratch, the pools) must be
contiguous tensors of the reference's dtype.
"""
from __future__ import annotations

import ctypes
import math
import weakref

import torch

import sphkv_lib
from sphkv_lib import check, current_stream

_lib = sphkv_lib.load()          # raises if libsphkv.so is missing


def _stream() -> int:
    return current_stream()


def _dev(t: torch.Tensor, name: str, dtype=None) -> torch.Tensor:
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise ValueError(f"{name} must be a CUDA (HIP) tensor")
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    return t.contiguous()


ROPE_FIT_BYTES = 1024            # SPHKV_ROPE_FIT_BYTES
# Fitted RoPE tables (sphkv_rope_table_fit), one entry per (cos, sin) tensor
# pair, valid while both tensors are alive at the same storage and version
# (torch bumps a tensor's version on every in-place change through it or its
# views; a write that bypasses torch, such as a raw kernel, is not seen).
_FITS: dict = {}
_FIT_LIMIT = 16
use_rope_fit = True             # False: every call reads the tables' rows
fit_calls = 0                   # table fits run so far


class _RopeFit:
    __slots__ = ("cos", "sin", "sig", "buf", "model", "dev")


def _fit_signature(cos_src, sin_src, dh):
    return (cos_src._version, sin_src._version, cos_src.data_ptr(), sin_src.data_ptr(), tuple(cos_src.shape),
            cos_src.dtype, sin_src.dtype, cos_src.device, int(dh))


def _rope_fit(cos_src, sin_src, cos32, sin32, dh) -> _RopeFit:
    """The fit of the caller's tables, from the cache or fitted now (one
    device pass over the tables and a wait)."""
    global fit_calls
    key = (id(cos_src), id(sin_src))
    sig = _fit_signature(cos_src, sin_src, dh)
    e = _FITS.get(key)
    if e is not None and e.cos() is cos_src and e.sin() is sin_src and e.sig == sig:
        return e
    buf = torch.empty(ROPE_FIT_BYTES, dtype=torch.uint8, device=cos32.device)
    model = ctypes.c_int32(0)
    dev = (ctypes.c_float * 2)()
    rc = _lib.sphkv_rope_table_fit(cos32.data_ptr(), sin32.data_ptr(), int(cos32.shape[0]), int(dh),
                                   buf.data_ptr(), ctypes.byref(model), dev, _stream())
    check(rc, "sphkv_rope_table_fit")
    fit_calls += 1
    e = _RopeFit()
    e.cos, e.sin, e.sig, e.buf, e.model, e.dev = (weakref.ref(cos_src), weakref.ref(sin_src), sig, buf,
                                                  int(model.value), (float(dev[0]), float(dev[1])))
    for k in [k for k, v in _FITS.items() if v.cos() is None or v.sin() is None]:
        del _FITS[k]
    while len(_FITS) >= _FIT_LIMIT:
        del _FITS[next(iter(_FITS))]
    _FITS[key] = e
    return e


def rope_fit_info(cos_tbl, sin_tbl):
    """(model, deviation of the exact-angle model, deviation of the fp32-angle
    model) of the tables' fit: model 0 = the tables are read as given, 1 =
    exact angles, 2 = fp32 angles (the HF construction)."""
    c, s = _dev(cos_tbl, "cos_tbl", torch.float32), _dev(sin_tbl, "sin_tbl", torch.float32)
    e = _rope_fit(cos_tbl, sin_tbl, c, s, int(c.shape[1]))
    return e.model, e.dev[0], e.dev[1]


def fused_decode_ragged(pages, ptable, head_ids, positions, cos_tbl, sin_tbl, q, grp, num_kv,
                        codebooks, dh, groups, group_size, b_theta, page_size):
    """Logits of every (q head, page slot) of one tier's packed pages.

    pages uint8 [bytes]; ptable int32 [P, 3]; head_ids int32 [P] (kv head of
    each page); positions int32 [P * page_size] (-1 = pad); cos/sin fp32
    [max_pos, dh] (HF layout); q fp32 [num_kv * grp, dh]; codebooks fp32
    [num_kv * groups, C, group_size].
    Returns fp32 [grp, P * page_size]: row i, slot p*page_size+s is q head
    head_ids[p]*grp + i against slot s of page p, scaled by 1/sqrt(dh);
    pad slots are -inf.

    The first call with a (cos, sin) pair fits them to a RoPE rotation and
    checks every entry (sphkv_rope_table_fit); while they stay unchanged,
    later calls form the phases in the kernel from the fit (each entry is
    within 2^-20 of it) instead of reading a table row per token.  Tables
    that fit neither model are read as given.
    """
    cos_src, sin_src = cos_tbl, sin_tbl
    pages = _dev(pages, "pages", torch.uint8)
    ptable = _dev(ptable, "ptable", torch.int32)
    head_ids = _dev(head_ids, "head_ids", torch.int32)
    positions = _dev(positions, "positions", torch.int32)
    cos_tbl = _dev(cos_tbl, "cos_tbl", torch.float32)
    sin_tbl = _dev(sin_tbl, "sin_tbl", torch.float32)
    q = _dev(q, "q", torch.float32)
    codebooks = _dev(codebooks, "codebooks", torch.float32)
    P = int(ptable.shape[0])
    if ptable.dim() != 2 or ptable.shape[1] != 3:
        raise ValueError("ptable must be [P, 3]")
    if head_ids.numel() != P or positions.numel() != P * page_size:
        raise ValueError("head_ids must be [P] and positions [P * page_size]")
    if cos_tbl.shape != sin_tbl.shape or cos_tbl.dim() != 2 or cos_tbl.shape[1] != dh:
        raise ValueError("cos/sin tables must be [max_pos, dh]")
    if q.dim() != 2 or q.shape[1] != dh or q.shape[0] < num_kv * grp:
        raise ValueError("q must be [num_kv * grp, dh]")
    C = 1 << int(b_theta)
    if tuple(codebooks.shape) != (num_kv * groups, C, group_size):
        raise ValueError(f"codebooks must be [{num_kv * groups}, {C}, {group_size}]")
    out = torch.empty((int(grp), P * int(page_size)), dtype=torch.float32, device=pages.device)
    fit_ptr, model = None, 0
    if use_rope_fit and P > 0:
        fit = _rope_fit(cos_src, sin_src, cos_tbl, sin_tbl, dh)
        if fit.model:
            fit_ptr, model = fit.buf.data_ptr(), fit.model
    rc = _lib.sphkv_fused_decode_ragged_fitted(
        pages.data_ptr(), pages.numel(), ptable.data_ptr(), head_ids.data_ptr(), positions.data_ptr(), P,
        cos_tbl.data_ptr(), sin_tbl.data_ptr(), cos_tbl.shape[0], q.data_ptr(), int(grp), int(num_kv),
        codebooks.data_ptr(), int(dh), int(groups), int(group_size), int(b_theta), int(page_size),
        fit_ptr, model, out.data_ptr(), _stream())
    check(rc, "fused_decode_ragged")
    return out


def _inplace(t: torch.Tensor, name: str, dtype) -> torch.Tensor:
    """A tensor the kernel writes through: must already be a contiguous CUDA
    tensor of the right dtype (a converted copy would drop the writes)."""
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise ValueError(f"{name} must be a CUDA (HIP) tensor")
    if t.dtype != dtype or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous {dtype} tensor (written in place)")
    return t


def sphkv_decode(q_all, cb_flat, tier_G, tier_g, theta_codes, radius_codes, r_scales, v_pool,
                 block_table, bits_table, ctx_lens, out, partial_scratch,
                 num_q_heads, num_kv_heads, kv_groups, num_tiers, max_blocks, page_size, dh,
                 G_max, cb_max, g_max, sm_scale, max_ctx):
    """Mode-A decode over LayerPool tables (fused_decode.py:12-26); writes and
    returns `out` fp32 [num_q_heads, dh].

    partial_scratch fp32 [num_q_heads, max_blocks, dh + 2] receives each (q
    head, logical page)'s (m, l) in [..., 0:2] (read by the omega-EMA update,
    spherical_kv_pipeline.py:1690-1701); its other entries are scratch.
    ctx_lens and max_ctx are unused, as in the reference kernel.
    """
    q_all = _dev(q_all, "q_all", torch.float32)
    cb_flat = _dev(cb_flat, "cb_flat", torch.float32)
    tier_G = _dev(tier_G, "tier_G", torch.int32)
    tier_g = _dev(tier_g, "tier_g", torch.int32)
    theta_codes = _dev(theta_codes, "theta_codes", torch.uint8)
    radius_codes = _dev(radius_codes, "radius_codes", torch.uint8)
    r_scales = _dev(r_scales, "r_scales", torch.float32)
    v_pool = _dev(v_pool, "v_pool", torch.float16)
    block_table = _dev(block_table, "block_table", torch.int32)
    bits_table = _dev(bits_table, "bits_table", torch.int32)
    out = _inplace(out, "out", torch.float32)
    partial_scratch = _inplace(partial_scratch, "partial_scratch", torch.float32)
    nq, nkv, mb, ps = int(num_q_heads), int(num_kv_heads), int(max_blocks), int(page_size)
    n_pages = int(theta_codes.shape[0])
    if tuple(theta_codes.shape) != (n_pages, ps, int(G_max)) or theta_codes.shape != radius_codes.shape:
        raise ValueError("theta_codes / radius_codes must be [n_pages, page_size, G_max]")
    if tuple(r_scales.shape) != (n_pages, int(G_max)) or tuple(v_pool.shape) != (n_pages, ps, int(dh)):
        raise ValueError("r_scales must be [n_pages, G_max] and v_pool [n_pages, page_size, dh]")
    if block_table.numel() != nkv * mb or bits_table.numel() != nkv * mb:
        raise ValueError("block_table / bits_table must be [num_kv_heads, max_blocks]")
    if cb_flat.numel() != nkv * int(num_tiers) * int(G_max) * int(cb_max) * int(g_max):
        raise ValueError("cb_flat must be [num_kv, num_tiers, G_max, cb_max, g_max]")
    if tier_G.numel() < int(num_tiers) or tier_g.numel() < int(num_tiers):
        raise ValueError("tier_G / tier_g need num_tiers entries")
    if q_all.numel() != nq * int(dh) or out.numel() != nq * int(dh):
        raise ValueError("q_all and out must be [num_q_heads, dh]")
    if partial_scratch.numel() < nq * mb * (int(dh) + 2):
        raise ValueError("partial_scratch must be [num_q_heads, max_blocks, dh + 2]")
    rc = _lib.sphkv_decode_modea(
        q_all.data_ptr(), cb_flat.data_ptr(), tier_G.data_ptr(), tier_g.data_ptr(), theta_codes.data_ptr(),
        radius_codes.data_ptr(), r_scales.data_ptr(), v_pool.data_ptr(), n_pages, block_table.data_ptr(),
        bits_table.data_ptr(), 0, out.data_ptr(), partial_scratch.data_ptr(), nq, nkv, int(kv_groups),
        int(num_tiers), mb, ps, int(dh), int(G_max), int(cb_max), int(g_max), float(sm_scale),
        int(max_ctx), _stream())
    check(rc, "sphkv_decode")
    return out


def sphkv_encode_append(k_post, v_new, decode_cb, theta_codes, radius_codes, r_scales, v_pool,
                        pids, slot, G, g, C, G_max, dh, page_size, is_new_page):
    """Decode-time single-token encode + append (fused_decode.py:28-35): writes
    slot `slot` of pool page pids[h] for every kv head h, in place."""
    k_post = _dev(k_post, "k_post", torch.float32)
    v_new = _dev(v_new, "v_new", torch.float32)
    decode_cb = _dev(decode_cb, "decode_cb", torch.float32)
    pids = _dev(pids, "pids", torch.int64)
    theta_codes = _inplace(theta_codes, "theta_codes", torch.uint8)
    radius_codes = _inplace(radius_codes, "radius_codes", torch.uint8)
    r_scales = _inplace(r_scales, "r_scales", torch.float32)
    v_pool = _inplace(v_pool, "v_pool", torch.float16)
    num_kv = int(k_post.shape[0])
    n_pages = int(theta_codes.shape[0])
    if k_post.numel() != num_kv * int(dh) or v_new.numel() != num_kv * int(dh) or pids.numel() != num_kv:
        raise ValueError("k_post / v_new must be [num_kv, dh] and pids [num_kv]")
    if decode_cb.numel() != num_kv * int(G) * int(C) * int(g):
        raise ValueError("decode_cb must be [num_kv, G, C, g]")
    if theta_codes.numel() != n_pages * int(page_size) * int(G_max) or radius_codes.shape != theta_codes.shape:
        raise ValueError("theta_codes / radius_codes must be [n_pages, page_size, G_max]")
    if r_scales.numel() != n_pages * int(G_max) or v_pool.numel() != n_pages * int(page_size) * int(dh):
        raise ValueError("r_scales must be [n_pages, G_max] and v_pool [n_pages, page_size, dh]")
    rc = _lib.sphkv_encode_append(
        k_post.data_ptr(), v_new.data_ptr(), decode_cb.data_ptr(), theta_codes.data_ptr(),
        radius_codes.data_ptr(), r_scales.data_ptr(), v_pool.data_ptr(), pids.data_ptr(), num_kv, n_pages,
        int(slot), int(G), int(g), int(C), int(G_max), int(dh), int(page_size), 1 if is_new_page else 0,
        _stream())
    check(rc, "sphkv_encode_append")


# Backwards-compatible aliases (fused_decode.py:37-41)
def sphkv_logits(*a, **k):
    return sphkv_decode(*a, **k)


def fused_decode(*a, **k):
    return sphkv_decode(*a, **k)
