"""Drop-in replacement of the reference's fused_decode.py on MI355X.

Same module name, function names and argument order as the reference
(fused_decode.py:12-41 and the fused_decode_ragged contract inferred from its
call sites spherical_kv_pipeline.py:1102-1125, 1865-1870, 1906-1910).  Instead
of JIT-compiling a CUDA extension at import (fused_decode.py:5-10) it binds the
prebuilt libsphkv.so through its C ABI; a missing library raises at import, so
the reference's availability probe (`from fused_decode import fused_decode`,
spherical_kv_pipeline.py:1053-1086) sees the failure.

Every call launches on torch.cuda.current_stream() (the reference used the
legacy default stream) and raises RuntimeError on a non-zero status.
"""
from __future__ import annotations

import math

import torch

import sphkv_lib
from sphkv_lib import check

_lib = sphkv_lib.load()          # raises if libsphkv.so is missing


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _dev(t: torch.Tensor, name: str, dtype=None) -> torch.Tensor:
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise ValueError(f"{name} must be a CUDA (HIP) tensor")
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    return t.contiguous()


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
    """
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
    rc = _lib.sphkv_fused_decode_ragged(
        pages.data_ptr(), pages.numel(), ptable.data_ptr(), head_ids.data_ptr(), positions.data_ptr(), P,
        cos_tbl.data_ptr(), sin_tbl.data_ptr(), cos_tbl.shape[0], q.data_ptr(), int(grp), int(num_kv),
        codebooks.data_ptr(), int(dh), int(groups), int(group_size), int(b_theta), int(page_size),
        out.data_ptr(), _stream())
    check(rc, "fused_decode_ragged")
    return out


def sphkv_decode(q_all, cb_flat, tier_G, tier_g, theta_codes, radius_codes, r_scales, v_pool,
                 block_table, bits_table, ctx_lens, out, partial_scratch,
                 num_q_heads, num_kv_heads, kv_groups, num_tiers, max_blocks, page_size, dh,
                 G_max, cb_max, g_max, sm_scale, max_ctx):
    """Mode-A decode over LayerPool tables (fused_decode.py:12-26)."""
    raise NotImplementedError("sphkv_decode (Mode-A LayerPool decode) is not built yet")


def sphkv_encode_append(k_post, v_new, decode_cb, theta_codes, radius_codes, r_scales, v_pool,
                        pids, slot, G, g, C, G_max, dh, page_size, is_new_page):
    """Decode-time single-token encode + append (fused_decode.py:28-35)."""
    raise NotImplementedError("sphkv_encode_append is not built yet")


# Backwards-compatible aliases (fused_decode.py:37-41)
def sphkv_logits(*a, **k):
    return sphkv_decode(*a, **k)


def fused_decode(*a, **k):
    return sphkv_decode(*a, **k)
