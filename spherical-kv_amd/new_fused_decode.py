"""Drop-in replacement of the reference's new_fused_decode.py on MI355X.

sphkv_logits keeps the reference's name and argument order
(new_fused_decode.py:22-43): logits of every (q head, context slot) from a
per-query q.centroid table over the Mode-A LayerPool tables; the softmax and
the V product stay with the caller, as the reference's docstring describes.
The reference never builds the table itself; build_q_lut does (same layout).
The library is the prebuilt libsphkv.so (a missing library raises at import).
"""
from __future__ import annotations

import torch

import sphkv_lib
from sphkv_lib import check, current_stream

_lib = sphkv_lib.load()          # raises if libsphkv.so is missing


def _stream() -> int:
    return current_stream()


def _dev(t, name, dtype):
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise ValueError(f"{name} must be a CUDA (HIP) tensor")
    if t.dtype is dtype and t.is_contiguous():      # the usual case: no dispatcher call
        return t
    return t.to(dtype).contiguous()


def build_q_lut(q_all, cb_flat, tier_G, tier_g, num_kv_heads, kv_groups, num_tiers, G_max, cb_max, g_max):
    """q_lut fp32 [num_q, num_tiers, G_max, cb_max]: q_lut[hq, t, g, c] =
    <q[hq, g*tier_g[t] : (g+1)*tier_g[t]], cb_flat[hq // kv_groups, t, g, c, :tier_g[t]]>
    for g < tier_G[t], 0 elsewhere."""
    q_all = _dev(q_all, "q_all", torch.float32)
    cb_flat = _dev(cb_flat, "cb_flat", torch.float32)
    tier_G = _dev(tier_G, "tier_G", torch.int32)
    tier_g = _dev(tier_g, "tier_g", torch.int32)
    nq, dh = int(q_all.shape[0]), int(q_all.shape[1])
    lut = torch.empty((nq, int(num_tiers), int(G_max), int(cb_max)), dtype=torch.float32, device=q_all.device)
    rc = _lib.sphkv_q_lut(q_all.data_ptr(), cb_flat.data_ptr(), tier_G.data_ptr(), tier_g.data_ptr(), nq,
                          int(num_kv_heads), int(kv_groups), int(num_tiers), dh, int(G_max), int(cb_max),
                          int(g_max), lut.data_ptr(), _stream())
    check(rc, "build_q_lut")
    return lut


def sphkv_logits(q_lut, theta_codes, radius_codes, r_scales, block_table, bits_table, ctx_lens, logits_out,
                 num_q_heads, num_kv_heads, kv_groups, num_tiers, max_blocks, page_size, G_max, cb_size_max,
                 sm_scale, max_ctx):
    """Writes and returns logits_out fp32 [num_q_heads, max_ctx]: token n of kv
    head hq // kv_groups (slot n % page_size of logical page n // page_size)
    scores sm_scale * sum_g r_hat_g * q_lut[hq, tier, g, code_g], r_hat =
    r_scale * code / 255; -inf beyond ctx_lens or for an absent page."""
    q_lut = _dev(q_lut, "q_lut", torch.float32)
    theta_codes = _dev(theta_codes, "theta_codes", torch.uint8)
    radius_codes = _dev(radius_codes, "radius_codes", torch.uint8)
    r_scales = _dev(r_scales, "r_scales", torch.float32)
    block_table = _dev(block_table, "block_table", torch.int32)
    bits_table = _dev(bits_table, "bits_table", torch.int32)
    ctx_lens = _dev(ctx_lens, "ctx_lens", torch.int32)
    if not isinstance(logits_out, torch.Tensor) or not logits_out.is_cuda or logits_out.dtype != torch.float32 \
            or not logits_out.is_contiguous():
        raise ValueError("logits_out must be a contiguous fp32 CUDA tensor (written in place)")
    nq, mc = int(num_q_heads), int(max_ctx)
    if logits_out.numel() < nq * mc:
        raise ValueError("logits_out must hold [num_q_heads, max_ctx]")
    if q_lut.numel() != nq * int(num_tiers) * int(G_max) * int(cb_size_max):
        raise ValueError("q_lut must be [num_q_heads, num_tiers, G_max, cb_size_max]")
    n_pages = int(theta_codes.shape[0])
    if theta_codes.numel() != n_pages * int(page_size) * int(G_max) or radius_codes.shape != theta_codes.shape:
        raise ValueError("theta_codes / radius_codes must be [n_pages, page_size, G_max]")
    if block_table.numel() != int(num_kv_heads) * int(max_blocks) or bits_table.numel() != block_table.numel():
        raise ValueError("block_table / bits_table must be [num_kv_heads, max_blocks]")
    if ctx_lens.numel() < int(num_kv_heads):
        raise ValueError("ctx_lens must be [num_kv_heads]")
    rc = _lib.sphkv_logits_lut(q_lut.data_ptr(), theta_codes.data_ptr(), radius_codes.data_ptr(),
                               r_scales.data_ptr(), n_pages, block_table.data_ptr(), bits_table.data_ptr(),
                               ctx_lens.data_ptr(), logits_out.data_ptr(), nq, int(num_kv_heads),
                               int(kv_groups), int(num_tiers), int(max_blocks), int(page_size), int(G_max),
                               int(cb_size_max), float(sm_scale), mc, _stream())
    check(rc, "sphkv_logits")
    return logits_out


# Keep the reference's alias (new_fused_decode.py:46-48)
def fused_decode(*args, **kwargs):
    return sphkv_logits(*args, **kwargs)
