"""Op-for-op torch restatements of the reference's Mode-B decode and of its
prefill encode / page build, for the CPU baselines of bench.py.  TEST /
MEASUREMENT INFRASTRUCTURE (never shipped).

Encode (encode_chunk, build_page, pack_bits): spherical_kv_pipeline.py:1136-1144
(view, norm, divide by r + EPS, einsum with the codebook, argmax),
pagebuilder.py:17-33 (r_scale, int8 radii, header, concatenation) and
bitpacking.py:5-29 (LSB-first scatter_add packing), called per page chunk as
_build_per_head_pages does (spherical_kv_pipeline.py:1187-1213).

Decode:

Follows spherical_kv_pipeline.py:2100-2179 per (kv head, tier block):
back-rotate q per token with cos/sin tables (:2143-2151, _rotate_half
:1004-1007), per-group normalise (:2158-2160), gather centroids (:2163-2167),
clipped cosine (:2170), sum_g ||q_g|| r_g cos / sqrt(dh) (:2175-2176), then
softmax over all tokens (:2348) and attn @ V (:2367).  Executed per kv head
like the reference (one _compressed_head_attention_batched call per head).
Dense fp16 K blocks use the textbook logit <q_rot, k> / sqrt(dh).
"""
from __future__ import annotations

import math
from typing import Dict, List

import numpy as np
import torch

import oracle


EPS = 1e-8                       # spherical_kv_pipeline.py EPS
HEADER_BYTES = 8                 # config.py:3


def encode_chunk(K_chunk: torch.Tensor, codebooks: torch.Tensor, g: int, G: int):
    """K_chunk fp32 [N, dh], codebooks [G, C, g] -> (r [N, G], codes int32 [N, G])."""
    N = K_chunk.shape[0]
    K_grouped = K_chunk.view(N, G, g)
    r_groups = K_grouped.norm(dim=-1)
    K_dir = K_grouped / (r_groups.unsqueeze(-1) + EPS)
    sims = torch.einsum('ngi,gci->ngc', K_dir, codebooks)
    return r_groups, sims.argmax(dim=-1).to(torch.int32)


def pack_bits(values: torch.Tensor, bits: int) -> torch.Tensor:
    """values int32 [n] -> uint8 [ceil(n*bits/8)], value i's bit k at global bit i*bits + k."""
    n = values.numel()
    out = torch.zeros((n * bits + 7) // 8, dtype=torch.uint8)
    bit_idx = torch.arange(bits)
    bit_matrix = ((values.unsqueeze(1) >> bit_idx) & 1).bool()
    global_bits = torch.arange(n).unsqueeze(1) * bits + bit_idx
    byte_idx = (global_bits >> 3).long().reshape(-1)
    bit_shift = (global_bits & 7).long().reshape(-1)
    contrib = bit_matrix.reshape(-1).to(torch.uint8) << bit_shift.to(torch.uint8)
    out.scatter_add_(0, byte_idx, contrib)
    return out


def build_page(r: torch.Tensor, codes: torch.Tensor, tier_id: int, b_theta: int) -> torch.Tensor:
    """One page's bytes: header (tier id, N, pad, fp32 r_scale[G]), packed codes, int8 radii."""
    N, G = r.shape
    r_scale = r.abs().max(dim=0).values
    safe = r_scale.clamp(min=1e-8).unsqueeze(0)
    rc = (r / safe * 127).round().clamp(-127, 127).to(torch.int8)
    packed = pack_bits(codes.flatten().to(torch.int32), b_theta)
    hdr = torch.zeros(HEADER_BYTES + 4 * G, dtype=torch.uint8)
    hdr[0] = tier_id & 0xFF
    hdr[1] = N & 0xFF
    hdr[HEADER_BYTES:] = r_scale.to(torch.float32).view(torch.uint8)
    return torch.cat([hdr, packed, rc.flatten().view(torch.uint8)])


def _rotate_half(x):
    half = x.shape[-1] // 2
    return torch.cat([-x[..., half:], x[..., :half]], dim=-1)


def head_blocks(pages: np.ndarray, v_pool: np.ndarray, plan, sh: int) -> List[dict]:
    """Per-tier token blocks of one (seq, kv head), as the reference keeps them
    in per_head_pages: (r_hat, codes, positions, V) or dense K."""
    dh = plan.dh
    by_tier: Dict[int, dict] = {}
    for p in range(int(plan.row_start[sh]), int(plan.row_start[sh + 1])):
        tid, n = int(plan.tier[p]), int(plan.count[p])
        d = by_tier.setdefault(tid, {"tier": tid, "r": [], "codes": [], "k": [], "pos": [], "v": []})
        if tid == oracle.DENSE_TIER_ID:
            d["k"].append(oracle.unpack_page(pages, plan.ptable[p], tid, n, dh).astype(np.float32))
        else:
            codes, r_hat = oracle.unpack_page(pages, plan.ptable[p], tid, n, dh)
            d["codes"].append(codes)
            d["r"].append(r_hat.astype(np.float32))
        d["pos"].append(plan.positions[p, :n].astype(np.int64))
        d["v"].append(oracle.v_page_rows(v_pool, plan.vslot[p], n, dh))
    out = []
    for tid, d in by_tier.items():
        blk = {"tier": tid, "pos": torch.from_numpy(np.concatenate(d["pos"])),
               "v": torch.from_numpy(np.ascontiguousarray(np.concatenate(d["v"])))}
        if tid == oracle.DENSE_TIER_ID:
            blk["k"] = torch.from_numpy(np.concatenate(d["k"]))
        else:
            blk["r"] = torch.from_numpy(np.concatenate(d["r"]))
            blk["codes"] = torch.from_numpy(np.concatenate(d["codes"]).astype(np.int64))
        out.append(blk)
    return out


def decode_head(q: torch.Tensor, blocks: List[dict], codebooks: Dict[int, torch.Tensor],
                cos_tbl: torch.Tensor, sin_tbl: torch.Tensor) -> torch.Tensor:
    """One kv head: q fp32 [num_q, dh] -> out fp32 [num_q, dh]."""
    num_q, dh = q.shape
    parts, vs = [], []
    for blk in blocks:
        positions = blk["pos"]
        n_tokens = positions.shape[0]
        cos_i = cos_tbl[positions]
        sin_i = sin_tbl[positions]
        q_expanded = q.unsqueeze(1)
        q_half = _rotate_half(q_expanded)
        q_rot = q_expanded * cos_i.unsqueeze(0) - q_half * sin_i.unsqueeze(0)
        if blk["tier"] == oracle.DENSE_TIER_ID:
            logits = (q_rot * blk["k"].unsqueeze(0)).sum(-1) / math.sqrt(dh)
        else:
            cb = codebooks[blk["tier"]]
            G, C, g = cb.shape
            q_rot_g = q_rot.view(num_q, n_tokens, G, g)
            q_norms = q_rot_g.norm(dim=-1, keepdim=True).clamp(min=1e-6)
            q_normed = q_rot_g / q_norms
            cw = cb[torch.arange(G).unsqueeze(1), blk["codes"].T]
            cw_t = cw.permute(1, 0, 2)
            cos_pg = (q_normed * cw_t.unsqueeze(0)).sum(-1).clamp(-1.0, 1.0)
            logits = (q_norms.squeeze(-1) * cos_pg * blk["r"].unsqueeze(0)).sum(-1) / math.sqrt(dh)
        parts.append(logits)
        vs.append(blk["v"])
    all_logits = torch.cat(parts, dim=1)
    attn = torch.softmax(all_logits, dim=1)
    V_full = torch.cat(vs, dim=0).float()
    return attn @ V_full
