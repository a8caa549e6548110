"""Op-for-op torch restatement of the reference's Mode-B decode, for the CPU
baseline of bench.py.  TEST / MEASUREMENT INFRASTRUCTURE (never shipped).

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
