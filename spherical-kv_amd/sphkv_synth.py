"""Seeded synthetic workloads for the five benchmark configurations.

numpy PCG64 (default_rng(seed)), deterministic across hosts.  Draw order:
codebooks -> K scale -> K -> tiers -> V -> q -> page permutation.

* Codebook rows: normalize(N(0,1)) in fp64, stored fp32, one codebook per
  (kv head, tier, group), [G, C, g] (the shape codebook_loader.py:7-59 returns,
  rows unit-normalised as at codebook_loader.py:43-44).
* K is pre-RoPE fp16; V and q are fp16 N(0,1).
* Tiers are drawn per (kv head, token), as the reference decides them per
  (layer, head, token) TokenState.
* Positions are token indices (each sequence uses its own 0..L-1).
* RoPE: default (no scaling), theta = 500000, HF rotate_half pairing.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional

import numpy as np

import sphkv_format as fmt


@dataclass
class Workload:
    name: str
    dh: int
    num_kv: int
    gqa: int
    num_seqs: int
    lengths: List[int]              # tokens per sequence
    rope_theta: float
    codebooks: Dict[int, np.ndarray]  # tier id -> [num_kv, G, C, g] fp32
    K: List[np.ndarray]             # per seq: [num_kv, L, dh] fp16 (pre-RoPE)
    V: List[np.ndarray]             # per seq: [num_kv, L, dh] fp16
    q: np.ndarray                   # [num_seqs, num_kv*gqa, dh] fp16
    tier_of: List[np.ndarray]       # per (seq*num_kv + head): [L] tier ids
    plan: fmt.PagePlan
    page_size: int = 16

    @property
    def num_q(self) -> int:
        return self.num_kv * self.gqa

    def k_rows(self) -> np.ndarray:
        """K of all sequences as one [rows, dh] fp16 matrix; row of
        (seq s, head h, token t) = row_base[s*num_kv+h] + t."""
        return np.concatenate([k.reshape(-1, self.dh) for k in self.K], axis=0)

    def v_rows(self) -> np.ndarray:
        return np.concatenate([v.reshape(-1, self.dh) for v in self.V], axis=0)

    def row_base(self) -> np.ndarray:
        base, acc = [], 0
        for s, L in enumerate(self.lengths):
            for h in range(self.num_kv):
                base.append(acc + h * L)
            acc += self.num_kv * L
        return np.asarray(base, np.int64)

    def src_rows(self) -> np.ndarray:
        """[P, page_size] int64 row of each page slot in k_rows() (-1 pad)."""
        base = self.row_base()
        tk = self.plan.tokens
        out = np.where(tk >= 0, tk + base[self.plan.seq_head][:, None], -1)
        return out.astype(np.int64)


def make_codebooks(rng, num_kv: int, dh: int, tier_ids) -> Dict[int, np.ndarray]:
    cbs = {}
    for tid in tier_ids:
        g, b = fmt.TIER_GEOMETRY[tid]
        G, C = dh // g, 2 ** b
        x = rng.standard_normal((num_kv, G, C, g))
        x /= np.linalg.norm(x, axis=-1, keepdims=True)
        cbs[tid] = x.astype(np.float32)
    return cbs


def _assign_tiers(rng, L: int, fracs, sink: int = 0, recent: int = 0) -> np.ndarray:
    """fracs: list of (tier_id, prob).  First `sink` and last `recent` tokens
    are forced dense."""
    ids = np.array([t for t, _ in fracs], np.int32)
    p = np.array([f for _, f in fracs], np.float64)
    t = ids[rng.choice(len(ids), size=L, p=p / p.sum())]
    D = fmt.DENSE_TIER_ID
    if sink:
        t[:sink] = D
    if recent:
        t[max(0, L - recent):] = D
    return t


def make_decode_workload(config: int, seed: Optional[int] = None, ctx_override: Optional[int] = None,
                         num_seqs_override: Optional[int] = None, layout: str = "default") -> Workload:
    """Decode configs 1, 2, 4, 5.  ctx_override shrinks
    the context (for oracle-sized parity cases) keeping everything else."""
    D = fmt.DENSE_TIER_ID
    if config == 1:
        dh, num_kv, gqa, num_seqs, theta = 64, 8, 4, 1, 500000.0
        lengths = [ctx_override or 4096]
        fracs, sink, recent, kscale, seed_d = [(1, 1.0)], 0, 0, False, 1
    elif config == 2:
        dh, num_kv, gqa, num_seqs, theta = 128, 8, 4, 1, 500000.0
        lengths = [ctx_override or 32768]
        fracs, sink, recent, kscale, seed_d = [(1, .6), (2, .3), (D, .1)], 64, 256, True, 2
    elif config == 4:
        dh, num_kv, gqa, theta = 128, 8, 4, 500000.0
        num_seqs = num_seqs_override or 64
        fracs, sink, recent, kscale, seed_d = [(1, .5), (2, .4), (D, .1)], 0, 0, True, 4
        lengths = None
    elif config == 5:
        dh, num_kv, gqa, theta = 128, 8, 8, 500000.0
        num_seqs = num_seqs_override or 4
        lengths = [ctx_override or 131072] * num_seqs
        fracs, sink, recent, kscale, seed_d = [(1, .4), (2, .55), (D, .05)], 0, 0, True, 5
    else:
        raise ValueError(f"no decode config {config}")
    rng = np.random.default_rng(seed_d if seed is None else seed)
    tier_ids = sorted({t for t, _ in fracs if t != D})
    cbs = make_codebooks(rng, num_kv, dh, tier_ids)
    if lengths is None:
        hi = ctx_override or 32768
        lo = min(2048, hi)
        lengths = [int(x) for x in rng.integers(lo, hi + 1, size=num_seqs)]
    scale = (np.exp(rng.normal(0.0, 0.5, size=(num_kv, dh))) if kscale
             else np.ones((num_kv, dh)))
    K = [(rng.standard_normal((num_kv, L, dh)) * scale[:, None, :]).astype(np.float16) for L in lengths]
    tier_of = []
    for L in lengths:
        for h in range(num_kv):
            tier_of.append(_assign_tiers(rng, L, fracs, sink, recent))
    V = [rng.standard_normal((num_kv, L, dh)).astype(np.float16) for L in lengths]
    q = rng.standard_normal((num_seqs, num_kv * gqa, dh)).astype(np.float16)
    # config 1 uses an identity page table, the others a random placement;
    # layout="sequential" forces the identity placement (for locality studies)
    permute = config != 1 and layout != "sequential"
    plan = fmt.plan_pages(tier_of, None, num_seqs, num_kv, dh, 16, rng=rng if permute else None)
    return Workload(name=f"config{config}", dh=dh, num_kv=num_kv, gqa=gqa, num_seqs=num_seqs,
                    lengths=lengths, rope_theta=theta, codebooks=cbs, K=K, V=V, q=q,
                    tier_of=tier_of, plan=plan)


def make_encode_workload(seed: int = 3, tokens: int = 8192, num_kv: int = 8, dh: int = 128) -> Workload:
    """Config 3: 8192 new pre-RoPE K tokens x 8 KV heads, N(0,1) x per-channel
    lognormal(0, 0.5), 1 % of channels x 8, per (head, token) 70/30 tier 1/2."""
    rng = np.random.default_rng(seed)
    cbs = make_codebooks(rng, num_kv, dh, [1, 2])
    scale = np.exp(rng.normal(0.0, 0.5, size=(num_kv, dh)))
    n_out = max(1, int(round(0.01 * dh)))
    for h in range(num_kv):
        scale[h, rng.choice(dh, size=n_out, replace=False)] *= 8.0
    K = [(rng.standard_normal((num_kv, tokens, dh)) * scale[:, None, :]).astype(np.float16)]
    tier_of = [_assign_tiers(rng, tokens, [(1, .7), (2, .3)]) for _ in range(num_kv)]
    V = [rng.standard_normal((num_kv, tokens, dh)).astype(np.float16)]
    q = np.zeros((1, num_kv, dh), np.float16)
    plan = fmt.plan_pages(tier_of, None, 1, num_kv, dh, 16, rng=None)
    return Workload(name="config3", dh=dh, num_kv=num_kv, gqa=1, num_seqs=1, lengths=[tokens],
                    rope_theta=500000.0, codebooks=cbs, K=K, V=V, q=q, tier_of=tier_of, plan=plan)
