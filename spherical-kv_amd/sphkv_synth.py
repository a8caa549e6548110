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
* Config 4 scatters its pages over one shared pool of POOL_PAGES_C4 (~1.2M)
  16-token pages: V slots drawn from that many slots, K pages placed with
  random gaps over a byte pool of the same proportion (reduced-size variants
  keep the ratio).

kv_device: K and V are drawn on that torch device instead (torch's Philox
generator seeded from the config seed; K = N(0,1) x the host-drawn channel
scale, rounded to fp16), for full-size workloads whose host draws take
minutes.  The host generator then skips the K and V draws, so the tiers, q
and placement are a different (equally deterministic) instance.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional

import sys

import numpy as np

import sphkv_format as fmt


POOL_PAGES_C4 = 1_200_000      # one shared pool of ~1.2M 16-token pages
FULL_ROWS_C4 = 571_036         # rows of the full config-4 instance (seed 4, host draws)


def _is_torch(x) -> bool:
    return type(x).__module__.startswith("torch")


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
    positions: Optional[List[np.ndarray]] = None   # per seq: absolute position of each token (None: index)

    @property
    def num_q(self) -> int:
        return self.num_kv * self.gqa

    def k_rows(self):
        """K of all sequences as one [rows, dh] fp16 matrix (a torch tensor on
        the device for device-drawn workloads); row of (seq s, head h, token
        t) = row_base[s*num_kv+h] + t."""
        if _is_torch(self.K[0]):
            import torch
            return torch.cat([k.reshape(-1, self.dh) for k in self.K], dim=0)
        return np.concatenate([k.reshape(-1, self.dh) for k in self.K], axis=0)

    def v_rows(self):
        if _is_torch(self.V[0]):
            import torch
            return torch.cat([v.reshape(-1, self.dh) for v in self.V], dim=0)
        return np.concatenate([v.reshape(-1, self.dh) for v in self.V], axis=0)

    def head_kv(self, s: int, h: int):
        """(K [L, dh], V [L, dh]) fp16 numpy arrays of one (seq, kv head)."""
        k, v = self.K[s][h], self.V[s][h]
        if _is_torch(k):
            return k.cpu().numpy(), v.cpu().numpy()
        return np.asarray(k), np.asarray(v)

    def head_workload(self, s: int, h: int) -> "Workload":
        """The workload of one (seq, kv head) alone -- one sequence, one kv
        head, its codebooks, K, V, tiers and queries -- with a logical-order
        plan (the grouping of a (seq, head) does not depend on the others)."""
        k, v = self.head_kv(s, h)
        t_of = [self.tier_of[s * self.num_kv + h]]
        plan = fmt.plan_pages(t_of, None, 1, 1, self.dh, self.page_size)
        return Workload(name=f"{self.name}[s{s}h{h}]", dh=self.dh, num_kv=1, gqa=self.gqa, num_seqs=1,
                        lengths=[self.lengths[s]], rope_theta=self.rope_theta,
                        codebooks={t: c[h:h + 1] for t, c in self.codebooks.items()},
                        K=[k[None]], V=[v[None]], q=self.q[s:s + 1, h * self.gqa:(h + 1) * self.gqa],
                        tier_of=t_of, plan=plan, page_size=self.page_size)

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


def hf_rope_tables(max_pos: int, dh: int, theta: float, device):
    """cos / sin tables [max_pos, dh] fp32 as a default-RoPE transformers
    rotary embedding builds them for spherical_kv_pipeline.py:1597-1608:
    inv_freq = 1 / theta ** (arange(0, dh, 2) / dh) in fp32 (torch's pow),
    angles fl32(inv_freq * pos), the halves concatenated, cos / sin in fp32."""
    import torch
    inv = 1.0 / (theta ** (torch.arange(0, dh, 2, dtype=torch.int64, device=device).float() / dh))
    ang = torch.arange(max_pos, device=device, dtype=torch.float32)[:, None] * inv.float()[None, :]
    ang = torch.cat([ang, ang], dim=1)
    return ang.cos().contiguous(), ang.sin().contiguous()


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
                         num_seqs_override: Optional[int] = None, layout: str = "default",
                         kv_device=None) -> Workload:
    """Decode configs 1, 2, 4, 5.  ctx_override shrinks
    the context (for oracle-sized parity cases) keeping everything else;
    kv_device draws K and V on that torch device (see the module docstring)."""
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
    # large workloads (configs 4, 5) take minutes on the host: report progress
    big = sum(lengths) * num_kv >= (1 << 22)

    def progress(what, i=None):
        if big and (i is None or i % 16 == 15):
            print(f"[synth] config{config}: {what}" + ("" if i is None else f" {i + 1}/{len(lengths)}"),
                  file=sys.stderr, flush=True)

    gen = None
    if kv_device is not None:
        import torch
        gen = torch.Generator(device=kv_device)
        gen.manual_seed(1_000_003 * (seed_d if seed is None else seed) + 17)
        scale_t = torch.as_tensor(scale, dtype=torch.float32, device=kv_device)

    def draw(L, scaled):
        if gen is None:
            x = rng.standard_normal((num_kv, L, dh))
            return (x * scale[:, None, :] if scaled else x).astype(np.float16)
        x = torch.randn((num_kv, L, dh), generator=gen, device=kv_device, dtype=torch.float32)
        return (x * scale_t[:, None, :] if scaled else x).to(torch.float16)

    K = []
    for i, L in enumerate(lengths):
        K.append(draw(L, True))
        progress("K", i)
    tier_of = []
    for L in lengths:
        for h in range(num_kv):
            tier_of.append(_assign_tiers(rng, L, fracs, sink, recent))
    progress("tiers")
    V = []
    for i, L in enumerate(lengths):
        V.append(draw(L, False))
        progress("V", i)
    q = rng.standard_normal((num_seqs, num_kv * gqa, dh)).astype(np.float16)
    # config 1 uses an identity page table, the others a random placement;
    # layout="sequential" forces the identity placement (for locality studies)
    permute = config != 1 and layout != "sequential"
    nv, spread = None, 1.0
    if config == 4 and permute:
        rows = sum(-(-int(np.count_nonzero(t == tid)) // 16) for t in tier_of for tid in np.unique(t) if tid != 0)
        full = ctx_override is None and num_seqs_override is None
        nv = max(POOL_PAGES_C4, rows) if full else int(np.ceil(rows * POOL_PAGES_C4 / FULL_ROWS_C4))
        spread = nv / max(rows, 1)
    plan = fmt.plan_pages(tier_of, None, num_seqs, num_kv, dh, 16, rng=rng if permute else None,
                          num_vpages=nv, byte_spread=spread)
    progress("page plan")
    return Workload(name=f"config{config}", dh=dh, num_kv=num_kv, gqa=gqa, num_seqs=num_seqs,
                    lengths=lengths, rope_theta=theta, codebooks=cbs, K=K, V=V, q=q,
                    tier_of=tier_of, plan=plan)


@dataclass
class TailSteps:
    """Inputs of T decode steps after a workload's context: the tier-3
    codebook that decode tokens are encoded with, and per step the new
    pre-RoPE keys and V rows of every (sequence, kv head), their positions
    (each sequence continues from its length) and the step's queries."""
    cb3: np.ndarray      # fp32 [num_kv, dh/32, 8, 32], unit rows
    k: np.ndarray        # fp16 [T, num_seqs, num_kv, dh]
    v: np.ndarray        # fp16 [T, num_seqs, num_kv, dh]
    pos: np.ndarray      # int32 [T, num_seqs]
    q: np.ndarray        # fp16 [T, num_seqs, num_kv*gqa, dh]


def make_tail_steps(wl: Workload, steps: int, seed: int = 77) -> TailSteps:
    """Decode-step inputs for wl (a generator of its own, so the workload's
    draws are unchanged).  K of the new tokens: N(0,1) fp16."""
    rng = np.random.default_rng(seed)
    cb3 = make_codebooks(rng, wl.num_kv, wl.dh, [3])[3]
    shp = (steps, wl.num_seqs, wl.num_kv, wl.dh)
    k = rng.standard_normal(shp).astype(np.float16)
    v = rng.standard_normal(shp).astype(np.float16)
    pos = (np.asarray(wl.lengths, np.int64)[None, :] + np.arange(steps)[:, None]).astype(np.int32)
    q = rng.standard_normal((steps, wl.num_seqs, wl.num_kv * wl.gqa, wl.dh)).astype(np.float16)
    return TailSteps(cb3=cb3, k=k, v=v, pos=pos, q=q)


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


# Mode-A tier geometry (tiers.py:35-41): tier id -> (g, b); G = dh / g, C = 2^b.
MODEA_TIERS = {1: (16, 6), 2: (16, 4), 3: (32, 3)}


def make_modea_workload(seed: int = 11, num_kv: int = 8, kv_groups: int = 4, dh: int = 128,
                        page_size: int = 16, ctx: int = 4096, tiers=(1, 2), fracs=None,
                        holes: float = 0.0, spare_pages: int = 0, G_pad: int = 0) -> Dict[str, object]:
    """LayerPool-shaped Mode-A tables (sphkv_lut.py:71-127) from a seeded draw.

    Every kv head holds ctx tokens in ceil(ctx / page_size) logical pages placed
    at random pool pages; each logical page has one tier (drawn with weights `fracs`, equal if None),
    uniform theta codes below that tier's C, uniform uint8 radius codes,
    lognormal radius scales; slots past ctx stay zero (codes 0, radius 0), the
    state sphkv_encode_append leaves them in.  `holes` is the fraction of
    logical pages marked absent (-1); G_pad widens G_max (code rows and tables)
    beyond the tiers' largest group count.  cb_flat rows are normalize(N(0,1)),
    zero padded to [G_max, cb_max, g_max]; V ~ N(0,1) fp16; q ~ N(0,1) fp32.
    """
    rng = np.random.default_rng(seed)
    T = len(tiers)
    fracs = np.ones(T) if fracs is None else np.asarray(fracs, np.float64)
    geo = [(dh // MODEA_TIERS[t][0], MODEA_TIERS[t][0], 1 << MODEA_TIERS[t][1]) for t in tiers]   # (G, g, C)
    G_max = max(max(G for G, _, _ in geo), G_pad)
    g_max = max(g for _, g, _ in geo)
    cb_max = max(C for _, _, C in geo)
    cb_flat = np.zeros((num_kv, T, G_max, cb_max, g_max), np.float32)
    for h in range(num_kv):
        for ti, (G, g, C) in enumerate(geo):
            x = rng.standard_normal((G, C, g))
            cb_flat[h, ti, :G, :C, :g] = (x / np.linalg.norm(x, axis=-1, keepdims=True)).astype(np.float32)
    nlog = -(-ctx // page_size)
    n_pages = num_kv * nlog + spare_pages
    perm = rng.permutation(n_pages)[:num_kv * nlog].reshape(num_kv, nlog).astype(np.int32)
    tier_idx = rng.choice(T, size=(num_kv, nlog), p=fracs / fracs.sum()).astype(np.int32)
    if holes > 0:
        perm = np.where(rng.random((num_kv, nlog)) < holes, -1, perm).astype(np.int32)
    theta = np.zeros((n_pages, page_size, G_max), np.uint8)
    radius = np.zeros((n_pages, page_size, G_max), np.uint8)
    r_scales = np.zeros((n_pages, G_max), np.float32)
    v_pool = rng.standard_normal((n_pages, page_size, dh)).astype(np.float16)
    for h in range(num_kv):
        for lb in range(nlog):
            ph = int(perm[h, lb])
            if ph < 0:
                continue
            G, g, C = geo[int(tier_idx[h, lb])]
            n = min(page_size, ctx - lb * page_size)
            theta[ph, :n, :G] = rng.integers(0, C, size=(n, G))
            radius[ph, :n, :G] = rng.integers(1, 256, size=(n, G))
            r_scales[ph, :G] = np.exp(rng.normal(1.0, 0.3, size=G)).astype(np.float32)
    q = rng.standard_normal((num_kv * kv_groups, dh)).astype(np.float32)
    return dict(q=q, cb_flat=cb_flat, tier_G=np.array([G for G, _, _ in geo], np.int32),
                tier_g=np.array([g for _, g, _ in geo], np.int32), theta=theta, radius=radius,
                r_scales=r_scales, v_pool=v_pool, block_table=perm, bits_table=tier_idx,
                ctx_lens=np.full(num_kv, ctx, np.int32), num_kv=num_kv, kv_groups=kv_groups, dh=dh,
                page_size=page_size, num_tiers=T, G_max=G_max, cb_max=cb_max, g_max=g_max, max_blocks=nlog,
                sm_scale=float(1.0 / np.sqrt(dh)), max_ctx=ctx, tiers=tuple(tiers))
