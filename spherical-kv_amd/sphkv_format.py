"""Page / pointer-table format of the angle-domain compressed KV cache.

Host-side description of the byte layout the HIP kernels read and write.  The
layout is the reference's, unchanged:

* tier geometry            tiers.py:3-41 (build_tiers)
* page header              paging.py:5-31 (tier id, count, 6 zero bytes,
                           G little-endian fp32 radius scales)
* page body                pagebuilder.py:8-33 (header | LSB-first packed theta
                           codes | int8 radius codes)
* pointer-table row        pointer_table.py:4-21 and spherical_kv_pipeline.py:1202-1213
                           (page_off, theta_off, radius_off), int32
* per-(head, tier) grouping, position sort and chunking into pages
                           spherical_kv_pipeline.py:1156-1213

Two additions, both encoded without changing the header layout:

* Dense fp16 pages (tier id DENSE_TIER_ID = 0xFF).  They have no radius scales
  (G = 0), so the header is the 8 fixed bytes and the "theta" section holds the
  page's pre-RoPE K rows as fp16 [N, dh].  The radius section is empty.
* Pages are placed at 16-byte aligned offsets (dense payloads at 16-byte
  aligned theta offsets) so that the decode kernel can use 128-bit loads.  The
  pointer table stores absolute offsets, so placement is free.

V is kept beside the pages in a pool of fp16 V pages, [num_vpages,
page_size * dh], each page dim-major: element (token k, dim d) lives at
d * 16 + k within its page (see v_page_index), so the 16 tokens of one dim are
32 contiguous bytes, the decode kernel's PV operand.  Row p of the pointer
table uses V page vslot[p].
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence

import numpy as np

HEADER_BYTES = 8            # config.py:3
EPS = 1e-8                  # config.py:5
DENSE_TIER_ID = 0xFF        # addition: dense fp16 K page
PAGE_ALIGN = 16             # page placement alignment in the byte pool


class Tier:
    """Tier geometry, tiers.py:3-29."""

    def __init__(self, tier_id: int, g: int, b_theta: int, dh: int):
        self.tier_id = tier_id
        self.g = g
        self.b_theta = b_theta
        self.dh = dh
        self.G = (dh // g) if g > 0 else 0

    @property
    def codebook_size(self) -> int:
        return 2 ** self.b_theta if self.b_theta > 0 else 0

    def __repr__(self) -> str:
        return f"Tier(id={self.tier_id}, g={self.g}, G={self.G}, b_theta={self.b_theta})"


def build_tiers(dh: int = 128) -> List[Tier]:
    """tiers.py:35-41: drop, b1 (g16, 6 bit), b2 (g16, 4 bit), b3 (g32, 3 bit)."""
    return [Tier(0, 0, 0, dh), Tier(1, 16, 6, dh), Tier(2, 16, 4, dh), Tier(3, 32, 3, dh)]


# Geometry compiled into the kernels (tier id -> (g, b_theta)).
TIER_GEOMETRY = {1: (16, 6), 2: (16, 4), 3: (32, 3)}


def theta_bytes(n: int, G: int, b: int) -> int:
    return (n * G * b + 7) // 8


def page_nbytes(tier_id: int, n: int, dh: int) -> int:
    """Byte size of one page with n tokens (pagebuilder.py:32 concatenation)."""
    if tier_id == DENSE_TIER_ID:
        return HEADER_BYTES + n * dh * 2
    g, b = TIER_GEOMETRY[tier_id]
    G = dh // g
    return HEADER_BYTES + 4 * G + theta_bytes(n, G, b) + n * G


def ptable_row(page_off: int, tier_id: int, n: int, dh: int):
    """spherical_kv_pipeline.py:1202-1205: (page_off, theta_off, radius_off)."""
    if tier_id == DENSE_TIER_ID:
        th = page_off + HEADER_BYTES
        return page_off, th, th + n * dh * 2
    g, b = TIER_GEOMETRY[tier_id]
    G = dh // g
    th = page_off + HEADER_BYTES + 4 * G
    return page_off, th, th + theta_bytes(n, G, b)


@dataclass
class PagePlan:
    """Which tokens go to which page, and where each page lives.

    Rows are pointer-table rows in logical order: for each (seq, kv_head) the
    rows of its pages, tiers in order of first appearance, positions ascending
    within a tier (spherical_kv_pipeline.py:1156-1163, 1187-1213).
    """
    dh: int
    page_size: int
    num_seqs: int
    num_kv: int
    tier: np.ndarray          # [P] int32 tier id of each row (1,2,3 or 0xFF)
    count: np.ndarray         # [P] int32 tokens in the page
    tokens: np.ndarray        # [P, page_size] int64 source token index (-1 pad)
    positions: np.ndarray     # [P, page_size] int32 absolute position (-1 pad)
    seq_head: np.ndarray      # [P] int32 seq * num_kv + head of each row
    row_start: np.ndarray     # [num_seqs*num_kv + 1] int32 CSR row ranges
    ptable: np.ndarray        # [P, 3] int32
    vslot: np.ndarray         # [P] int32 V page of each row
    pages_bytes: int          # size of the byte pool
    num_vpages: int           # size of the V pool in pages

    @property
    def num_rows(self) -> int:
        return int(self.tier.shape[0])


def plan_pages(tier_of: Sequence[np.ndarray], positions_of: Optional[Sequence[np.ndarray]],
               num_seqs: int, num_kv: int, dh: int, page_size: int = 16,
               rng: Optional[np.random.Generator] = None,
               num_vpages: Optional[int] = None, byte_spread: float = 1.0) -> PagePlan:
    """Group tokens by (seq, head, tier), sort, chunk into pages and place them.

    tier_of[s*num_kv + h] is an int array over the sequence's tokens giving the
    tier id of each token for that head (0 = dropped, 1/2/3, 0xFF = dense).
    positions_of[s] gives each token's absolute position (default 0..L-1).
    If rng is given, pages are placed in a random physical order (random byte
    offsets and random V slots drawn from num_vpages >= P slots); otherwise in
    logical order.  byte_spread > 1 (with rng) leaves a random gap after each
    page, uniform in [0, 2 (byte_spread - 1) x the page's bytes], so the pages
    are scattered over a byte pool about byte_spread times their total size
    (a shared pool that holds other sequences' pages too).
    """
    tiers_l, counts_l, toks_l, pos_l, sh_l = [], [], [], [], []
    row_start = [0]
    for s in range(num_seqs):
        for h in range(num_kv):
            t_of = np.asarray(tier_of[s * num_kv + h])
            L = t_of.shape[0]
            pos = np.arange(L, dtype=np.int64) if positions_of is None else np.asarray(positions_of[s], np.int64)
            # tiers in order of first appearance (dict insertion order in the reference)
            order = []
            for tid in t_of[np.sort(np.unique(t_of, return_index=True)[1])]:
                if int(tid) != 0:
                    order.append(int(tid))
            for tid in order:
                idx = np.nonzero(t_of == tid)[0]            # ascending token index
                for i in range(0, idx.shape[0], page_size):
                    chunk = idx[i:i + page_size]
                    n = chunk.shape[0]
                    tk = np.full(page_size, -1, np.int64); tk[:n] = chunk
                    ps = np.full(page_size, -1, np.int32); ps[:n] = pos[chunk]
                    tiers_l.append(tid); counts_l.append(n); toks_l.append(tk); pos_l.append(ps)
                    sh_l.append(s * num_kv + h)
            row_start.append(len(tiers_l))
    P = len(tiers_l)
    tier = np.asarray(tiers_l, np.int32).reshape(P)
    count = np.asarray(counts_l, np.int32).reshape(P)
    tokens = np.asarray(toks_l, np.int64).reshape(P, page_size)
    positions = np.asarray(pos_l, np.int32).reshape(P, page_size)
    seq_head = np.asarray(sh_l, np.int32).reshape(P)

    # physical placement
    phys_order = np.arange(P) if rng is None else rng.permutation(P)
    ptable = np.zeros((P, 3), np.int64)
    off = 0
    for p in phys_order:
        tid, n = int(tier[p]), int(count[p])
        if tid == DENSE_TIER_ID:
            # payload (header + 8) must be 16-byte aligned
            off = ((off + 8 + PAGE_ALIGN - 1) // PAGE_ALIGN) * PAGE_ALIGN - 8
            if off < 0:
                off += PAGE_ALIGN
        else:
            off = ((off + PAGE_ALIGN - 1) // PAGE_ALIGN) * PAGE_ALIGN
        ptable[p] = ptable_row(off, tid, n, dh)
        nb = page_nbytes(tid, n, dh)
        off += nb
        if rng is not None and byte_spread > 1.0:
            off += int(rng.integers(0, int(2 * (byte_spread - 1.0) * nb) + 1))
    pages_bytes = ((off + PAGE_ALIGN - 1) // PAGE_ALIGN) * PAGE_ALIGN + PAGE_ALIGN
    if pages_bytes >= 2 ** 31:
        raise ValueError("page byte pool exceeds int32 offsets")
    nv = P if num_vpages is None else int(num_vpages)
    if nv < P:
        raise ValueError("num_vpages smaller than the number of pages")
    if rng is None:
        vslot = np.arange(P, dtype=np.int32)
    else:
        vslot = rng.choice(nv, size=P, replace=False).astype(np.int32) if nv > P else rng.permutation(P).astype(np.int32)
    return PagePlan(dh=dh, page_size=page_size, num_seqs=num_seqs, num_kv=num_kv, tier=tier,
                    count=count, tokens=tokens, positions=positions, seq_head=seq_head,
                    row_start=np.asarray(row_start, np.int32), ptable=ptable.astype(np.int32),
                    vslot=vslot, pages_bytes=int(pages_bytes), num_vpages=nv)


def v_page_index(dh: int) -> np.ndarray:
    """[16, dh] int: position of element (token k, dim d) inside a V page."""
    k = np.arange(16)[:, None]
    d = np.arange(dh)[None, :]
    return d * 16 + k


def rope_inv_freq(dh: int, theta: float) -> np.ndarray:
    """Default RoPE inverse frequencies, fp64: theta ** (-2j/dh), j < dh/2."""
    j = np.arange(dh // 2, dtype=np.float64)
    return theta ** (-2.0 * j / dh)


def rope_tables(max_pos: int, dh: int, theta: float):
    """HF-layout cos/sin tables [max_pos, dh] fp32 (second half repeats the
    first), the format spherical_kv_pipeline.py:1591-1610 passes to the
    ragged kernel.  Angles are formed in fp64."""
    ang = np.arange(max_pos, dtype=np.float64)[:, None] * rope_inv_freq(dh, theta)[None, :]
    ang = np.concatenate([ang, ang], axis=1)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def decode_bytes(plan: PagePlan) -> int:
    """Algorithmic HBM bytes of one decode step over `plan`: packed K pages,
    dense K pages, fp16 V, int32 positions and pointer-table rows."""
    tot = 0
    for tid in np.unique(plan.tier):
        m = plan.tier == tid
        n = plan.count[m]
        tid = int(tid)
        tot += int(sum(page_nbytes(tid, int(x), plan.dh) for x in n))
    ntok = int(plan.count.sum())
    tot += ntok * plan.dh * 2                  # V
    tot += plan.num_rows * plan.page_size * 4  # positions
    tot += plan.num_rows * 12                  # pointer table
    return tot
