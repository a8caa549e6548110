"""CPU restatement of the reference's page grouping.  TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module, as the checker of the build's planners (sphkv_format.plan_pages on the
host, sphkv_plan.hip on the GPU).  The product never imports it.

Restated reference lines (paths relative to the reference repository root):

* retained_tokens       the order allocate() returns its tokens in:
                        sinks + recents + ctrl (allocation.py:28-37, 207-217)
                        over the prefill token list built layer -> head ->
                        index (spherical_kv_pipeline.py:1444-1466); tier-0
                        (dropped) tokens are not retained (allocation.py:214-216).
* group_pages           _build_per_head_pages' grouping, sort and chunking
                        (spherical_kv_pipeline.py:1156-1163, 1187-1190): one
                        group per (layer, head, tier) key in order of first
                        appearance in the retained list (dict insertion
                        order), tokens sorted by index, chunks of PAGE_SIZE;
                        per (layer, head) the groups in key order (:1160-1162,
                        :1215).
* page_offsets          the pointer-table rows of one (layer, head, tier)
                        buffer (:1198-1213): pages back to back from offset 0,
                        theta_offset = offset + 8 + 4G, radius_offset =
                        theta_offset + ceil(N*G*b/8).
* build_per_head_pages  the whole function (:1146-1228): per (layer, head) a
                        list of 7-tuples (pages, ptable, b_theta, n_tokens, V,
                        (r, theta), positions); a group with no codebook is
                        skipped (:1166-1172).

The build's batch of sequences takes the place of the reference's layers: one
page set per (sequence, kv head).  Its dense fp16 tier (id 0xFF, an addition
of this build) groups like any tier; its page is the 8-byte header and the
fp16 K rows (theta_offset = offset + 8, radius_offset = theta_offset + 2*N*dh).
"""
from __future__ import annotations

from collections import namedtuple
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

HEADER_BYTES = 8                    # config.py:3
DENSE_TIER_ID = 0xFF
TIER_GEOMETRY = {1: (16, 6), 2: (16, 4), 3: (32, 3)}     # tiers.py:35-41: tier -> (g, b_theta)

# One retained token: (layer or sequence, kv head, tier id, token index).
RetainedToken = namedtuple("RetainedToken", "seq head tier index")


def retained_tokens(tier_of: Sequence[np.ndarray], num_seqs: int, num_kv: int,
                    sink: int = 0, recent: int = 0) -> List[RetainedToken]:
    """The retained list as allocate() returns it: every token of every (seq,
    head) enumerated seq -> head -> index, split into sinks (index < sink),
    recents (index >= L - recent) and the rest, concatenated sinks + recents +
    rest; tokens of tier 0 are dropped.  tier_of[s*num_kv + h] gives the
    tier of each token of that (seq, head)."""
    sinks, recents, ctrl = [], [], []
    for s in range(num_seqs):
        for h in range(num_kv):
            t_of = np.asarray(tier_of[s * num_kv + h]).astype(np.int64)
            L = t_of.shape[0]
            for i in range(L):
                tok = RetainedToken(s, h, int(t_of[i]), i)
                if i < sink:
                    sinks.append(tok)
                elif i >= L - recent:
                    recents.append(tok)
                else:
                    ctrl.append(tok)
    return [t for t in sinks + recents + ctrl if t.tier != 0]


def group_pages(retained: Sequence[RetainedToken], page_size: int = 16
                ) -> Dict[Tuple[int, int], List[Tuple[int, List[List[int]]]]]:
    """{(seq, head): [(tier, [chunk token indices, ...]), ...]} in the
    reference's order (see the module docstring)."""
    groups: Dict[Tuple[int, int, int], List[RetainedToken]] = {}
    for ts in retained:                                  # insertion order = first appearance
        groups.setdefault((ts.seq, ts.head, ts.tier), []).append(ts)
    per_head: Dict[Tuple[int, int], List[Tuple[int, List[List[int]]]]] = {}
    for (s, h, tier), toks in groups.items():
        idx = [t.index for t in sorted(toks, key=lambda t: t.index)]
        chunks = [idx[i:i + page_size] for i in range(0, len(idx), page_size)]
        per_head.setdefault((s, h), []).append((tier, chunks))
    return per_head


def section_sizes(tier: int, n: int, dh: int) -> Tuple[int, int, int]:
    """(header bytes, theta bytes, radius bytes) of a page of n tokens."""
    if tier == DENSE_TIER_ID:
        return HEADER_BYTES, 2 * n * dh, 0
    g, b = TIER_GEOMETRY[tier]
    G = dh // g
    return HEADER_BYTES + 4 * G, (n * G * b + 7) // 8, n * G


def page_offsets(tier: int, counts: Sequence[int], dh: int) -> np.ndarray:
    """Pointer-table rows int32 [P, 3] of one (head, tier) buffer whose pages
    hold counts[i] tokens, placed back to back from offset 0."""
    rows, off = [], 0
    for n in counts:
        hdr, tb, rb = section_sizes(tier, int(n), dh)
        rows.append((off, off + hdr, off + hdr + tb))
        off += hdr + tb + rb
    return np.asarray(rows, np.int32).reshape(-1, 3)


def build_per_head_pages(retained: Sequence[RetainedToken], K: Dict[Tuple[int, int], np.ndarray],
                         V: Dict[Tuple[int, int], np.ndarray], codebooks: Dict[int, np.ndarray], dh: int,
                         page_size: int = 16):
    """K[(seq, head)], V[(seq, head)]: [L, dh] arrays; codebooks[tier]:
    [num_kv, G, C, g] fp32.  Returns {(seq, head): [(pages uint8, ptable int32
    [P, 3], b_theta, n_tokens, V [n, dh], (r [n, G] fp32, theta [n, G]
    int32), positions int64 [n]), ...]} -- the reference's per_head dict, with
    the encode and page build of the C oracle (bit-exact with torch CPU)."""
    import oracle                       # the C encode / page build
    per_head: Dict[Tuple[int, int], list] = {}
    for (s, h), tiers in group_pages(retained, page_size).items():
        for tier, chunks in tiers:
            if tier != DENSE_TIER_ID and tier not in codebooks:
                continue                                 # no codebook for the key: skipped
            K_lh, V_lh = K[(s, h)], V[(s, h)]
            pages, r_parts, th_parts, v_parts, pos_parts = [], [], [], [], []
            for chunk in chunks:
                ix = np.asarray(chunk, np.int64)
                if tier == DENSE_TIER_ID:
                    hdr = np.zeros(HEADER_BYTES, np.uint8)
                    hdr[0], hdr[1] = DENSE_TIER_ID, len(chunk) & 0xFF
                    pages.append(np.concatenate([hdr, np.frombuffer(
                        np.ascontiguousarray(K_lh[ix], np.float16).tobytes(), np.uint8)]))
                else:
                    g, b = TIER_GEOMETRY[tier]
                    r, codes = oracle.encode_groups(np.asarray(K_lh[ix], np.float32), codebooks[tier][h])
                    pages.append(oracle.build_page(r, codes, tier, b))
                    r_parts.append(r)
                    th_parts.append(codes)
                v_parts.append(np.asarray(V_lh[ix]))
                pos_parts.append(ix)
            ptable = page_offsets(tier, [len(c) for c in chunks], dh)
            b_theta = 16 if tier == DENSE_TIER_ID else TIER_GEOMETRY[tier][1]
            rt = (np.concatenate(r_parts), np.concatenate(th_parts)) if r_parts else (None, None)
            per_head.setdefault((s, h), []).append(
                (np.concatenate(pages), ptable, b_theta, int(sum(len(c) for c in chunks)),
                 np.concatenate(v_parts), rt, np.concatenate(pos_parts)))
    return per_head


def check_plan(plan, groups: Dict[Tuple[int, int], List[Tuple[int, List[List[int]]]]],
               heads: Optional[Sequence[int]] = None, positions_of: Optional[Sequence[np.ndarray]] = None) -> None:
    """Assert that a planner's rows (sphkv_format.PagePlan, or DevicePlan.to_host())
    are the reference grouping: for every (seq, head) `sh` (all, or those in
    `heads`), its rows row_start[sh] .. row_start[sh+1] are, in order, the
    chunks of group_pages' tiers in their order -- tier id, count and token
    indices -- and each row's theta / radius offsets lie where the
    reference's buffer puts them relative to the page offset.  Placement
    (absolute, aligned offsets; V slots) is the build's own and not compared.
    Positions are the token indices (:1199), or positions_of[seq][index]."""
    num_sh = plan.num_seqs * plan.num_kv
    for sh in (range(num_sh) if heads is None else heads):
        s, h = divmod(int(sh), plan.num_kv)
        want = groups.get((s, h), [])
        rows = list(range(int(plan.row_start[sh]), int(plan.row_start[sh + 1])))
        exp = [(tier, chunk) for tier, chunks in want for chunk in chunks]
        assert len(rows) == len(exp), f"(seq {s}, head {h}): {len(rows)} rows, reference grouping has {len(exp)}"
        k = 0
        for tier, chunks in want:
            rel = page_offsets(tier, [len(c) for c in chunks], plan.dh)
            rel = rel - rel[:, :1]
            for ci, chunk in enumerate(chunks):
                p = rows[k]
                n = len(chunk)
                assert int(plan.tier[p]) == tier, f"row {p}: tier {int(plan.tier[p])} != {tier}"
                assert int(plan.count[p]) == n, f"row {p}: count {int(plan.count[p])} != {n}"
                tok = np.asarray(plan.tokens[p])
                assert (tok[:n] == np.asarray(chunk)).all() and (tok[n:] == -1).all(), f"row {p}: tokens differ"
                # positions are the token indices (:1199, positions_parts)
                pos = np.asarray(plan.positions[p])
                want_pos = np.asarray(chunk) if positions_of is None else np.asarray(positions_of[s])[chunk]
                assert (pos[:n] == want_pos).all() and (pos[n:] == -1).all(), f"row {p}: positions differ"
                pt = np.asarray(plan.ptable[p], np.int64)
                assert (pt - pt[0] == rel[ci]).all(), f"row {p}: section offsets {pt - pt[0]} != {rel[ci]}"
                k += 1
