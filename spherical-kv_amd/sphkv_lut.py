"""LayerPool: the per-layer Mode-A page pool that the reference's decode
loop keeps per layer (sphkv_lut.py:17-206).  The constructor arguments,
`append_and_compute` and the attributes the pipeline reads -- num_kv,
kv_groups, max_blocks, device, _partial_scratch
(spherical_kv_pipeline.py:1632-1699) -- are the reference's; the rest is this
build's own:

* the layer's page plan is computed once with numpy over all of its
  (kv head, tier) runs: pages per run, page ids, block-table columns and the
  source offsets of every page, instead of a loop that builds each page;
* every prefill page is quantised and written by one kernel launch
  (sphkv_build_layer_pool), from the runs' radii, codes and V uploaded as
  three flat arrays;
* the codebooks of the tiers whose every kv head has one are gathered into a
  host array of cb_flat's shape and uploaded once;
* per decode step, a page opened for the new token changes one block-table
  column on the device (the host keeps a numpy mirror), and the append and
  the decode run as the two fused_decode calls.
"""
from __future__ import annotations

from typing import Dict, List, Optional

import numpy as np
import torch

import sphkv_lib
from fused_decode import sphkv_decode, sphkv_encode_append
from sphkv_lib import check

_lib = sphkv_lib.load()


def make_tier_idx_map(tiers) -> Dict[int, int]:
    """Tier id -> index of the tier among the stored ones (tier_id != 0), in
    `tiers` order: the tier index of the bits table and of cb_flat
    (sphkv_lut.py:7-14)."""
    stored = [t.tier_id for t in tiers if getattr(t, "tier_id", 0) != 0]
    return {tid: rank for rank, tid in enumerate(stored)}


def _host(x, dtype) -> np.ndarray:
    """A tensor or array as a host numpy array of `dtype`."""
    if isinstance(x, torch.Tensor):
        x = x.detach().cpu().numpy()
    return np.asarray(x).astype(dtype, copy=False)


class LayerPool:
    """Mode-A pool of one layer.  `pipeline.per_head_pages[(layer, h)]` lists
    tuples whose first six entries are (pages, ptable, b_theta, n_tokens,
    V [n, dh], (r [n, G], theta [n, G])); `pipeline.codebooks[(layer, h,
    tier_id)]` is [G, C, g].  Pools: theta_codes / radius_codes uint8 [P,
    page_size, G_max], r_scales fp32 [P, G_max], v_pool fp16 [P, page_size,
    dh], P = prefill pages + decode_capacity; tables block_table_gpu /
    bits_table_gpu int32 [num_kv, max_blocks] (page id / tier index of each
    logical block), ctx_lens_gpu int32 [num_kv]."""

    def __init__(self, pipeline, layer_idx, page_size, G_max, cb_size_max,
                 decode_capacity, device, tiers, tier_idx_map,
                 num_q, num_kv, kv_groups, dh):
        self.page_size, self.G_max, self.cb_size_max = page_size, G_max, cb_size_max
        self.tier_idx_map = tier_idx_map
        self.num_q, self.num_kv, self.kv_groups, self.dh = num_q, num_kv, kv_groups, dh
        self.device = device
        stored = [t for t in tiers if getattr(t, "tier_id", 0) != 0]
        self.g_max = max(t.g for t in stored)
        # a run's tier is the first stored tier with its b_theta (sphkv_lut.py:42-45)
        tier_of_b: Dict[int, object] = {}
        for t in stored:
            tier_of_b.setdefault(t.b_theta, t)

        # ---- the runs of retained tokens, kv head by kv head, in the
        #      pipeline's order (that order is the page-id order) ----------
        run_head, run_tidx, run_G, run_n = [], [], [], []
        r_parts: List[np.ndarray] = []
        th_parts: List[np.ndarray] = []
        v_parts: List[np.ndarray] = []
        for h in range(num_kv):
            for entry in pipeline.per_head_pages.get((layer_idx, h), []):
                _, _, b_theta, n_tokens, v_tier, (r_full, theta_full) = entry[:6]
                tier = tier_of_b[b_theta]
                n = int(n_tokens)
                run_head.append(h)
                run_tidx.append(tier_idx_map[tier.tier_id])
                run_G.append(tier.G)
                run_n.append(n)
                r_parts.append(_host(r_full, np.float32)[:n].reshape(n * tier.G))
                th_parts.append((_host(theta_full, np.int64)[:n].reshape(n * tier.G) & 0xFF).astype(np.int32))
                v_parts.append(_host(v_tier, np.float16)[:n].reshape(n, dh))
        run_head = np.asarray(run_head, np.int64)
        run_G = np.asarray(run_G, np.int64)
        run_n = np.asarray(run_n, np.int64)

        # ---- page plan: pages of each run, their ids and block-table columns
        run_pages = (run_n + page_size - 1) // page_size
        P = int(run_pages.sum())
        page_run = np.repeat(np.arange(run_n.size), run_pages)
        first_page_of_run = np.cumsum(run_pages) - run_pages
        page_in_run = np.arange(P) - first_page_of_run[page_run]
        page_head = run_head[page_run]
        head_pages = np.bincount(page_head, minlength=num_kv) if P else np.zeros(num_kv, np.int64)
        first_page_of_head = np.cumsum(head_pages) - head_pages
        page_col = np.arange(P) - first_page_of_head[page_head]           # heads' pages are contiguous ids
        tok0 = page_in_run * page_size                                   # first token of each page in its run
        elem_base = np.cumsum(run_n * run_G) - run_n * run_G             # run offsets into the flat r / theta
        tok_base = np.cumsum(run_n) - run_n                              # run offsets into the flat V

        self.num_pages_used = P
        self.max_blocks = int(head_pages.max(initial=0)) + decode_capacity // max(num_kv, 1) + 2
        n_total = P + decode_capacity
        self.theta_codes = torch.zeros((n_total, page_size, G_max), dtype=torch.uint8, device=device)
        self.radius_codes = torch.zeros((n_total, page_size, G_max), dtype=torch.uint8, device=device)
        self.r_scales = torch.zeros((n_total, G_max), dtype=torch.float32, device=device)
        self.v_pool = torch.zeros((n_total, page_size, dh), dtype=torch.float16, device=device)
        if P:
            # per page: (first r / theta element, first V row, tokens, G)
            src = np.stack([elem_base[page_run] + tok0 * run_G[page_run], tok_base[page_run] + tok0,
                            np.minimum(run_n[page_run] - tok0, page_size), run_G[page_run]], axis=1)
            r_all = torch.from_numpy(np.concatenate(r_parts)).to(device)
            th_all = torch.from_numpy(np.concatenate(th_parts)).to(device)
            v_all = torch.from_numpy(np.concatenate(v_parts)).to(device)
            page_src = torch.from_numpy(src.astype(np.int32)).to(device)
            check(_lib.sphkv_build_layer_pool(
                r_all.data_ptr(), th_all.data_ptr(), r_all.numel(), v_all.data_ptr(), v_all.shape[0],
                page_src.data_ptr(), P, 0, self.theta_codes.data_ptr(), self.radius_codes.data_ptr(),
                self.r_scales.data_ptr(), self.v_pool.data_ptr(), n_total, page_size, G_max, dh,
                sphkv_lib.current_stream()), "LayerPool page build")

        # ---- tables: host mirror (numpy) and device copies ------------------
        self.block_table_cpu = np.full((num_kv, self.max_blocks), -1, np.int32)
        self.bits_table_cpu = np.zeros((num_kv, self.max_blocks), np.int32)
        self.block_table_cpu[page_head, page_col] = np.arange(P, dtype=np.int32)
        self.bits_table_cpu[page_head, page_col] = np.asarray(run_tidx, np.int32)[page_run]
        self.ctx_lens_cpu = (head_pages * page_size).astype(np.int32)
        self.block_table_gpu = torch.from_numpy(self.block_table_cpu.copy()).to(device)
        self.bits_table_gpu = torch.from_numpy(self.bits_table_cpu.copy()).to(device)
        self.ctx_lens_gpu = torch.from_numpy(self.ctx_lens_cpu.copy()).to(device)

        # ---- codebooks: tiers whose every kv head has one (sphkv_lut.py:100-127)
        cb = np.zeros((num_kv, len(tier_idx_map), G_max, cb_size_max, self.g_max), np.float32)
        dec_cb: Optional[np.ndarray] = None
        for t in stored:
            per_head = [pipeline.codebooks.get((layer_idx, h, t.tier_id)) for h in range(num_kv)]
            if any(x is None for x in per_head):
                continue
            arr = np.stack([_host(x, np.float32) for x in per_head])        # [num_kv, G, C, g]
            cb[:, tier_idx_map[t.tier_id], :t.G, :2 ** t.b_theta, :t.g] = arr
            if t.tier_id == 1:                                             # appended tokens use tier 1
                dec_cb = arr
        self.cb_flat = torch.from_numpy(cb).to(device)
        self.decode_cb = None if dec_cb is None else torch.from_numpy(np.ascontiguousarray(dec_cb)).to(device)
        self._decode_cb_flat = self.decode_cb
        self.tier_G_gpu = torch.tensor([t.G for t in stored], dtype=torch.int32, device=device)
        self.tier_g_gpu = torch.tensor([t.g for t in stored], dtype=torch.int32, device=device)

        # ---- decode-step state ----------------------------------------------
        dec = next(t for t in stored if t.tier_id == 1)
        self._G_dec, self._g_dec, self._C_dec = dec.G, dec.g, 2 ** dec.b_theta
        self._dec_tier_idx = tier_idx_map[1]
        self._heads = torch.arange(num_kv, dtype=torch.long, device=device)
        self._pids = torch.zeros(num_kv, dtype=torch.long, device=device)
        self._capacity = n_total
        self._out_buf = torch.zeros(num_q, dh, dtype=torch.float32, device=device)
        self._partial_scratch = torch.zeros(num_q, self.max_blocks, dh + 2, dtype=torch.float32, device=device)
        self._uniform_ctx = int(self.ctx_lens_cpu[0]) if num_kv else 0

    def _open_page(self, block: int) -> None:
        """Give every kv head a fresh page for logical block `block` (the next
        num_kv page ids) and record it in both tables (sphkv_lut.py:160-171)."""
        start = self.num_pages_used
        if start + self.num_kv > self._capacity or block >= self.max_blocks:
            raise RuntimeError(f"LayerPool: decode capacity exhausted (block {block}, pages {start})")
        self.num_pages_used = start + self.num_kv
        self.block_table_cpu[:, block] = np.arange(start, start + self.num_kv, dtype=np.int32)
        self.bits_table_cpu[:, block] = self._dec_tier_idx
        torch.add(self._heads, start, out=self._pids)
        self.block_table_gpu[:, block] = self._pids.to(torch.int32)
        self.bits_table_gpu[:, block] = self._dec_tier_idx

    def append_and_compute(self, q_post, k_post, v_new, tiers, sm_scale):
        """One decode step (sphkv_lut.py:150-206): append the token's K / V
        of every kv head (slot ctx % page_size of the head's last page, a new
        page every page_size tokens), then decode the layer's q heads over
        the pool.  Returns the fp32 output [num_q, dh] (an internal buffer)."""
        ctx = self._uniform_ctx
        slot = ctx % self.page_size
        if slot == 0:
            self._open_page(ctx // self.page_size)
        self._uniform_ctx = ctx + 1
        sphkv_encode_append(k_post, v_new, self._decode_cb_flat, self.theta_codes, self.radius_codes,
                            self.r_scales, self.v_pool, self._pids, slot, self._G_dec, self._g_dec, self._C_dec,
                            self.G_max, self.dh, self.page_size, int(slot == 0))
        self.ctx_lens_gpu.add_(1)
        sphkv_decode(q_post, self.cb_flat, self.tier_G_gpu, self.tier_g_gpu, self.theta_codes, self.radius_codes,
                     self.r_scales, self.v_pool, self.block_table_gpu, self.bits_table_gpu, self.ctx_lens_gpu,
                     self._out_buf, self._partial_scratch, self.num_q, self.num_kv, self.kv_groups,
                     len(self.tier_idx_map), self.max_blocks, self.page_size, self.dh, self.G_max,
                     self.cb_size_max, self.g_max, sm_scale, self._uniform_ctx)
        return self._out_buf
