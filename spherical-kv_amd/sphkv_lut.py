"""LayerPool on MI355X: the reference's per-layer Mode-A pool
(sphkv_lut.py:17-206) with the same constructor, attributes and
`append_and_compute`, built for HIP.

The constructor plans pages on the host in the reference's order (kv head,
then each (layer, head) page tuple, then page) and builds every page in one
kernel launch (sphkv_build_layer_pool) instead of a Python loop of torch ops
per page; per decode step the new page's block-table column is written in
place instead of re-uploading the whole table.  Decode and append go through
fused_decode (the HIP drop-in), as in the reference.
"""
from __future__ import annotations

from typing import Dict

import numpy as np
import torch

import sphkv_lib
from fused_decode import sphkv_decode, sphkv_encode_append
from sphkv_lib import check

_lib = sphkv_lib.load()


def make_tier_idx_map(tiers) -> Dict[int, int]:
    """Rank of each stored tier in `tiers` order (sphkv_lut.py:7-14)."""
    out, rank = {}, 0
    for t in tiers:
        if getattr(t, "tier_id", 0) == 0:
            continue
        out[t.tier_id] = rank
        rank += 1
    return out


def _get_codebook(codebooks, layer: int, kv_head: int, tier_id: int):
    """codebook_loader.py:62-69."""
    return codebooks.get((layer, kv_head, tier_id))


class LayerPool:
    """sphkv_lut.py:17-206.  `pipeline` needs `per_head_pages[(layer, h)]`
    (lists of tuples whose first six entries are (pages, ptable, b_theta,
    n_tokens, V [n, dh], (r [n, G], theta [n, G]))) and `codebooks[(layer, h,
    tier_id)]` ([G, C, g])."""

    def __init__(self, pipeline, layer_idx, page_size, G_max, cb_size_max,
                 decode_capacity, device, tiers, tier_idx_map,
                 num_q, num_kv, kv_groups, dh):
        self.page_size = page_size
        self.G_max = G_max
        self.cb_size_max = cb_size_max
        self.tier_idx_map = tier_idx_map
        self.num_kv = num_kv
        self.num_q = num_q
        self.kv_groups = kv_groups
        self.dh = dh
        self.device = device
        self.g_max = max(t.g for t in tiers if getattr(t, "tier_id", 0) != 0)

        # ---- page plan (sphkv_lut.py:36-68): order of pages = order of pids
        r_parts, th_parts, v_parts, src = [], [], [], []
        head_blocks = {h: [] for h in range(num_kv)}
        ctx_lens = [0] * num_kv
        e_off = v_off = 0
        for h in range(num_kv):
            for ph_tuple in pipeline.per_head_pages.get((layer_idx, h), []):
                _pt, _ptt, b_theta, n_tokens, V_tier, K_tier = ph_tuple[:6]
                r_full, theta_full = K_tier
                tier_obj = next(t for t in tiers if getattr(t, "tier_id", 0) != 0 and t.b_theta == b_theta)
                t_idx = tier_idx_map[tier_obj.tier_id]
                G_t = tier_obj.G
                n_tokens = int(n_tokens)
                r_parts.append(torch.as_tensor(r_full)[:n_tokens].reshape(n_tokens, G_t).to(torch.float32).cpu())
                th_parts.append(torch.as_tensor(theta_full)[:n_tokens].reshape(n_tokens, G_t).to(torch.int64)
                                .bitwise_and(0xFF).to(torch.int32).cpu())
                v_parts.append(torch.as_tensor(V_tier)[:n_tokens].reshape(n_tokens, dh).to(torch.float16).cpu())
                for pg in range((n_tokens + page_size - 1) // page_size):
                    s = pg * page_size
                    e = min(s + page_size, n_tokens)
                    head_blocks[h].append((len(src), t_idx))
                    src.append((e_off + s * G_t, v_off + s, e - s, G_t))
                e_off += n_tokens * G_t
                v_off += n_tokens
            ctx_lens[h] = len(head_blocks[h]) * page_size

        n_used = len(src)
        n_total = n_used + decode_capacity
        max_blk = max((len(v) for v in head_blocks.values()), default=0)
        max_blk += (decode_capacity // max(num_kv, 1)) + 2
        self.max_blocks = max_blk
        self.num_pages_used = n_used

        self.theta_codes = torch.zeros((n_total, page_size, G_max), dtype=torch.uint8, device=device)
        self.radius_codes = torch.zeros((n_total, page_size, G_max), dtype=torch.uint8, device=device)
        self.r_scales = torch.zeros((n_total, G_max), dtype=torch.float32, device=device)
        self.v_pool = torch.zeros((n_total, page_size, dh), dtype=torch.float16, device=device)
        if n_used:
            r_all = torch.cat([x.reshape(-1) for x in r_parts]).to(device)
            th_all = torch.cat([x.reshape(-1) for x in th_parts]).to(device)
            v_all = torch.cat(v_parts).to(device).contiguous()
            page_src = torch.tensor(np.asarray(src, np.int64).astype(np.int32), device=device)
            rc = _lib.sphkv_build_layer_pool(
                r_all.data_ptr(), th_all.data_ptr(), r_all.numel(), v_all.data_ptr(), v_all.shape[0],
                page_src.data_ptr(), n_used, 0, self.theta_codes.data_ptr(), self.radius_codes.data_ptr(),
                self.r_scales.data_ptr(), self.v_pool.data_ptr(), n_total, page_size, G_max, dh,
                torch.cuda.current_stream().cuda_stream)
            check(rc, "LayerPool page build")

        self.ctx_lens_cpu = list(ctx_lens)
        self.block_table_cpu = [[-1] * max_blk for _ in range(num_kv)]
        self.bits_table_cpu = [[0] * max_blk for _ in range(num_kv)]
        for h, blist in head_blocks.items():
            for lb, (pid, ti) in enumerate(blist):
                self.block_table_cpu[h][lb] = pid
                self.bits_table_cpu[h][lb] = ti
        self.block_table_gpu = torch.tensor(self.block_table_cpu, dtype=torch.int32, device=device)
        self.bits_table_gpu = torch.tensor(self.bits_table_cpu, dtype=torch.int32, device=device)
        self.ctx_lens_gpu = torch.tensor(self.ctx_lens_cpu, dtype=torch.int32, device=device)

        # ---- codebooks (sphkv_lut.py:100-127)
        num_tiers = len(tier_idx_map)
        self.cb_flat = torch.zeros((num_kv, num_tiers, G_max, cb_size_max, self.g_max),
                                   dtype=torch.float32, device=device)
        self.decode_cb = None
        self._decode_cb_flat = None
        for tier_obj in tiers:
            tid = getattr(tier_obj, "tier_id", 0)
            if tid == 0:
                continue
            t_idx = tier_idx_map[tid]
            G, g, C = tier_obj.G, tier_obj.g, 2 ** tier_obj.b_theta
            heads = []
            for h_kv in range(num_kv):
                cb = _get_codebook(pipeline.codebooks, layer_idx, h_kv, tid)
                if cb is None:
                    break
                heads.append(torch.as_tensor(cb).to(device).float())
            if len(heads) == num_kv:
                stacked = torch.stack(heads)
                self.cb_flat[:, t_idx, :G, :C, :g] = stacked
                if tid == 1:                                  # recent tokens are appended at b1
                    self.decode_cb = stacked
                    self._decode_cb_flat = stacked.contiguous()

        active_tiers = [t for t in tiers if getattr(t, "tier_id", 0) != 0]
        self.tier_G_gpu = torch.tensor([t.G for t in active_tiers], dtype=torch.int32, device=device)
        self.tier_g_gpu = torch.tensor([t.g for t in active_tiers], dtype=torch.int32, device=device)

        self._pids = torch.zeros(num_kv, dtype=torch.long, device=device)
        self._dec_tier_idx = tier_idx_map[1]
        b_dec = next(t for t in tiers if getattr(t, "tier_id", 0) == 1)
        self._G_dec = b_dec.G
        self._g_dec = b_dec.g
        self._C_dec = 2 ** b_dec.b_theta

        self._out_buf = torch.zeros(num_q, dh, dtype=torch.float32, device=device)
        self._partial_scratch = torch.zeros(num_q, max_blk, dh + 2, dtype=torch.float32, device=device)
        self._uniform_ctx = ctx_lens[0] if ctx_lens else 0

    def append_and_compute(self, q_post, k_post, v_new, tiers, sm_scale):
        """sphkv_lut.py:150-206: append this step's token to every kv head
        (opening a page every page_size steps), then decode."""
        cur_len = self._uniform_ctx
        slot = cur_len % self.page_size
        is_new_page = slot == 0
        if is_new_page:
            pg = cur_len // self.page_size
            start_pid = self.num_pages_used
            self.num_pages_used += self.num_kv
            for h in range(self.num_kv):
                self.block_table_cpu[h][pg] = start_pid + h
                self.bits_table_cpu[h][pg] = self._dec_tier_idx
            # only the new page's column changes
            self.block_table_gpu[:, pg] = torch.arange(start_pid, start_pid + self.num_kv, dtype=torch.int32,
                                                       device=self.device)
            self.bits_table_gpu[:, pg] = self._dec_tier_idx
            self._pids[:] = torch.arange(start_pid, start_pid + self.num_kv, dtype=torch.long, device=self.device)
        self._uniform_ctx = cur_len + 1

        sphkv_encode_append(k_post, v_new, self._decode_cb_flat, self.theta_codes, self.radius_codes,
                            self.r_scales, self.v_pool, self._pids, slot, self._G_dec, self._g_dec, self._C_dec,
                            self.G_max, self.dh, self.page_size, 1 if is_new_page else 0)
        self.ctx_lens_gpu.add_(1)
        num_tiers = len(self.tier_idx_map)
        sphkv_decode(q_post, self.cb_flat, self.tier_G_gpu, self.tier_g_gpu, self.theta_codes, self.radius_codes,
                     self.r_scales, self.v_pool, self.block_table_gpu, self.bits_table_gpu, self.ctx_lens_gpu,
                     self._out_buf, self._partial_scratch, self.num_q, self.num_kv, self.kv_groups, num_tiers,
                     self.max_blocks, self.page_size, self.dh, self.G_max, self.cb_size_max, self.g_max,
                     sm_scale, self._uniform_ctx)
        return self._out_buf
