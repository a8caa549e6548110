"""omega importance EMA on MI355X: the update the reference runs after each
Mode-A decode (spherical_kv_pipeline.py:952-987 `_omega_ema_eager` /
`_omega_ema_compiled`, driven by `_update_omega_gpu` at :1669-1701).

Same argument meaning as the reference: m_q, l_q are the [num_q, max_blocks]
(m, l) views of the decode's partial_scratch ([..., 0] and [..., 1]); the
strided views are read in place.  Returns the new omega [num_kv, max_blocks]
fp32 (out of place, like the reference; pass `out=omega_prev` to update in
place).  One HIP kernel; raises if libsphkv.so is missing.
"""
from __future__ import annotations

from typing import Optional

import torch

import sphkv_lib
from sphkv_lib import check

_lib = sphkv_lib.load()

EMA_BETA = 0.9          # spherical_kv_pipeline.py EMA_BETA


def _view_ok(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor) or not t.is_cuda or t.dtype != torch.float32 or t.dim() != 2:
        raise ValueError(f"{name} must be a 2-D fp32 CUDA (HIP) tensor")


def omega_ema(m_q: torch.Tensor, l_q: torch.Tensor, omega_prev: torch.Tensor, num_kv: int, kv_groups: int,
              max_blocks: int, ema_beta: float, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """omega_prev * ema_beta + mean over each kv head's q heads of the
    per-page attention mass (spherical_kv_pipeline.py:970-987)."""
    _view_ok(m_q, "m_q")
    _view_ok(l_q, "l_q")
    nq = int(num_kv) * int(kv_groups)
    if tuple(m_q.shape) != (nq, int(max_blocks)) or m_q.shape != l_q.shape or m_q.stride() != l_q.stride():
        raise ValueError(f"m_q and l_q must be [{nq}, {max_blocks}] views with equal strides")
    omega_prev = omega_prev.contiguous()
    if omega_prev.dtype != torch.float32 or tuple(omega_prev.shape) != (int(num_kv), int(max_blocks)):
        raise ValueError(f"omega_prev must be fp32 [{num_kv}, {max_blocks}]")
    if out is None:
        out = torch.empty_like(omega_prev)
    elif out.dtype != torch.float32 or not out.is_contiguous() or out.shape != omega_prev.shape:
        raise ValueError("out must be a contiguous fp32 tensor shaped like omega_prev")
    rc = _lib.sphkv_omega_ema(m_q.data_ptr(), l_q.data_ptr(), m_q.stride(0), m_q.stride(1), omega_prev.data_ptr(),
                              out.data_ptr(), int(num_kv), int(kv_groups), int(max_blocks), float(ema_beta),
                              sphkv_lib.current_stream())
    check(rc, "omega_ema")
    return out


def update_omega_gpu(omega: dict, layer_idx: int, pool, ema_beta: float = EMA_BETA) -> torch.Tensor:
    """`_update_omega_gpu` (spherical_kv_pipeline.py:1669-1701) for a
    LayerPool-like `pool` (num_kv, kv_groups, max_blocks, device,
    _partial_scratch): lazily starts the layer's omega at ones and replaces it
    with the EMA of this step's page masses."""
    if layer_idx not in omega:
        omega[layer_idx] = torch.ones(pool.num_kv, pool.max_blocks, device=pool.device, dtype=torch.float32)
    ml = pool._partial_scratch[:, :, :2]
    omega[layer_idx] = omega_ema(ml[..., 0], ml[..., 1], omega[layer_idx], pool.num_kv, pool.kv_groups,
                                 pool.max_blocks, ema_beta)
    return omega[layer_idx]
