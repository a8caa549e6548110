"""Shared helpers of the GPU parity tests."""
import sys

import numpy as np
import torch

import oracle
import sphkv_format as fmt
import sphkv_ops as ops


def log(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def pool_from_oracle(wl, dev, rows_per_item=None):
    """Upload a CPU-oracle-built pool to the GPU (isolates the decode kernel
    from the GPU encoder)."""
    cpu = oracle.build_pool(wl)
    pool = ops.PagedPool.allocate(wl.plan, wl.codebooks, dev, rows_per_item)
    pool.pages.copy_(torch.from_numpy(cpu["pages"]))
    pool.v_pool.copy_(torch.from_numpy(cpu["v_pool"]))
    return pool, cpu


def single_page_plan(n: int, tier_id: int, dh: int):
    return fmt.plan_pages([np.full(n, tier_id, np.int32)], None, 1, 1, dh, 16)


def max_err(a, b) -> float:
    return float(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64)).max())
