"""sphkv_decode_paged_noalloc (the allocation-free variant of
sphkv_decode_paged, its partials in the library's per-device scratch array)
against sphkv_decode_paged with a caller workspace, through the C ABI: the
same inputs give the same output bit for bit, on two calls in a row (the
second with a smaller input, so the scratch keeps the first call's larger
contents), and requests beyond the scratch size are refused with an error."""
import ctypes

import numpy as np
import pytest
import torch

import sphkv_lib
import sphkv_ops as ops
import sphkv_synth as synth
from gpu_helpers import log, pool_from_oracle

pytestmark = pytest.mark.gpu


def _noalloc(pool, q, gqa, theta, out):
    plan = pool.plan
    c1, c2, c3 = pool.cb_ptrs()
    rc = sphkv_lib.load().sphkv_decode_paged_noalloc(
        pool.pages.data_ptr(), plan.pages_bytes, pool.ptable.data_ptr(), pool.vslot.data_ptr(),
        pool.positions.data_ptr(), plan.num_rows, pool.v_pool.data_ptr(), plan.num_vpages,
        c1, c2, c3, pool.work.data_ptr(), pool.num_items, pool.work_start.data_ptr(),
        plan.num_seqs, plan.num_kv, gqa, q.data_ptr(), out.data_ptr(), plan.dh, plan.page_size,
        float(1.0 / np.sqrt(plan.dh)), float(theta), torch.cuda.current_stream().cuda_stream)
    sphkv_lib.check(rc, "sphkv_decode_paged_noalloc")
    return out


def test_noalloc_equals_workspace_decode_on_two_calls(gpu):
    for ctx, rpi in ((6000, 16), (1500, 64)):            # the second call: fewer rows and items
        wl = synth.make_decode_workload(2, ctx_override=ctx)
        pool, _ = pool_from_oracle(wl, gpu, rows_per_item=rpi)
        log(f"noalloc: ctx {ctx}, {pool.num_items} items")
        q = torch.as_tensor(wl.q, device=gpu)
        ref = ops.decode_paged(pool, q, wl.gqa, wl.rope_theta, check=True)
        out = torch.full_like(q, float("nan"))
        _noalloc(pool, q, wl.gqa, wl.rope_theta, out)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)


def test_noalloc_rejects_more_items_than_the_scratch_holds(gpu):
    lib = sphkv_lib.load()
    per_item = lib.sphkv_decode_paged_workspace_bytes(1, 4, 128) - lib.sphkv_decode_paged_workspace_bytes(0, 4, 128)
    too_many = (8 << 20) // per_item + 1
    rc = lib.sphkv_decode_paged_noalloc(None, 0, None, None, None, 0, None, 0, None, None, None, None, too_many,
                                        None, 1, 8, 4, None, None, 128, 16, 0.088, 5e5, None)
    assert rc == -1 and "scratch" in lib.sphkv_last_error().decode()
