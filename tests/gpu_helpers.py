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


def check_sampled_heads(wl, pool, out, n_heads: int, seed: int, tol: float = 2e-3) -> float:
    """Parity of a full-size decode on a seeded sample of (seq, kv head)
    pairs.  For each: the oracle encodes the head's own workload (its tiers,
    K, V, codebooks; grouping from oracle/paging.py), whose pages and V rows
    must equal the GPU pool's bytes for that head's rows (bit-exact); then
    the fp64 oracle decode of the head must match out[seq, head*gqa:(head+1)*gqa]
    within tol.  Returns the largest error."""
    rng = np.random.default_rng(seed)
    num_sh = wl.num_seqs * wl.num_kv
    pick = rng.choice(num_sh, size=min(n_heads, num_sh), replace=False)
    plan = wl.plan
    ptab = pool.ptable.cpu().numpy().astype(np.int64)
    vsl = pool.vslot.cpu().numpy().astype(np.int64)
    worst = 0.0
    for sh in sorted(int(x) for x in pick):
        s, h = divmod(sh, wl.num_kv)
        sub = wl.head_workload(s, h)
        cpu = oracle.build_pool(sub)
        rows = np.arange(int(plan.row_start[sh]), int(plan.row_start[sh + 1]))
        assert rows.size == sub.plan.num_rows
        # page bytes and V of the head's rows, copied back from the GPU pool
        for i, p in enumerate(rows):
            n = int(sub.plan.count[i])
            size = fmt.page_nbytes(int(sub.plan.tier[i]), n, wl.dh)
            a0, b0 = int(ptab[p, 0]), int(sub.plan.ptable[i, 0])
            got = pool.pages[a0:a0 + size].cpu().numpy()
            assert (got == cpu["pages"][b0:b0 + size]).all(), f"(seq {s}, head {h}) row {p}: page bytes differ"
        vg = pool.v_pool[torch.as_tensor(vsl[rows], device=pool.device)].cpu().numpy()
        assert (vg.view(np.uint16) == cpu["v_pool"][sub.plan.vslot].view(np.uint16)).all(), \
            f"(seq {s}, head {h}): V pages differ"
        want = oracle.decode_mode_b(cpu, sub.plan, sub.codebooks, sub.q, sub.gqa, sub.rope_theta)[0]
        got = out[s, h * wl.gqa:(h + 1) * wl.gqa].float().cpu().numpy()
        err = max_err(got, want)
        log(f"  (seq {s}, head {h}): {rows.size} rows, max abs err {err:.3e}")
        worst = max(worst, err)
        assert err <= tol
    return worst
