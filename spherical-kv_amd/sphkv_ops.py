"""torch-facing operations over the paged angle-domain KV pool.

PyTorch provides device memory and the stream; all compute runs in
libsphkv.so (HIP, gfx950).  No CPU or torch fallback exists: inputs on the
wrong device, or a missing library, raise.
"""
from __future__ import annotations

import math
import weakref
from dataclasses import dataclass
from typing import Dict, Optional, Tuple

import numpy as np
import torch

import sphkv_format as fmt
from sphkv_lib import check, current_stream, load

_check_rc = check      # decode_paged's `check` argument shadows the name there

ROWS_PER_ITEM = 64     # pointer-table rows per decode work item (8 pages per wave, 8 waves)


def _stream() -> int:
    return current_stream()


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _need(t: torch.Tensor, dtype, name: str, device=None):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_cuda:
        raise ValueError(f"{name} must be on a GPU device (the library has no CPU path)")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if device is not None and t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")


def _row_start32(row_start) -> np.ndarray:
    """row_start as contiguous int32 (num_sh + 1 rows), checked to fit."""
    rs = np.asarray(row_start)
    if rs.ndim != 1 or rs.size < 1:
        raise ValueError("row_start must be 1-D with num_sh + 1 entries")
    if rs.dtype != np.int32:
        if int(rs.min()) < 0 or int(rs.max()) > 2 ** 31 - 1:
            raise ValueError("row_start entries must lie in [0, 2^31)")
        rs = rs.astype(np.int32)
    return np.ascontiguousarray(rs)


def auto_rows_per_item(row_start: np.ndarray, num_cus: int, slots_per_cu: int = 1) -> int:
    """Rows per work item (library routine sphkv_work_rows_per_item).  When
    one item per CU can cover every (seq, head) range, the smallest row count
    whose item total fits num_cus * slots_per_cu (one workgroup per CU, all
    running at once; at least 8 rows).  When there are more ranges than that
    (each needs an item of its own), about four smaller items per CU, which
    the dispatcher balances as CUs free up."""
    rs = _row_start32(row_start)
    r = load().sphkv_work_rows_per_item(rs.ctypes.data, rs.size - 1, int(num_cus), int(slots_per_cu))
    check(min(r, 0), "sphkv_work_rows_per_item")
    return int(r)


def _work_fill(rs: np.ndarray, rows_per_item: int, interleave: bool, buf_ptr: int, head: int, cap: int) -> int:
    """Fill work_start at buf_ptr and the work rows `head` int32 further on."""
    n = load().sphkv_work_fill(rs.ctypes.data, rs.size - 1, int(rows_per_item), int(bool(interleave)),
                               buf_ptr + 4 * head, cap, buf_ptr)
    check(min(n, 0), "sphkv_work_fill")
    return int(n)


def _work_capacity(rs: np.ndarray, rows_per_item: int) -> int:
    # sum_i max(1, ceil(len_i / r)) <= num_sh + floor(total / r)
    if rows_per_item < 1:
        raise ValueError("rows_per_item must be >= 1")
    return rs.size - 1 + (int(rs[-1]) - int(rs[0])) // int(rows_per_item)


def make_work(row_start: np.ndarray, rows_per_item: int = ROWS_PER_ITEM, interleave: bool = True):
    """Split each (seq, head) row range [b, e) into n = ceil((e - b) /
    rows_per_item) items of <= rows_per_item rows (an empty range gets one
    empty item: its output is still written); library routine
    sphkv_work_fill.  Returns (work int32 [n_items, 4] = (sh, first_row,
    end_row, stride), work_start int32 [num_sh + 1]).

    interleave (default): item i takes rows b + i, b + i + n, ... -- a head's
    rows are grouped by tier, so contiguous items would each hold one tier and
    run at that tier's cost (dense pages load 4 KB of K more); interleaved
    items all hold the head's tier mix.  Otherwise items are contiguous
    ranges (stride 1)."""
    rs = _row_start32(row_start)
    cap = _work_capacity(rs, rows_per_item)
    head = rs.size
    buf = np.empty(head + 4 * max(cap, 1), np.int32)
    n = _work_fill(rs, rows_per_item, interleave, buf.ctypes.data, head, cap)
    return buf[head:head + 4 * n].reshape(-1, 4).copy(), buf[:head].copy()


def _work_device(row_start, rows_per_item: int, dev) -> Tuple[torch.Tensor, torch.Tensor]:
    """The interleaved work list and its per-range starts on the device:
    filled in pinned host memory and uploaded without a host wait (torch's
    pinned-memory cache keeps the buffer until the copy has run)."""
    rs = _row_start32(row_start)
    cap = _work_capacity(rs, rows_per_item)
    head = (rs.size + 3) & ~3              # work_start, padded: the work rows start 16-byte aligned
    buf = torch.empty(head + 4 * max(cap, 1), dtype=torch.int32, pin_memory=True)
    n = _work_fill(rs, rows_per_item, True, buf.data_ptr(), head, cap)
    d = buf[:head + 4 * n].to(dev, non_blocking=True)
    return d[head:].view(-1, 4), d[:rs.size]


def validate_plan(plan: fmt.PagePlan) -> None:
    """Host-side checks of a plan's pointer table against the kernels' needs."""
    pt = plan.ptable.astype(np.int64)
    if plan.page_size != 16:
        raise ValueError("page_size must be 16")
    if (plan.count < 0).any() or (plan.count > plan.page_size).any():
        raise ValueError("page counts must be in [0, page_size]")
    for tid in np.unique(plan.tier):
        m = plan.tier == tid
        n = plan.count[m].astype(np.int64)
        if int(tid) == fmt.DENSE_TIER_ID:
            end = pt[m, 1] + n * plan.dh * 2
            if (pt[m, 1] % 16).any():
                raise ValueError("dense page payloads must be 16-byte aligned")
        elif int(tid) in fmt.TIER_GEOMETRY:
            g, b = fmt.TIER_GEOMETRY[int(tid)]
            G = plan.dh // g
            end = pt[m, 2] + n * G
            if (pt[m, 1] != pt[m, 0] + fmt.HEADER_BYTES + 4 * G).any() or \
               (pt[m, 2] != pt[m, 1] + (n * G * b + 7) // 8).any():
                raise ValueError("pointer-table theta/radius offsets disagree with the page layout")
            if ((pt[m, 2] - (pt[m, 0] & ~15)) + n * G > 512).any():
                raise ValueError("compressed page sections must lie within 512 bytes of the page's 16-byte line")
        else:
            raise ValueError(f"unknown tier id {int(tid)}")
        if (pt[m, 0] % 4).any():
            raise ValueError("page offsets must be 4-byte aligned")
        if (pt[m, 0] < 0).any() or (end > plan.pages_bytes).any():
            raise ValueError("page extends beyond the byte pool")
    if (plan.vslot < 0).any() or (plan.vslot >= plan.num_vpages).any():
        raise ValueError("vslot out of range")


@dataclass
class PagedPool:
    """Device-resident paged KV of one layer: byte pool, pointer table,
    positions, dim-major V pages, per-tier codebooks and the decode work
    list."""
    plan: fmt.PagePlan
    pages: torch.Tensor        # uint8 [pages_bytes]
    ptable: torch.Tensor       # int32 [P, 3]
    vslot: torch.Tensor        # int32 [P]
    positions: torch.Tensor    # int32 [P, 16]
    v_pool: torch.Tensor       # fp16 [num_vpages, 16 * dh] (dim-major pages: [dh][16])
    codebooks: Dict[int, torch.Tensor]   # tier -> fp32 [num_kv, G, C, g]
    work: torch.Tensor         # int32 [n_items, 4] (sh, first_row, end_row, stride)
    work_start: torch.Tensor   # int32 [num_seqs*num_kv + 1]
    tier: torch.Tensor         # int32 [P]
    count: torch.Tensor        # int32 [P]
    seq_head: torch.Tensor     # int32 [P]

    @property
    def device(self):
        return self.pages.device

    @property
    def num_items(self) -> int:
        return int(self.work.shape[0])

    @staticmethod
    def allocate(plan: fmt.PagePlan, codebooks: Dict[int, np.ndarray], device="cuda",
                 rows_per_item: Optional[int] = None) -> "PagedPool":
        validate_plan(plan)
        dev = torch.device(device)
        if rows_per_item is None:
            rows_per_item = auto_rows_per_item(plan.row_start, torch.cuda.get_device_properties(dev).multi_processor_count)
        work, work_start = _work_device(plan.row_start, rows_per_item, dev)
        cbs = {int(t): torch.as_tensor(np.ascontiguousarray(c, np.float32), device=dev)
               for t, c in codebooks.items()}
        for tid in np.unique(plan.tier):
            tid = int(tid)
            if tid != fmt.DENSE_TIER_ID and tid not in cbs:
                raise ValueError(f"no codebook for tier {tid}")
        for tid, c in cbs.items():
            g, b = fmt.TIER_GEOMETRY[tid]
            want = (plan.num_kv, plan.dh // g, 2 ** b, g)
            if tuple(c.shape) != want:
                raise ValueError(f"tier {tid} codebook shape {tuple(c.shape)} != {want}")
        return PagedPool(
            plan=plan,
            pages=torch.zeros(plan.pages_bytes, dtype=torch.uint8, device=dev),
            ptable=torch.as_tensor(plan.ptable, device=dev),
            vslot=torch.as_tensor(plan.vslot, device=dev),
            positions=torch.as_tensor(plan.positions, device=dev),
            v_pool=torch.zeros((plan.num_vpages, plan.page_size * plan.dh), dtype=torch.float16, device=dev),
            codebooks=cbs,
            work=work, work_start=work_start,
            tier=torch.as_tensor(plan.tier, device=dev),
            count=torch.as_tensor(plan.count, device=dev),
            seq_head=torch.as_tensor(plan.seq_head, device=dev),
        )

    @staticmethod
    def allocate_device(plan: "DevicePlan", codebooks: Dict[int, np.ndarray], device="cuda",
                        rows_per_item: Optional[int] = None) -> "PagedPool":
        """A pool over a plan built on the GPU (plan_pages_gpu): the plan's
        device arrays are used in place; its layout holds by construction.
        Codebooks may be given as resident fp32 tensors (used in place)."""
        dev = torch.device(device)
        if rows_per_item is None:
            rows_per_item = auto_rows_per_item(plan.row_start, torch.cuda.get_device_properties(dev).multi_processor_count)
        work, work_start = _work_device(plan.row_start, rows_per_item, dev)
        cbs = {}
        for t, c in codebooks.items():
            if isinstance(c, torch.Tensor) and c.device == dev and c.dtype == torch.float32 and c.is_contiguous():
                cbs[int(t)] = c                       # already resident: used in place
            else:
                cbs[int(t)] = torch.as_tensor(np.ascontiguousarray(np.asarray(c), np.float32), device=dev)
        for tid, c in cbs.items():
            g, b = fmt.TIER_GEOMETRY[tid]
            if tuple(c.shape) != (plan.num_kv, plan.dh // g, 2 ** b, g):
                raise ValueError(f"tier {tid} codebook shape {tuple(c.shape)}")
        # every V slot of every page is written by encode_pages (zeros past a page's tokens)
        return PagedPool(
            plan=plan, pages=torch.zeros(plan.pages_bytes, dtype=torch.uint8, device=dev), ptable=plan.ptable,
            vslot=plan.vslot, positions=plan.positions,
            v_pool=torch.empty((plan.num_vpages, plan.page_size * plan.dh), dtype=torch.float16, device=dev),
            codebooks=cbs, work=work, work_start=work_start,
            tier=plan.tier, count=plan.count, seq_head=plan.seq_head)

    def cb_ptrs(self):
        return tuple(_ptr(self.codebooks.get(t)) for t in (1, 2, 3))

    def workspace_bytes(self, gqa: int) -> int:
        n = load().sphkv_decode_paged_workspace_bytes(self.num_items, gqa, self.plan.dh)
        if n < 0:
            raise ValueError("bad gqa / dh for the decode workspace")
        return int(n)


def encode_pages(pool: PagedPool, k: torch.Tensor, v: torch.Tensor, src_rows: torch.Tensor,
                 r_out: Optional[torch.Tensor] = None, code_out: Optional[torch.Tensor] = None) -> None:
    """Fused encode + bitpack of every page of the pool's plan (GPU).
    k: [rows, dh] fp16 or fp32; v: [rows, dh] fp16; src_rows int64 [P, 16]."""
    plan = pool.plan
    dev = pool.device
    if k.dtype not in (torch.float16, torch.float32):
        raise TypeError("k must be fp16 or fp32")
    _need(k, k.dtype, "k", dev)
    _need(v, torch.float16, "v", dev)
    _need(src_rows, torch.int64, "src_rows", dev)
    if k.dim() != 2 or k.shape[1] != plan.dh or v.shape != k.shape:
        raise ValueError("k and v must be [rows, dh]")
    if tuple(src_rows.shape) != (plan.num_rows, plan.page_size):
        raise ValueError("src_rows must be [P, page_size]")
    for t, name in ((r_out, "r_out"), (code_out, "code_out")):
        if t is not None:
            _need(t, torch.float32 if name == "r_out" else torch.int32, name, dev)
            if tuple(t.shape) != (plan.num_rows, plan.page_size, plan.dh // 16):
                raise ValueError(f"{name} must be [P, page_size, dh/16]")
    c1, c2, c3 = pool.cb_ptrs()
    rc = load().sphkv_encode_pages(
        k.data_ptr(), 1 if k.dtype == torch.float32 else 0, v.data_ptr(), k.shape[0],
        src_rows.data_ptr(), pool.tier.data_ptr(), pool.count.data_ptr(), pool.ptable.data_ptr(),
        pool.vslot.data_ptr(), pool.seq_head.data_ptr(), plan.num_rows, plan.num_kv,
        c1, c2, c3, pool.pages.data_ptr(), plan.pages_bytes, pool.v_pool.data_ptr(), plan.num_vpages,
        _ptr(r_out), _ptr(code_out), plan.dh, plan.page_size, _stream())
    check(rc, "sphkv_encode_pages")


class CodesAll:
    """The all-tier re-encode of every token (_codes_all,
    spherical_kv_pipeline.py:1536-1553) for one token layout, with the batch's
    sequences in place of the reference's layers: built once per layout (the
    page list of 16 consecutive tokens per (seq, head, tier) and the output
    buffers on the device), then called per K (sphkv_encode_codes).  The
    tokens of (seq s, head h) are K rows row_base[s*num_kv + h] + 0 .. L_s - 1;
    `tiers` are the tier ids encoded (those with a codebook)."""

    def __init__(self, row_base, lengths, num_kv: int, dh: int, tiers, device):
        self.lengths = [int(x) for x in lengths]
        self.num_kv, self.dh, self.tiers, self.device = num_kv, dh, list(tiers), device
        base = np.asarray(row_base, np.int64)
        num_sh = len(self.lengths) * num_kv
        if base.shape != (num_sh,):
            raise ValueError("row_base needs one entry per (seq, kv head)")
        sh_len = np.repeat(np.asarray(self.lengths, np.int64), num_kv)
        pages_per_sh = (sh_len + 15) // 16
        self.P_t = P_t = int(pages_per_sh.sum())                 # pages per tier
        sh_of_page = np.repeat(np.arange(num_sh), pages_per_sh)
        self.first = np.cumsum(pages_per_sh) - pages_per_sh      # first page of each (seq, head)
        tok0 = (np.arange(P_t) - self.first[sh_of_page]) * 16
        count = np.minimum(sh_len[sh_of_page] - tok0, 16)
        slot = np.arange(16)
        src = np.where(slot[None, :] < count[:, None], base[sh_of_page][:, None] + tok0[:, None] + slot[None, :], -1)
        nt = len(self.tiers)
        self.P = P_t * nt

        def dev(x, dt):
            return torch.from_numpy(np.ascontiguousarray(np.concatenate([x] * nt), dtype=dt)).to(device)

        self.src, self.count = dev(src, np.int64), dev(count, np.int32)
        self.order_n, self.seq_head = dev(sh_len[sh_of_page], np.int32), dev(sh_of_page, np.int32)
        self.tier = torch.from_numpy(np.repeat(np.asarray(self.tiers, np.int32), P_t)).to(device)
        self.r = torch.empty((self.P, 16, dh // 16), dtype=torch.float32, device=device)
        self.codes = torch.empty((self.P, 16, dh // 16), dtype=torch.int32, device=device)

    def launch(self, k: torch.Tensor, codebooks: Dict[int, torch.Tensor]) -> None:
        """Encode into the output buffers (asynchronous, current stream)."""
        if k.dtype not in (torch.float16, torch.float32) or k.dim() != 2 or k.shape[1] != self.dh:
            raise TypeError(f"k must be fp16 or fp32 [rows, {self.dh}]")
        _need(k, k.dtype, "k", self.device)
        cb = [codebooks.get(t) for t in (1, 2, 3)]
        for t in self.tiers:
            if cb[t - 1] is None:
                raise ValueError(f"no codebook for tier {t}")
        for t in cb:
            if t is not None:
                _need(t, torch.float32, "codebook", self.device)
        if self.P:
            rc = load().sphkv_encode_codes(
                k.data_ptr(), 1 if k.dtype == torch.float32 else 0, k.shape[0], self.src.data_ptr(),
                self.tier.data_ptr(), self.count.data_ptr(), self.order_n.data_ptr(), self.seq_head.data_ptr(),
                self.P, self.num_kv, *[_ptr(t) for t in cb], self.r.data_ptr(), self.codes.data_ptr(), self.dh, 16,
                _stream())
            check(rc, "sphkv_encode_codes")

    def result(self) -> Dict[Tuple[int, int], Dict[int, Tuple[torch.Tensor, torch.Tensor]]]:
        """{(s, h): {tier: (r fp32 [L_s, G], codes int32 [L_s, G])}}: views of the
        output buffers (valid until the next launch)."""
        out: Dict[Tuple[int, int], Dict[int, Tuple[torch.Tensor, torch.Tensor]]] = {}
        for i, t in enumerate(self.tiers):
            G = self.dh // (32 if t == 3 else 16)
            r_t = self.r[i * self.P_t:(i + 1) * self.P_t, :, :G].reshape(-1, G)
            c_t = self.codes[i * self.P_t:(i + 1) * self.P_t, :, :G].reshape(-1, G)
            for sh in range(len(self.lengths) * self.num_kv):
                s, h = divmod(sh, self.num_kv)
                a0 = int(self.first[sh]) * 16
                out.setdefault((s, h), {})[t] = (r_t[a0:a0 + self.lengths[s]], c_t[a0:a0 + self.lengths[s]])
        return out


def encode_codes_all(k: torch.Tensor, row_base, lengths, num_kv: int, codebooks: Dict[int, torch.Tensor]
                     ) -> Dict[Tuple[int, int], Dict[int, Tuple[torch.Tensor, torch.Tensor]]]:
    """Every token of every (sequence, kv head) encoded at every tier that has
    a codebook (see CodesAll): {(s, h): {tier: (r fp32 [L_s, G], codes int32
    [L_s, G])}} on the device, bit-exact with one _encode_keys_with_codebooks
    call (spherical_kv_pipeline.py:1130-1144) over the L_s tokens.
    codebooks[tier]: [num_kv, G, C, g] fp32 on the device."""
    ca = CodesAll(row_base, lengths, num_kv, k.shape[1], [t for t in (1, 2, 3) if codebooks.get(t) is not None],
                  k.device)
    ca.launch(k, codebooks)
    return ca.result()


def _decode_workspace(pool: PagedPool, gqa: int, workspace: Optional[torch.Tensor]) -> torch.Tensor:
    """A caller's workspace, or a new zeroed one (its trailing status words
    must start at zero)."""
    wsb = pool.workspace_bytes(gqa)
    if workspace is None:
        workspace = torch.zeros(max(wsb, 4), dtype=torch.uint8, device=pool.device)
    _need(workspace, torch.uint8, "workspace", pool.device)
    if workspace.numel() < wsb:
        raise ValueError(f"workspace needs {wsb} bytes, got {workspace.numel()}")
    return workspace


def _check_q(pool: PagedPool, q: torch.Tensor, gqa: int) -> None:
    plan = pool.plan
    _need(q, torch.float16, "q", pool.device)
    want = (plan.num_seqs, plan.num_kv * gqa, plan.dh)
    if tuple(q.shape) != want:
        raise ValueError(f"q must be {want}, got {tuple(q.shape)}")


def decode_paged(pool: PagedPool, q: torch.Tensor, gqa: int, rope_theta: float,
                 sm_scale: Optional[float] = None, out: Optional[torch.Tensor] = None,
                 workspace: Optional[torch.Tensor] = None, check: bool = False) -> torch.Tensor:
    """Angle-domain paged attention decode.  q fp16 [num_seqs, num_kv*gqa, dh]
    -> out fp16 of the same shape.  check=True waits for the decode and raises
    SphkvError if it skipped malformed pointer-table rows or pages
    (sphkv_decode_paged_checked); the default call is asynchronous and leaves
    that count in the workspace (decode_status)."""
    plan = pool.plan
    _check_q(pool, q, gqa)
    if out is None:
        out = torch.empty_like(q)
    _need(out, torch.float16, "out", pool.device)
    if out.shape != q.shape:
        raise ValueError("out must match q")
    workspace = _decode_workspace(pool, gqa, workspace)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(plan.dh)
    c1, c2, c3 = pool.cb_ptrs()
    lib = load()
    fn, name = ((lib.sphkv_decode_paged_checked, "sphkv_decode_paged_checked") if check
                else (lib.sphkv_decode_paged, "sphkv_decode_paged"))
    rc = fn(
        pool.pages.data_ptr(), plan.pages_bytes, pool.ptable.data_ptr(), pool.vslot.data_ptr(),
        pool.positions.data_ptr(), plan.num_rows, pool.v_pool.data_ptr(), plan.num_vpages,
        c1, c2, c3, pool.work.data_ptr(), pool.num_items, pool.work_start.data_ptr(),
        plan.num_seqs, plan.num_kv, gqa, q.data_ptr(), out.data_ptr(), workspace.data_ptr(),
        workspace.numel(), plan.dh, plan.page_size, float(sm_scale), float(rope_theta), _stream())
    _check_rc(rc, name)
    return out


class DecodeRunner:
    """decode_paged bound to one pool (sphkv_decode_plan): the pool's
    pointers, gqa, RoPE base, scale and workspace are checked once here, and
    each call is one ctypes call of four arguments.  Holds the pool and the
    workspace; calls that share the workspace must not overlap on the device.

    runner(q, out) checks q and out like decode_paged and returns out;
    runner.raw() returns fn(q_ptr, out_ptr) over raw device addresses, bound
    to the stream current when raw() is called (no checks: the serving-loop
    form)."""

    def __init__(self, pool: PagedPool, gqa: int, rope_theta: float, sm_scale: Optional[float] = None,
                 workspace: Optional[torch.Tensor] = None):
        import ctypes
        plan = pool.plan
        self.pool, self.gqa, self.rope_theta = pool, int(gqa), float(rope_theta)
        self.workspace = _decode_workspace(pool, gqa, workspace)
        self.sm_scale = float(1.0 / math.sqrt(plan.dh) if sm_scale is None else sm_scale)
        self._plan = None
        lib = load()
        c1, c2, c3 = pool.cb_ptrs()
        h = ctypes.c_void_p()
        rc = lib.sphkv_decode_plan_create(
            pool.pages.data_ptr(), plan.pages_bytes, pool.ptable.data_ptr(), pool.vslot.data_ptr(),
            pool.positions.data_ptr(), plan.num_rows, pool.v_pool.data_ptr(), plan.num_vpages, c1, c2, c3,
            pool.work.data_ptr(), pool.num_items, pool.work_start.data_ptr(), plan.num_seqs, plan.num_kv,
            self.gqa, self.workspace.data_ptr(), self.workspace.numel(), plan.dh, plan.page_size, self.sm_scale,
            self.rope_theta, ctypes.byref(h))
        check(rc, "sphkv_decode_plan_create")
        self._plan = h.value
        self._run = lib.sphkv_decode_plan_run
        self._pages, self._v_pool = pool.pages, pool.v_pool

    def __call__(self, q: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        if self.pool.pages is not self._pages or self.pool.v_pool is not self._v_pool:
            raise ValueError("the pool's byte pool or V pool was replaced after the runner was bound")
        _check_q(self.pool, q, self.gqa)
        if out is None:
            out = torch.empty_like(q)
        _need(out, torch.float16, "out", self.pool.device)
        if out.shape != q.shape:
            raise ValueError("out must match q")
        check(self._run(self._plan, q.data_ptr(), out.data_ptr(), _stream()), "sphkv_decode_plan_run")
        return out

    def raw(self):
        run, stream, owner = self._run, _stream(), self

        def fn(q_ptr: int, out_ptr: int) -> None:
            # the closure holds the runner: its plan lives as long as fn
            rc = run(owner._plan, q_ptr, out_ptr, stream)
            if rc:
                check(rc, "sphkv_decode_plan_run")
        return fn

    def __del__(self):
        try:
            if self._plan is not None:
                load().sphkv_decode_plan_destroy(self._plan)
        except Exception:
            pass


def decode_status(pool: PagedPool, workspace: torch.Tensor, gqa: int) -> int:
    """Malformed rows / pages skipped by the last merged decode on this
    workspace (waits for the current stream)."""
    import ctypes
    n = ctypes.c_int32(0)
    rc = load().sphkv_decode_paged_status(workspace.data_ptr(), workspace.numel(), pool.num_items, gqa,
                                          pool.plan.dh, ctypes.byref(n), _stream())
    check(rc, "sphkv_decode_paged_status")
    return int(n.value)


def decode_paged_partials(pool: PagedPool, q: torch.Tensor, gqa: int, rope_theta: float,
                          workspace: torch.Tensor, sm_scale: Optional[float] = None) -> torch.Tensor:
    """First phase of decode_paged: one (m, l, acc) partial per work item into
    `workspace` (fp32 [num_items, 16 + gqa*dh] viewed as bytes); returns the
    fp32 view of the partials."""
    plan = pool.plan
    _check_q(pool, q, gqa)
    workspace = _decode_workspace(pool, gqa, workspace)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(plan.dh)
    c1, c2, c3 = pool.cb_ptrs()
    rc = load().sphkv_decode_paged_partials(
        pool.pages.data_ptr(), plan.pages_bytes, pool.ptable.data_ptr(), pool.vslot.data_ptr(),
        pool.positions.data_ptr(), plan.num_rows, pool.v_pool.data_ptr(), plan.num_vpages,
        c1, c2, c3, pool.work.data_ptr(), pool.num_items, pool.work_start.data_ptr(),
        plan.num_seqs, plan.num_kv, gqa, q.data_ptr(), workspace.data_ptr(),
        workspace.numel(), plan.dh, plan.page_size, float(sm_scale), float(rope_theta), _stream())
    check(rc, "sphkv_decode_paged_partials")
    n = pool.num_items * (16 + gqa * plan.dh)
    return workspace[:4 * n].view(torch.float32).view(pool.num_items, 16 + gqa * plan.dh)


def merge_partials(pool: PagedPool, workspace: torch.Tensor, gqa: int,
                   out: torch.Tensor) -> torch.Tensor:
    """Second phase of decode_paged: log-sum-exp merge of the partials in
    `workspace` into out fp16 [num_seqs, num_kv*gqa, dh]."""
    plan = pool.plan
    _need(out, torch.float16, "out", pool.device)
    if tuple(out.shape) != (plan.num_seqs, plan.num_kv * gqa, plan.dh):
        raise ValueError("out has the wrong shape")
    workspace = _decode_workspace(pool, gqa, workspace)
    rc = load().sphkv_decode_merge_partials(
        workspace.data_ptr(), workspace.numel(), pool.num_items, pool.work_start.data_ptr(),
        plan.num_seqs, plan.num_kv, gqa, plan.dh, out.data_ptr(), _stream())
    check(rc, "sphkv_decode_merge_partials")
    return out


TAIL_SLOTS = 16          # staged tokens + the new one: one decode page


def tail_slot_bytes(dh: int) -> int:
    """Bytes of one decode-page slot: a 16-token tier-3 page, 16-byte aligned."""
    return (fmt.page_nbytes(3, TAIL_SLOTS, dh) + 15) & ~15


_TAILS: "weakref.WeakValueDictionary[int, DecodeTail]" = None     # id(pool) -> its attached tail


class DecodeTail:
    """Decode-time state of a pool for full reference decode steps
    (_compressed_head_attention_batched + _append_decode_kv,
    spherical_kv_pipeline.py:2057-2475) of one layer (gqa, RoPE theta and
    sm_scale fixed): per (sequence, kv head) the staged tokens (tier-3 codes,
    fp32 radii, fp16 V, positions; at most 15), room for `capacity` decode
    pages in the pool, and the decode-time pointer table, positions, V slots
    and work list in which each (seq, head)'s reserved rows follow its
    prefill rows (sphkv_tail_relayout).  A flush writes the page, its
    positions and V, and extends that (seq, head)'s work items by one row, all
    on the device.

    The static arguments are bound once in a C step plan
    (sphkv_step_plan_create), which also keeps the host's mirror of the
    staged / flushed counts and refuses a step that would need a decode page
    past `capacity`.  Attaching grows the pool's byte pool and V pool (copies
    once) when they have no room for the decode pages."""

    def __init__(self, pool: "PagedPool", gqa: int, rope_theta: float, capacity: int = 64,
                 sm_scale: Optional[float] = None, rows_per_item: Optional[int] = None):
        import ctypes
        plan = pool.plan
        dev = pool.device
        if capacity < 0:
            raise ValueError("capacity must be >= 0")
        if pool.codebooks.get(3) is None:
            raise ValueError("decode steps need the tier-3 codebook (decode tokens are tier 3)")
        global _TAILS
        if _TAILS is None:
            _TAILS = weakref.WeakValueDictionary()
        other = _TAILS.get(id(pool))
        if other is not None and other.pool is pool:
            # a second tail would share (or reallocate) the decode-page region
            raise ValueError("this pool already has a DecodeTail")
        self.pool, self.capacity, self.gqa, self.rope_theta = pool, int(capacity), int(gqa), float(rope_theta)
        self.sm_scale = float(1.0 / math.sqrt(plan.dh) if sm_scale is None else sm_scale)
        self.num_sh = num_sh = plan.num_seqs * plan.num_kv
        dh = plan.dh
        G3 = dh // 32
        slot = tail_slot_bytes(dh)
        nres = num_sh * self.capacity
        # decode pages after the prefill pool's bytes and V pages
        self.dec_byte0 = (plan.pages_bytes + 15) & ~15
        self.dec_vpage0 = plan.num_vpages
        need_b, need_v = self.dec_byte0 + nres * slot, plan.num_vpages + nres
        if pool.pages.numel() < need_b:
            grown = torch.zeros(need_b, dtype=torch.uint8, device=dev)
            grown[:pool.pages.numel()].copy_(pool.pages)
            pool.pages = grown
        if pool.v_pool.shape[0] < need_v:
            grown = torch.zeros((need_v, pool.v_pool.shape[1]), dtype=torch.float16, device=dev)
            grown[:pool.v_pool.shape[0]].copy_(pool.v_pool)
            pool.v_pool = grown
        self.pages_bytes = int(pool.pages.numel())
        self.num_vpages = int(pool.v_pool.shape[0])
        self._pages, self._v_pool = pool.pages, pool.v_pool          # the storage the step plan binds
        _TAILS[id(pool)] = self
        # decode-time table: prefill rows of sh shifted by sh * capacity, then sh's reserved rows
        self.num_rows = plan.num_rows + nres
        rs = _row_start32(plan.row_start)
        rs_dev = torch.as_tensor(rs, device=dev)
        self.ptable = torch.empty((max(self.num_rows, 1), 3), dtype=torch.int32, device=dev)
        self.vslot = torch.empty(max(self.num_rows, 1), dtype=torch.int32, device=dev)
        self.positions = torch.empty((max(self.num_rows, 1), 16), dtype=torch.int32, device=dev)
        lib = load()
        rc = lib.sphkv_tail_relayout(rs_dev.data_ptr(), num_sh, plan.num_rows, pool.ptable.data_ptr(),
                                     pool.vslot.data_ptr(), pool.positions.data_ptr(), self.capacity,
                                     self.dec_byte0, self.dec_vpage0, dh, self.ptable.data_ptr(),
                                     self.vslot.data_ptr(), self.positions.data_ptr(), _stream())
        check(rc, "sphkv_tail_relayout")
        # the work list over the prefill rows, in the decode-time row numbering
        if rows_per_item is None:
            rows_per_item = auto_rows_per_item(rs, torch.cuda.get_device_properties(dev).multi_processor_count)
        w, ws = make_work(rs, rows_per_item)
        shift = w[:, 0].astype(np.int64) * self.capacity
        w[:, 1] = (w[:, 1] + shift).astype(np.int32)
        w[:, 2] = (w[:, 2] + shift).astype(np.int32)
        self._work0 = np.ascontiguousarray(w)
        self.work = torch.as_tensor(self._work0, device=dev)
        self.work_start = torch.as_tensor(ws, device=dev)
        self.num_items = int(w.shape[0])
        # staging
        self.stg_r = torch.zeros((num_sh, TAIL_SLOTS, G3), dtype=torch.float32, device=dev)
        self.stg_code = torch.zeros((num_sh, TAIL_SLOTS, G3), dtype=torch.int32, device=dev)
        self.stg_v = torch.zeros((num_sh, TAIL_SLOTS, dh), dtype=torch.float16, device=dev)
        self.stg_pos = torch.zeros((num_sh, TAIL_SLOTS), dtype=torch.int32, device=dev)
        self.state = torch.zeros((num_sh, 2, 4), dtype=torch.int32, device=dev)
        n = lib.sphkv_decode_paged_workspace_bytes(self.num_items, self.gqa, dh)
        if n < 0:
            raise ValueError("bad gqa / dh for the decode workspace")
        self.workspace = torch.zeros(max(int(n), 4), dtype=torch.uint8, device=dev)
        self._plan = None
        self._bind(0, 0, 0)

    def _bind(self, staged: int, flushed: int, parity: int) -> None:
        import ctypes
        lib = load()
        if self._plan is not None:
            lib.sphkv_step_plan_destroy(self._plan)
            self._plan = None
        pool, plan = self.pool, self.pool.plan
        c1, c2, c3 = pool.cb_ptrs()
        h = ctypes.c_void_p()
        rc = lib.sphkv_step_plan_create(
            pool.pages.data_ptr(), self.pages_bytes, self.ptable.data_ptr(), self.vslot.data_ptr(),
            self.positions.data_ptr(), self.num_rows, pool.v_pool.data_ptr(), self.num_vpages, c1, c2, c3,
            self.work.data_ptr(), self.num_items, self.work_start.data_ptr(), plan.num_seqs, plan.num_kv, self.gqa,
            self.stg_r.data_ptr(), self.stg_code.data_ptr(), self.stg_v.data_ptr(), self.stg_pos.data_ptr(),
            self.state.data_ptr(), self.dec_byte0, self.dec_vpage0, self.capacity, staged, flushed, parity,
            self.workspace.data_ptr(), self.workspace.numel(), plan.dh, plan.page_size, self.sm_scale,
            self.rope_theta, ctypes.byref(h))
        check(rc, "sphkv_step_plan_create")
        self._plan = h.value
        self._run = lib.sphkv_step_plan_run

    def __del__(self):
        try:
            if self._plan is not None:
                load().sphkv_step_plan_destroy(self._plan)
        except Exception:
            pass

    def counts(self) -> Tuple[int, int, int]:
        """(staged tokens, flushed decode pages, step parity) per (seq, head)."""
        import ctypes
        a, b, p = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
        check(load().sphkv_step_plan_counts(self._plan, ctypes.byref(a), ctypes.byref(b), ctypes.byref(p)),
              "sphkv_step_plan_counts")
        return int(a.value), int(b.value), int(p.value)

    @property
    def staged(self) -> int:
        return self.counts()[0]

    @property
    def flushed(self) -> int:
        return self.counts()[1]

    def reset(self) -> None:
        """Empty tail: no staged tokens, no decode pages (the work list's rows
        back to the prefill rows).  Asynchronous, current stream."""
        self.state.zero_()
        self.work.copy_(torch.as_tensor(self._work0), non_blocking=False)
        self._bind(0, 0, 0)

    def runner(self):
        """The fastest call of a step: fn(q_ptr, k_ptr, k_is_fp32, v_ptr, pos_ptr, out_ptr, mode) with raw
        device addresses (mode 1 decode, 2 append, 3 both) on the stream current when runner() is called;
        one ctypes call, no checks of the inputs."""
        run, stream, owner = self._run, _stream(), self

        def fn(q, k, k32, v, pos, out, mode):
            # the closure holds the tail, and reads its current plan (reset()
            # binds a new one)
            check(run(owner._plan, q, k, k32, v, pos, out, mode, stream), "sphkv_step_plan_run")
        return fn

    def _step_inputs(self, k_new: torch.Tensor, v_new: torch.Tensor, cur_pos: torch.Tensor):
        plan, dev = self.pool.plan, self.pool.device
        if k_new.dtype not in (torch.float16, torch.float32):
            raise TypeError("k_new must be fp16 or fp32")
        _need(k_new, k_new.dtype, "k_new", dev)
        _need(v_new, torch.float16, "v_new", dev)
        _need(cur_pos, torch.int32, "cur_pos", dev)
        want = (plan.num_seqs, plan.num_kv, plan.dh)
        if tuple(k_new.shape) != want or tuple(v_new.shape) != want:
            raise ValueError(f"k_new and v_new must be {want}")
        if tuple(cur_pos.shape) != (plan.num_seqs,):
            raise ValueError("cur_pos must be [num_seqs]")

    def _call(self, q, k_new, v_new, cur_pos, out, mode: int) -> None:
        if self.pool.pages is not self._pages or self.pool.v_pool is not self._v_pool:
            raise ValueError("the pool's byte pool or V pool was replaced after the DecodeTail was attached")
        rc = self._run(self._plan, _ptr(q), k_new.data_ptr(), 1 if k_new.dtype == torch.float32 else 0,
                       v_new.data_ptr(), cur_pos.data_ptr(), _ptr(out), mode, _stream())
        if rc != 0:
            msg = load().sphkv_last_error().decode(errors="replace")
            if "no decode-page slot" in msg:
                raise ValueError(msg)
            check(rc, "sphkv_step_plan_run")

    def state_host(self) -> Dict[str, np.ndarray]:
        """Copies of the tail state (waits for the current stream); "state" is
        the copy of the counts the next step reads ([num_sh, 4])."""
        par = self.counts()[2]
        return {"state": self.state[:, par].cpu().numpy(), "stg_r": self.stg_r.cpu().numpy(),
                "stg_code": self.stg_code.cpu().numpy(), "stg_v": self.stg_v.cpu().numpy(),
                "stg_pos": self.stg_pos.cpu().numpy(), "work": self.work.cpu().numpy()}


def decode_step(pool: "PagedPool", tail: DecodeTail, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                cur_pos: torch.Tensor, out: Optional[torch.Tensor] = None, append: bool = True) -> torch.Tensor:
    """One reference decode step on the GPU (sphkv_decode_step through the
    tail's step plan): attention of q fp16 [num_seqs, num_kv*gqa, dh] over the
    prefill pages, the flushed decode pages, the staged tokens and the new
    token (k_new pre-RoPE [num_seqs, num_kv, dh] fp16/fp32, v_new fp16,
    cur_pos int32 [num_seqs]); then, with append, the new token is staged
    (and a full page flushed).  Returns out fp16, q's shape."""
    if tail.pool is not pool:
        raise ValueError("the tail belongs to another pool")
    _check_q(pool, q, tail.gqa)
    tail._step_inputs(k_new, v_new, cur_pos)
    if out is None:
        out = torch.empty_like(q)
    _need(out, torch.float16, "out", pool.device)
    if out.shape != q.shape:
        raise ValueError("out must match q")
    tail._call(q, k_new, v_new, cur_pos, out, 3 if append else 1)
    return out


def decode_append(pool: "PagedPool", tail: DecodeTail, k_new: torch.Tensor, v_new: torch.Tensor,
                  cur_pos: torch.Tensor) -> None:
    """_append_decode_kv for every (seq, head) (sphkv_decode_append's work,
    through the tail's step plan): stage the new tokens, flushing full pages;
    no attention."""
    if tail.pool is not pool:
        raise ValueError("the tail belongs to another pool")
    tail._step_inputs(k_new, v_new, cur_pos)
    tail._call(None, k_new, v_new, cur_pos, None, 2)


def time_next_decode_kernel(start: "torch.cuda.Event", stop: "torch.cuda.Event") -> None:
    """The next paged-decode kernel launch on this thread records its own
    start and stop in these timing events (kernel-only timestamps,
    sphkv_time_next_decode_kernel)."""
    for e in (start, stop):
        if not e.cuda_event:
            e.record()
    check(load().sphkv_time_next_decode_kernel(start.cuda_event, stop.cuda_event), "sphkv_time_next_decode_kernel")


@dataclass
class DevicePlan:
    """A page plan built on the GPU by plan_pages_gpu.  Per-row arrays stay on
    the device; only the totals and the (seq, head) row ranges come back to
    the host.  Duck-types the fields of sphkv_format.PagePlan that pools and
    kernels use."""
    dh: int
    page_size: int
    num_seqs: int
    num_kv: int
    pages_bytes: int
    num_vpages: int
    rows: int
    row_start: np.ndarray       # [num_seqs*num_kv + 1] int32 (host)
    tier: torch.Tensor          # [P] int32
    count: torch.Tensor         # [P] int32
    ptable: torch.Tensor        # [P, 3] int32
    seq_head: torch.Tensor      # [P] int32
    vslot: torch.Tensor         # [P] int32
    tokens: torch.Tensor        # [P, 16] int64
    positions: torch.Tensor     # [P, 16] int32
    src_rows: Optional[torch.Tensor]   # [P, 16] int64 rows of the K/V matrices, or None

    @property
    def num_rows(self) -> int:
        return self.rows

    def to_host(self) -> fmt.PagePlan:
        return fmt.PagePlan(dh=self.dh, page_size=self.page_size, num_seqs=self.num_seqs, num_kv=self.num_kv,
                            tier=self.tier.cpu().numpy(), count=self.count.cpu().numpy(),
                            tokens=self.tokens.cpu().numpy(), positions=self.positions.cpu().numpy(),
                            seq_head=self.seq_head.cpu().numpy(), row_start=self.row_start.copy(),
                            ptable=self.ptable.cpu().numpy(), vslot=self.vslot.cpu().numpy(),
                            pages_bytes=self.pages_bytes, num_vpages=self.num_vpages)


def plan_pages_gpu(tier_of: torch.Tensor, lens: torch.Tensor, num_kv: int, dh: int,
                   positions: Optional[torch.Tensor] = None, row_base: Optional[torch.Tensor] = None) -> DevicePlan:
    """Device-side equivalent of sphkv_format.plan_pages (logical placement):
    the grouping / sort / chunk / offset steps of _build_per_head_pages
    (spherical_kv_pipeline.py:1146-1228) on the GPU.

    tier_of: uint8 [num_seqs*num_kv, L_max] tier id per token (row s*num_kv+h);
    lens: int32 [num_seqs], each <= L_max; positions: int32 [num_seqs, L_max] or None (token
    index); row_base: int64 [num_seqs*num_kv] K row of each (seq, head)'s
    token 0, or None (no src_rows).  One host synchronisation (the totals)."""
    dev = tier_of.device
    _need(tier_of, torch.uint8, "tier_of", dev)
    _need(lens, torch.int32, "lens", dev)
    if tier_of.dim() != 2 or lens.dim() != 1 or tier_of.shape[0] != lens.shape[0] * num_kv:
        raise ValueError("tier_of must be [num_seqs*num_kv, L_max] and lens [num_seqs]")
    num_seqs, num_sh = int(lens.shape[0]), int(tier_of.shape[0])
    if positions is not None:
        _need(positions, torch.int32, "positions", dev)
        if positions.dim() != 2 or positions.shape[0] != num_seqs or positions.shape[1] < tier_of.shape[1]:
            raise ValueError("positions must be [num_seqs, >= L_max]")
    if row_base is not None:
        _need(row_base, torch.int64, "row_base", dev)
        if tuple(row_base.shape) != (num_sh,):
            raise ValueError("row_base must be [num_seqs*num_kv]")
    lib = load()
    max_len = int(tier_of.shape[1])
    nw = lib.sphkv_plan_pages_work_ints(num_seqs, int(num_kv), max_len)
    if nw < 0:
        raise ValueError("bad planner sizes")
    work = torch.empty(max(nw, 1), dtype=torch.int32, device=dev)
    # totals and row_start in one buffer: phase 1 writes both whole (nothing
    # when there are no sequences), so one copy to the host (the planner's
    # only synchronisation) brings back both
    meta = (torch.empty if num_sh else torch.zeros)(4 + num_sh + 1, dtype=torch.int32, device=dev)
    totals, row_start = meta[:4], meta[4:]
    rc = lib.sphkv_plan_pages_count(tier_of.data_ptr(), tier_of.stride(0), lens.data_ptr(), num_seqs, int(num_kv),
                                    max_len, int(dh), work.data_ptr(), work.numel(), row_start.data_ptr(),
                                    totals.data_ptr(), _stream())
    check(rc, "sphkv_plan_pages_count")
    meta_h = meta.cpu().numpy()
    rows, nbytes, bad, ovf = (int(x) for x in meta_h[:4])
    if bad:
        raise ValueError(f"{bad} tokens carry a tier id outside {{0, 1, 2, 3, 0xFF}}")
    if nbytes < 0 or ovf:
        raise ValueError("a sequence length exceeds tier_of's width, or the byte pool exceeds int32 offsets")
    # the plan's arrays as views of two allocations (int32, int64)
    b32 = torch.empty(rows * 23, dtype=torch.int32, device=dev)
    b64 = torch.empty(rows * (16 if row_base is None else 32), dtype=torch.int64, device=dev)
    out = dict(tier=b32[:rows], count=b32[rows:2 * rows], ptable=b32[2 * rows:5 * rows].view(rows, 3),
               seq_head=b32[5 * rows:6 * rows], vslot=b32[6 * rows:7 * rows],
               positions=b32[7 * rows:].view(rows, 16), tokens=b64[:16 * rows].view(rows, 16),
               src_rows=None if row_base is None else b64[16 * rows:].view(rows, 16))
    rc = lib.sphkv_plan_pages_fill(
        tier_of.data_ptr(), tier_of.stride(0), lens.data_ptr(), _ptr(positions),
        0 if positions is None else positions.stride(0), _ptr(row_base), num_seqs, int(num_kv), max_len, int(dh),
        work.data_ptr(), rows, out["tier"].data_ptr(), out["count"].data_ptr(), out["ptable"].data_ptr(),
        out["seq_head"].data_ptr(), out["vslot"].data_ptr(), out["tokens"].data_ptr(), out["positions"].data_ptr(),
        _ptr(out["src_rows"]), _stream())
    check(rc, "sphkv_plan_pages_fill")
    return DevicePlan(dh=int(dh), page_size=16, num_seqs=num_seqs, num_kv=int(num_kv), pages_bytes=nbytes,
                      num_vpages=rows, rows=rows, row_start=meta_h[4:].copy(), **out)


def build_pool_gpu(wl, device="cuda", rows_per_item: Optional[int] = None, with_codes: bool = False):
    """Allocate a pool for a synthetic workload and encode it on the GPU.
    Returns (pool, r_out, code_out) (the last two None unless with_codes)."""
    pool = PagedPool.allocate(wl.plan, wl.codebooks, device, rows_per_item)
    k = torch.as_tensor(wl.k_rows(), device=pool.device)
    v = torch.as_tensor(wl.v_rows(), device=pool.device)
    src = torch.as_tensor(wl.src_rows(), device=pool.device)
    r_out = code_out = None
    if with_codes:
        shp = (wl.plan.num_rows, wl.plan.page_size, wl.dh // 16)
        r_out = torch.zeros(shp, dtype=torch.float32, device=pool.device)
        code_out = torch.zeros(shp, dtype=torch.int32, device=pool.device)
    encode_pages(pool, k, v, src, r_out, code_out)
    del k, v, src
    return pool, r_out, code_out
