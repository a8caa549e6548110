"""Benchmark of the angle-domain paged decode on one MI355X.

`python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 2]`

A step is one full reference decode step of one layer (all kv heads) for the
workload named in BASELINE.json's metric: config 2, Llama-3.1-8B attention
shape (32 q / 8 kv heads, dh 128), 32K context, 60/30/10 tier mix, randomly
permuted page table: attention over the page-resident context, the tokens
staged since the last decode page and the step's new token in one softmax,
then the new token's append (tier-3 encode, staging, a page flush every 16
steps) -- decode_kernel + decode_tail_kernel through the bound step call
(DecodeTail.runner()).  Inputs are resident in HBM before timing; the
Infinity Cache (256 MB) is defeated by rotating through ROTATE independent
copies of the KV pool (each ~80 MB).  Timing uses HIP events on the stream the
kernels run on (torch's current stream), around exactly K steps; the
roofline object's kernel time is decode_kernel's own start / stop timestamps
(hipExtLaunchKernel) over K more steps, the duration rocprofv3 reports.

Before the W counted warmup steps, every path runs an untimed settle phase
of the same step for at least SETTLE_S seconds: on a fresh process the GPU's
clocks and translation caches take a few hundred steps to reach steady state
(measured: 31.2, 28.8, 28.3 us/step over three consecutive 220-step rounds).

Prints one JSON line (see the "roofline" and "cpu_baseline" objects).

`--path modea` measures the Mode-A (LayerPool) decode instead, on the same
attention shape with unpacked uint8 pools (fused_decode.sphkv_decode);
`--path prefill` measures prefill paging of the same layer on the GPU (device
page plan + fused encode / bitpack / V placement); `--path ragged` measures
fused_decode_ragged (logits only) over the same layer's tier-1 and tier-2
pages, with the caller's RoPE tables fitted once; `--path pages` measures the
page-resident decode alone (decode_kernel + decode_merge_kernel through the
bound DecodeRunner).  The default line is the full decode step above.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "spherical-kv_amd"))

import numpy as np  # noqa: E402
import torch  # noqa: E402

import sphkv_format as fmt  # noqa: E402
import sphkv_ops as ops  # noqa: E402
import sphkv_synth as synth  # noqa: E402

PEAK_HBM_GBPS = 8000.0
METRIC = "µs/decode step + achieved HBM GB/s (compressed KV), 8B shape, 32K ctx, 1 GPU"
# the same measurement on the other decode configs of BASELINE.json (parity
# cases there; bench lines here with their own workload named)
METRICS = {
    1: "µs/decode step + achieved HBM GB/s (compressed KV), 1B shape (32 q / 8 kv, dh 64), 4K ctx, all tier 1, 1 GPU",
    2: METRIC,
    4: "µs/decode step + achieved HBM GB/s (compressed KV), 8B shape, 64 seqs x U[2K, 32K] ctx on a ~1.2M-page "
       "shared pool, 1 GPU",
    5: "µs/decode step + achieved HBM GB/s (compressed KV), 70B shape (64 q / 8 kv), 4 seqs x 131K ctx, 1 GPU",
}
ROTATE = 6
COPY_BYTES = 256 << 20
SETTLE_S = 0.3


def settle(step_fn):
    """Untimed: repeat step_fn(i) until SETTLE_S seconds of wall time have
    passed (synchronising every 50 steps)."""
    t0, i = time.perf_counter(), 0
    while time.perf_counter() - t0 < SETTLE_S:
        for _ in range(50):
            step_fn(i)
            i += 1
        torch.cuda.synchronize()


def calibrate_copies(dev):
    """Four plain device copies of COPY_BYTES (torch copy_): the reference of
    known traffic for the FETCH_SIZE / WRITE_SIZE counters."""
    src = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"[bench] calibration: 4 device copies of {COPY_BYTES} bytes")


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def clone_pool(pool: ops.PagedPool) -> ops.PagedPool:
    """An independent copy of the KV bytes (pages and V) at new addresses."""
    return ops.PagedPool(**{**pool.__dict__, "pages": pool.pages.clone(), "v_pool": pool.v_pool.clone()})


# HBM bytes per decode_kernel launch from rocprofv3 counters on MI355X:
# (FETCH_SIZE * 2 + WRITE_SIZE) KiB per dispatch.  On this part FETCH_SIZE
# reads exactly half of a plain device copy's bytes (256 MiB copy -> 131083
# KiB) and WRITE_SIZE all of them (262144 KiB), hence the factor 2.  Measured
# with `bench.py --calibrate` under rocprofv3 --pmc (summary and commands in
# profiles/decode_config2_hbm_traffic.txt); re-measured when the kernel changes.
TRAFFIC_BYTES = {(2, "default"): 86515541}

# encode_pages_kernel at config 3, from rocprofv3 --pmc on MI355X
# (profiles/encode_config3_counters.txt): VALU instructions per launch (MFMA
# included) and HBM bytes (FETCH_SIZE * 2 + WRITE_SIZE).  The VALU-issue bound
# is that count at one wave64 VALU instruction per 4 cycles on each of the
# 1024 SIMDs at 2.4 GHz.
ENCODE_VALU_INSTS = {3: 7061123}
ENCODE_TRAFFIC_BYTES = {3: 55632656}
# HBM bytes per Mode-A decode (modea_fast_kernel, page_size 16; profiles/
# modea_config2shape_counters.txt) and per fused_decode_ragged step (both
# tiers' ragged_pipe_kernel launches; profiles/ragged_config2_hbm_traffic.txt),
# FETCH_SIZE * 2 + WRITE_SIZE as above.
MODEA_TRAFFIC_BYTES = {16: 80479122}
RAGGED_TRAFFIC_BYTES = {"fit": 13705673, "table": 47988605}   # phases in the kernel / table rows read
# VALU instructions (MFMA included) of both ragged launches of a step with
# fitted tables, SQ_INSTS_VALU from the same profile; the VALU-issue bound as
# for the encode above.
RAGGED_VALU_INSTS = {"fit": 7657312}
SIMDS, CLOCK_HZ = 1024, 2.4e9


def measured_traffic(config, layout):
    v = TRAFFIC_BYTES.get((config, layout))
    return None if v is None else int(v)


def counter_gbps(config, layout, kern_ms):
    """The counters' HBM bytes per launch over the live kernel time (GB/s)."""
    v = measured_traffic(config, layout)
    return None if v is None or kern_ms <= 0 else round(v / (kern_ms * 1e-3) / 1e9, 1)


def host_cpu() -> dict:
    """The host CPU this process runs on: model name, logical CPUs of the
    machine, CPUs in this process's affinity mask, the cgroup CPU quota (if
    any), and `threads` = the CPUs the process can actually use (affinity,
    capped by the quota)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    affinity = len(os.sched_getaffinity(0))
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, per = f.read().split()[:2]
            if q != "max":
                quota = int(q) / int(per)
    except (OSError, ValueError):
        pass
    threads = affinity if quota is None else max(1, min(affinity, int(math.ceil(quota))))
    return {"cpu_model": model, "host_cpus": os.cpu_count(), "affinity_cpus": affinity,
            "cgroup_cpus": quota, "threads": threads}


def cpu_baseline(wl, pool: ops.PagedPool, budget_s: float = 20.0):
    """Reference Mode-B path restated in torch (oracle/torch_port.py), on all
    the host CPUs this process may use, over a bounded sample of the same
    workload: whole kv heads of the config, as many as fit the time budget (at
    least one)."""
    sys.path.insert(0, ROOT)
    from oracle import torch_port
    cpu = host_cpu()
    threads = cpu["threads"]
    torch.set_num_threads(threads)
    pages = pool.pages.cpu().numpy()
    v_pool = pool.v_pool.cpu().numpy()
    cos_t, sin_t = fmt.rope_tables(max(wl.lengths) + 64, wl.dh, wl.rope_theta)
    cos_t, sin_t = torch.from_numpy(cos_t), torch.from_numpy(sin_t)
    times, heads_done = [], 0
    t_start = time.perf_counter()
    for sh in range(wl.plan.num_seqs * wl.plan.num_kv):
        s, h = divmod(sh, wl.plan.num_kv)
        blocks = torch_port.head_blocks(pages, v_pool, wl.plan, sh)
        cbs = {t: torch.from_numpy(c[h]) for t, c in wl.codebooks.items()}
        q = torch.from_numpy(wl.q[s, h * wl.gqa:(h + 1) * wl.gqa].astype(np.float32))
        torch_port.decode_head(q, blocks, cbs, cos_t, sin_t)          # warm-up
        t0 = time.perf_counter()
        torch_port.decode_head(q, blocks, cbs, cos_t, sin_t)
        times.append(time.perf_counter() - t0)
        heads_done += 1
        if time.perf_counter() - t_start > budget_s:
            break
    per_head = float(np.median(times))
    step_us = per_head * wl.plan.num_seqs * wl.plan.num_kv * 1e6
    return {"value": round(step_us, 1), "unit": "µs/decode step (extrapolated from per-head time)",
            "cores": threads, "kind": "port", **{k: v for k, v in cpu.items() if k != "threads"},
            "sample": f"{heads_done} of {wl.plan.num_seqs * wl.plan.num_kv} kv heads of {wl.name}, "
                      f"median per-head time x {wl.plan.num_seqs * wl.plan.num_kv} heads; torch CPU "
                      f"restatement of spherical_kv_pipeline.py:2143-2177,2348,2367"}


def cpu_baseline_prefill(wl, budget_s: float = 20.0):
    """Reference prefill paging restated in torch (oracle/torch_port.py) on all
    the host CPUs this process may use: the reference grouping of the retained
    tokens (oracle/paging.py, spherical_kv_pipeline.py:1156-1190), then per
    16-token chunk the encode (:1136-1144) and page build (pagebuilder.py:8-33)
    of _build_per_head_pages (:1187-1213); dense chunks are header + K bytes.
    (seq, head)s are processed in order until the time budget is spent; the
    layer time is extrapolated by retained tokens."""
    sys.path.insert(0, ROOT)
    from oracle import paging, torch_port
    cpu = host_cpu()
    torch.set_num_threads(cpu["threads"])
    groups = paging.group_pages(paging.retained_tokens(wl.tier_of, wl.num_seqs, wl.num_kv))
    cbs = {t: torch.from_numpy(np.ascontiguousarray(c, np.float32)) for t, c in wl.codebooks.items()}
    total = sum(len(c) for tiers in groups.values() for _, chunks in tiers for c in chunks)
    done, elapsed, heads = 0, 0.0, 0
    for (s, h), tiers in groups.items():
        K, V = wl.head_kv(s, h)
        Kt = torch.from_numpy(K.astype(np.float32))
        t0 = time.perf_counter()
        for tier, chunks in tiers:
            for chunk in chunks:
                ix = torch.as_tensor(chunk, dtype=torch.long)
                if tier == fmt.DENSE_TIER_ID:
                    torch.cat([torch.zeros(8, dtype=torch.uint8), Kt[ix].half().reshape(-1).view(torch.uint8)])
                else:
                    g, b = paging.TIER_GEOMETRY[tier]
                    r, codes = torch_port.encode_chunk(Kt[ix], cbs[tier][h], g, wl.dh // g)
                    torch_port.build_page(r, codes, tier, b)
                _ = V[chunk]                                             # the chunk's V rows
                done += len(chunk)
        elapsed += time.perf_counter() - t0
        heads += 1
        if elapsed > budget_s:
            break
    layer_us = elapsed / max(done, 1) * total * 1e6
    return {"value": round(layer_us, 1), "unit": "µs/layer (extrapolated by retained tokens)",
            "cores": cpu["threads"], "kind": "port", **{k: v for k, v in cpu.items() if k != "threads"},
            "sample": f"{heads} of {len(groups)} (seq, kv head)s, {done} of {total} retained tokens of {wl.name}; "
                      f"torch CPU restatement of spherical_kv_pipeline.py:1136-1144,1156-1213 + "
                      f"pagebuilder.py:8-33 + bitpacking.py:5-29"}


def modea_bytes(w) -> int:
    """Algorithmic HBM bytes of one Mode-A decode: per present logical page
    its theta and radius codes (page_size x G_tier bytes each), r_scales
    (G_tier fp32), fp16 V (page_size x dh) and its two table entries, plus the
    per-(q head, page) (m, l) written to partial_scratch."""
    total = 0
    ps, dh = w["page_size"], w["dh"]
    for h in range(w["num_kv"]):
        for p in range(w["max_blocks"]):
            if w["block_table"][h, p] < 0:
                continue
            Gt = int(w["tier_G"][w["bits_table"][h, p]])
            total += 2 * ps * Gt + 4 * Gt + 2 * ps * dh + 8
    return total + w["q"].shape[0] * w["max_blocks"] * 8


def cpu_baseline_modea(w, budget_s: float = 20.0):
    """The fp64 numpy restatement of decode_kernel.cu:108-246, one kv head at a
    time on one host core, as many heads as fit the budget."""
    sys.path.insert(0, ROOT)
    import oracle
    kvg = w["kv_groups"]
    times, done = [], 0
    t_start = time.perf_counter()
    for h in range(w["num_kv"]):
        t0 = time.perf_counter()
        oracle.decode_mode_a(w["q"][h * kvg:(h + 1) * kvg], w["cb_flat"][h:h + 1], w["tier_G"], w["tier_g"],
                             w["theta"], w["radius"], w["r_scales"], w["v_pool"], w["block_table"][h:h + 1],
                             w["bits_table"][h:h + 1], kvg, w["sm_scale"])
        times.append(time.perf_counter() - t0)
        done += 1
        if time.perf_counter() - t_start > budget_s:
            break
    step_us = float(np.median(times)) * w["num_kv"] * 1e6
    cpu = host_cpu()
    return {"value": round(step_us, 1), "unit": "µs/decode step (extrapolated from per-head time)", "cores": 1,
            "kind": "port", **{k: v for k, v in cpu.items() if k != "threads"}, "sample": f"{done} of {w['num_kv']} kv heads, median per-head time x {w['num_kv']}; "
                                      f"numpy fp64 restatement of decode_kernel.cu:108-246"}


def modea_aux(args, dev, w, d, part):
    """The Mode-A step's companions on the same tables, µs per call (HIP
    events, back-to-back calls): the omega EMA on the decode's (m, l)
    (spherical_kv_pipeline.py:1690-1701), the q_lut build and LUT logits
    (new_fused_decode.sphkv_logits), and the decode-time append of one token
    per kv head (fused_decode.sphkv_encode_append)."""
    import fused_decode
    import new_fused_decode
    import omega_ema
    nq, mb = w["q"].shape[0], w["max_blocks"]
    om = torch.rand((w["num_kv"], mb), device=dev)
    om_out = torch.empty_like(om)
    lut = new_fused_decode.build_q_lut(d["q"], d["cb_flat"], d["tier_G"], d["tier_g"], w["num_kv"], w["kv_groups"],
                                       w["num_tiers"], w["G_max"], w["cb_max"], w["g_max"])
    logits = torch.empty((nq, w["max_ctx"]), dtype=torch.float32, device=dev)
    # append into spare copies of the pools (the decode's stay as they are)
    th, rd, rs, vp = (d[k].clone() for k in ("theta", "radius", "r_scales", "v_pool"))
    G, g = int(w["tier_G"][0]), int(w["tier_g"][0])
    C = int(w["cb_max"])
    dcb = d["cb_flat"][:, 0, :G, :C, :g].contiguous()
    kk = torch.randn((w["num_kv"], w["dh"]), device=dev)
    vv = torch.randn((w["num_kv"], w["dh"]), device=dev)
    pids = torch.arange(w["num_kv"], dtype=torch.int64, device=dev)
    ps = w["page_size"]
    calls = {
        "omega_ema": lambda i: omega_ema.omega_ema(part[..., 0], part[..., 1], om, w["num_kv"], w["kv_groups"], mb,
                                                   0.9, out=om_out),
        "build_q_lut": lambda i: new_fused_decode.build_q_lut(d["q"], d["cb_flat"], d["tier_G"], d["tier_g"],
                                                              w["num_kv"], w["kv_groups"], w["num_tiers"],
                                                              w["G_max"], w["cb_max"], w["g_max"]),
        "sphkv_logits": lambda i: new_fused_decode.sphkv_logits(
            lut, d["theta"], d["radius"], d["r_scales"], d["block_table"], d["bits_table"], d["ctx_lens"], logits,
            nq, w["num_kv"], w["kv_groups"], w["num_tiers"], mb, ps, w["G_max"], w["cb_max"], w["sm_scale"],
            w["max_ctx"]),
        "sphkv_encode_append": lambda i: fused_decode.sphkv_encode_append(
            kk, vv, dcb, th, rd, rs, vp, pids, i % ps, G, g, C, w["G_max"], w["dh"], ps, (i % ps) == 0),
    }
    res = {}
    for name, f in calls.items():
        for i in range(20):
            f(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(100):
            f(i)
        e1.record()
        torch.cuda.synchronize()
        res[name] = round(e0.elapsed_time(e1) * 10.0, 2)       # ms per 100 calls -> us per call
    log(f"[bench] Mode-A companions, us per call: {res}")
    return res


def bench_modea(args, dev):
    import fused_decode
    log(f"[bench] building Mode-A workload (page_size {args.page_size})")
    w = synth.make_modea_workload(seed=2, num_kv=8, kv_groups=4, dh=128, page_size=args.page_size, ctx=32768,
                                  tiers=(1, 2), fracs=(0.6, 0.4))
    names = ("q", "cb_flat", "tier_G", "tier_g", "theta", "radius", "r_scales", "v_pool", "block_table",
             "bits_table", "ctx_lens")
    d = {k: torch.from_numpy(np.ascontiguousarray(w[k])).to(dev) for k in names}
    pools = [(d["theta"], d["radius"], d["r_scales"], d["v_pool"])]
    for _ in range(args.rotate - 1):
        pools.append(tuple(t.clone() for t in pools[0]))
    nq, mb = w["q"].shape[0], w["max_blocks"]
    out = torch.empty((nq, w["dh"]), dtype=torch.float32, device=dev)
    part = torch.zeros((nq, mb, w["dh"] + 2), dtype=torch.float32, device=dev)
    nbytes = modea_bytes(w)

    def step(i):
        th, rd, rs, vp = pools[i % len(pools)]
        fused_decode.sphkv_decode(d["q"], d["cb_flat"], d["tier_G"], d["tier_g"], th, rd, rs, vp,
                                  d["block_table"], d["bits_table"], d["ctx_lens"], out, part, nq, w["num_kv"],
                                  w["kv_groups"], w["num_tiers"], mb, w["page_size"], w["dh"], w["G_max"],
                                  w["cb_max"], w["g_max"], w["sm_scale"], w["max_ctx"])

    settle(step)
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(args.steps):
        step(i)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    gbps = nbytes / (ms * 1e-3) / 1e9
    log(f"[bench] Mode-A {ms * 1e3:.2f} us/step  {gbps:.1f} GB/s  ({gbps / PEAK_HBM_GBPS * 100:.1f}% of 8 TB/s)")
    aux = modea_aux(args, dev, w, d, part)
    cpu = None if args.no_cpu_baseline else cpu_baseline_modea(w)
    line = {
        "metric": "µs/decode step + achieved HBM GB/s (Mode-A LayerPool decode), 8B shape, 32K ctx, 1 GPU",
        "value": round(ms * 1e3, 3), "unit": "µs/decode step", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 6), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "u8 codes, fp16 V, fp32 math",
        "data": "synthetic (sphkv_synth.make_modea_workload seed 2)", "achieved_hbm_gbps": round(gbps, 1),
        "config": {"workload": f"Mode A: 32 q / 8 kv heads, dh 128, 32768 ctx, {w['page_size']}-token pages, "
                               f"60/40 tier 1/2, random page placement", "pages": int(w["num_kv"] * mb),
                   "rotated_pools": len(pools), "algorithmic_bytes_per_step": nbytes},
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(gbps / PEAK_HBM_GBPS, 4), "traffic": MODEA_TRAFFIC_BYTES.get(w["page_size"]),
                     "kernel": "modea_fast_kernel + modea_merge_kernel", "kernel_us": round(ms * 1e3, 3)},
        "aux_us_per_call": aux,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def bench_ragged(args, dev):
    """fused_decode_ragged (logits only, the reference's tiered call,
    spherical_kv_pipeline.py:1860-1875): one step = one call per compressed
    tier over config 2's pages of that tier, all kv heads, with RoPE tables
    built as the reference builds them (a default transformers rotary
    embedding, :1597-1608; fp32 angles).  The tables are fitted on the first
    call (untimed; its cost is reported) and the timed calls form the phases
    in the kernel; --no-rope-fit reads the tables' rows instead.  Algorithmic
    bytes per call: the tier's pointer-table rows, head ids, pages, positions
    and logits, plus (table path only) the cos / sin rows (first halves) of the
    distinct positions.  CPU baseline: the oracle's fp64 restatement on a
    bounded sample of pages, scaled by page count."""
    import fused_decode
    import oracle
    log("[bench] building config2 workload for fused_decode_ragged")
    wl = synth.make_decode_workload(2)
    pool, _, _ = ops.build_pool_gpu(wl, dev)
    plan = wl.plan
    max_pos = max(wl.lengths) + 64
    if args.rope_tables == "hf":
        cos_t, sin_t = synth.hf_rope_tables(max_pos, wl.dh, wl.rope_theta, dev)
    else:
        cos_t, sin_t = (torch.as_tensor(x, device=dev) for x in fmt.rope_tables(max_pos, wl.dh, wl.rope_theta))
    cos_h, sin_h = cos_t.cpu().numpy(), sin_t.cpu().numpy()
    fused_decode.use_rope_fit = not args.no_rope_fit
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    model = fused_decode.rope_fit_info(cos_t, sin_t)[0] if fused_decode.use_rope_fit else 0
    fit_ms = (time.perf_counter() - t0) * 1e3
    log(f"[bench] RoPE tables ({args.rope_tables}): fit model {model} in {fit_ms:.2f} ms (once per table)")
    q_h = wl.q[0].astype(np.float32)
    q = torch.as_tensor(q_h, device=dev)
    calls, host, nbytes, npages = [], [], 0, 0
    for tid in (1, 2):
        g, b = fmt.TIER_GEOMETRY[tid]
        G = wl.dh // g
        rows = np.nonzero(plan.tier == tid)[0]
        heads = (plan.seq_head[rows] % plan.num_kv).astype(np.int32)
        pos = plan.positions[rows].reshape(-1).astype(np.int32)
        cb = wl.codebooks[tid].reshape(plan.num_kv * G, 2 ** b, g)
        calls.append((pool.pages, torch.as_tensor(plan.ptable[rows], device=dev), torch.as_tensor(heads, device=dev),
                      torch.as_tensor(pos, device=dev), cos_t, sin_t, q, wl.gqa, plan.num_kv,
                      torch.as_tensor(cb, device=dev), wl.dh, G, g, b, 16))
        host.append((rows, heads, pos, cb, G, g, b))
        n_tok = int((pos >= 0).sum())
        nbytes += (int(sum(fmt.page_nbytes(tid, int(n), wl.dh) for n in plan.count[rows])) + 4 * pos.size
                   + 4 * wl.gqa * pos.size + 16 * rows.size
                   + (0 if model else 2 * 4 * (wl.dh // 2) * int(np.unique(pos[pos >= 0]).size)))
        npages += rows.size
        log(f"[bench] tier {tid}: {rows.size} pages, {n_tok} tokens")

    def step(i):
        for c in calls:
            fused_decode.fused_decode_ragged(*c)

    settle(step)
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    h0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    host_us = (time.perf_counter() - h0) / args.steps * 1e6
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    gbps = nbytes / (ms * 1e-3) / 1e9
    log(f"[bench] fused_decode_ragged {ms * 1e3:.2f} us per step (tiers 1 + 2)  {gbps:.1f} GB/s; "
        f"host {host_us:.2f} us per step to enqueue")
    if args.calibrate:
        calibrate_copies(dev)
    cpu = None
    if not args.no_cpu_baseline:
        pages_h = pool.pages.cpu().numpy()
        t0, done = time.perf_counter(), 0
        for rows, heads, pos, cb, G, g, b in host:
            k = min(rows.size, 150)
            oracle.ragged_logits(pages_h, plan.ptable[rows[:k]], heads[:k], pos[:16 * k], cos_h, sin_h, q_h, wl.gqa,
                                 cb, wl.dh, G, g, b, 16)
            done += k
        sec = time.perf_counter() - t0
        cpu = {"value": round(sec / done * npages * 1e6, 1), "unit": "µs per step (extrapolated by pages)",
               "cores": 1, "kind": "port",
               "sample": f"{done} of {npages} pages (150 per tier); oracle.ragged_logits, fp64 numpy"}
        log(f"[bench] CPU {cpu['value']} us per step")
    line = {
        "metric": "µs per fused_decode_ragged step (tier 1 + tier 2 logits), 8B shape, 32K ctx, 1 GPU",
        "value": round(ms * 1e3, 3), "unit": "µs/step", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 6), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "u8 codes, fp32 tables and math", "data": "synthetic (config 2 spec of BASELINE.json)",
        "config": {"workload": "config2 tier-1 and tier-2 pages (16 tokens), 8 kv heads, grp 4, dh 128",
                   "pages": int(npages), "algorithmic_bytes_per_step": int(nbytes),
                   "rope_tables": args.rope_tables, "rope_model": int(model), "rope_fit_once_ms": round(fit_ms, 2),
                   "host_us_per_step": round(host_us, 2)},
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(gbps / PEAK_HBM_GBPS, 4),
                     "traffic": RAGGED_TRAFFIC_BYTES["fit" if model else "table"], "kernel": "ragged_pipe_kernel",
                     "kernel_us": round(ms * 1e3, 3),
                     "frac_of": "both tiers' launches back to back (HIP events around the step); algorithmic bytes",
                     "traffic_of": "both launches, rocprofv3 FETCH_SIZE x2 + WRITE_SIZE "
                                   "(profiles/ragged_config2_hbm_traffic.txt)",
                     **({} if not model else {
                         "valu_bound_us": round(RAGGED_VALU_INSTS["fit"] * 4 / SIMDS / CLOCK_HZ * 1e6, 2),
                         "valu_frac": round(RAGGED_VALU_INSTS["fit"] * 4 / SIMDS / CLOCK_HZ / ms * 1e3, 4),
                         "valu_of": "SQ_INSTS_VALU of both launches (profiles/ragged_config2_hbm_traffic.txt) at "
                                    "one wave64 instruction per 4 cycles on 1024 SIMDs, 2.4 GHz"})},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def bench_prefill(args, dev):
    """One step = page one layer's retained K/V: device plan
    (plan_pages_gpu, including its one host synchronisation) + fused encode
    into a fresh pool.  CPU baseline: the host planner plus the oracle's C
    encode / page build over the same tokens."""
    log(f"[bench] building config{args.config} workload for prefill paging")
    wl = synth.make_encode_workload() if args.config == 3 else synth.make_decode_workload(args.config,
                                                                                         layout="sequential")
    L_max = max(wl.lengths)
    t = np.zeros((len(wl.tier_of), L_max), np.uint8)
    for sh, arr in enumerate(wl.tier_of):
        t[sh, :len(arr)] = np.asarray(arr, np.int64) & 0xFF
    tier_of = torch.from_numpy(t).to(dev)
    lens = torch.tensor(np.asarray(wl.lengths, np.int32), device=dev)
    row_base = torch.from_numpy(wl.row_base()).to(dev)
    k = torch.as_tensor(wl.k_rows(), device=dev)
    v = torch.as_tensor(wl.v_rows(), device=dev)
    cbs = {t: torch.as_tensor(np.ascontiguousarray(c, np.float32), device=dev) for t, c in wl.codebooks.items()}
    enc_ms = []

    def step(time_encode=False):
        dp = ops.plan_pages_gpu(tier_of, lens, wl.num_kv, wl.dh, row_base=row_base)
        pool = ops.PagedPool.allocate_device(dp, cbs, dev)
        if time_encode:
            a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a0.record()
        ops.encode_pages(pool, k, v, dp.src_rows)
        if time_encode:
            a1.record()
            enc_ms.append((a0, a1))
        return dp, pool

    for _ in range(args.warmup):
        dp, pool = step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        dp, pool = step()
    e1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    ms = e0.elapsed_time(e1) / args.steps
    n_tok = int(sum(len(x) for x in wl.tier_of))
    kept = int(sum(int(np.count_nonzero(np.asarray(x))) for x in wl.tier_of))
    nbytes = kept * wl.dh * 2 * 2 + dp.pages_bytes + dp.rows * 16 * wl.dh * 2
    for _ in range(args.steps):
        step(time_encode=True)
    torch.cuda.synchronize()
    enc_us = float(np.median([a.elapsed_time(b) for a, b in enc_ms])) * 1e3
    # the all-tier re-encode of every token (_codes_all, spherical_kv_pipeline.py:1536-1553),
    # which the reference's prefill runs after the page build; timed on its own
    ca = ops.CodesAll(wl.row_base(), wl.lengths, wl.num_kv, wl.dh, sorted(cbs), dev)
    ca_ms = []
    for _ in range(max(args.steps // 4, 5)):
        c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        c0.record()
        ca.launch(k, cbs)
        c1.record()
        ca_ms.append((c0, c1))
    torch.cuda.synchronize()
    codes_all_us = float(np.median([a.elapsed_time(b) for a, b in ca_ms])) * 1e3
    gbps = nbytes / (enc_us * 1e-6) / 1e9
    log(f"[bench] prefill paging {ms * 1e3:.1f} us/layer ({wall_ms * 1e3:.1f} us host wall), rows {dp.rows}; "
        f"encode_pages_kernel alone {enc_us:.1f} us; all-tier re-encode (_codes_all) {codes_all_us:.1f} us")
    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline (torch restatement of the reference prefill paging)")
        cpu = cpu_baseline_prefill(wl)
        log(f"[bench] CPU {cpu['value']} us/layer on {cpu['cores']} threads")
    line = {
        "metric": "µs per prefill paging of one layer (plan + encode + bitpack + V placement), 1 GPU",
        "value": round(ms * 1e3, 3), "unit": "µs/layer", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 6), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp16 in, u8 pages", "data": "synthetic (seeded generator, config spec of BASELINE.json)",
        "config": {"workload": f"config{args.config}: {wl.num_kv} kv heads, dh {wl.dh}, {wl.num_seqs} seq x "
                               f"{L_max} tokens, tier mix of BASELINE", "rows": dp.rows,
                   "algorithmic_bytes_per_step": int(nbytes),
                   "codes_all_us": round(codes_all_us, 1)},
        "roofline": {"bound": "valu", "achieved": round(gbps, 1), "peak": PEAK_HBM_GBPS,
                     "unit": "GB/s", "frac": round(gbps / PEAK_HBM_GBPS, 4),
                     "traffic": ENCODE_TRAFFIC_BYTES.get(args.config),
                     "kernel": "encode_pages_kernel", "kernel_us": round(enc_us, 3),
                     "hbm_bound_us": round(nbytes / (PEAK_HBM_GBPS * 1e9) * 1e6, 2),
                     **({} if args.config not in ENCODE_VALU_INSTS else {
                         "valu_bound_us": round(ENCODE_VALU_INSTS[args.config] * 4 / SIMDS / CLOCK_HZ * 1e6, 2),
                         "valu_frac": round(ENCODE_VALU_INSTS[args.config] * 4 / SIMDS / CLOCK_HZ * 1e6 / enc_us, 4)})},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def bench_step(args, dev):
    """The headline: one full reference decode step per timed step
    (_compressed_head_attention_batched + _append_decode_kv,
    spherical_kv_pipeline.py:2057-2475) through the bound step plan: the
    paged decode kernel over the context pages and the decode pages flushed
    so far, then the tail kernel (log-sum-exp merge with the staged tokens
    and the new token, output, append / flush).  The contexts grow by one
    token per step; algorithmic bytes are counted per step from each pool's
    exact tail state."""
    log(f"[bench] building config{args.config} workload")
    wl = synth.make_decode_workload(args.config, layout=args.layout,
                                    kv_device=dev if args.config in (4, 5) else None)
    n_in = 16                                        # rotating sets of new-token inputs
    st = synth.make_tail_steps(wl, n_in)
    wl.codebooks[3] = st.cb3
    pool0, _, _ = ops.build_pool_gpu(wl, dev)
    pools = [pool0] + [clone_pool(pool0) for _ in range(args.rotate - 1)]
    R = len(pools)
    appends = args.warmup + 2 * args.steps             # appending steps: warmup, timed, kernel-timed
    per_pool = -(-appends // R)
    cap = per_pool // ops.TAIL_SLOTS + 2
    tails = [ops.DecodeTail(p, wl.gqa, wl.rope_theta, capacity=cap) for p in pools]
    torch.cuda.synchronize()
    num_sh = wl.num_seqs * wl.num_kv
    q = torch.as_tensor(wl.q, device=dev)
    out = torch.empty_like(q)
    kin = torch.as_tensor(st.k, device=dev)
    vin = torch.as_tensor(st.v, device=dev)
    # positions: pool p's j-th appending step is at length + j
    posbuf = torch.as_tensor((np.asarray(wl.lengths, np.int64)[None, :] + np.arange(per_pool + 1)[:, None])
                             .astype(np.int32), device=dev)
    runs = [t.runner() for t in tails]
    kstride, pstride = kin[0].numel() * 2, wl.num_seqs * 4
    qp, op, kp, vp, pp = q.data_ptr(), out.data_ptr(), kin.data_ptr(), vin.data_ptr(), posbuf.data_ptr()
    done = [0] * R                                     # appending steps taken per pool

    def step(i, mode=3):
        p = i % R
        j = done[p]
        runs[p](qp, kp + (i % n_in) * kstride, 0, vp + (i % n_in) * kstride, pp + j * pstride, op, mode)
        if mode & 2:
            done[p] = j + 1

    base = fmt.decode_bytes(wl.plan)
    dh, G3 = wl.dh, wl.dh // 32
    dec_page = fmt.page_nbytes(3, 16, dh) + 16 * dh * 2 + 64 + 12          # K page, V, positions, ptable row
    stg_tok = 4 * G3 + 4 * G3 + 2 * dh + 4                                 # radii, codes, V, position
    new_tok = 2 * dh * 2                                                   # k_new, v_new

    def step_bytes(j):
        """(decode kernel, whole step) algorithmic bytes of a pool's step
        after j appending steps on it."""
        kern = base + num_sh * (j // 16) * dec_page
        return kern, kern + num_sh * ((j % 16) * stg_tok + new_tok)

    def steps_bytes(n, which):
        """Bytes of the next n steps (pool i mod R, each appending)."""
        sim, tot = list(done), 0
        for i in range(n):
            tot += step_bytes(sim[i % R])[which]
            sim[i % R] += 1
        return tot

    log(f"[bench] rows={wl.plan.num_rows} items={tails[0].num_items} pools={R} decode-page capacity={cap}")
    # untimed settle without appending (the contexts do not grow)
    settle(lambda i: step(i, 1))
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    tot_bytes = steps_bytes(args.steps, 1)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    h0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    host_us = (time.perf_counter() - h0) / args.steps * 1e6
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    us = ms * 1e3
    nbytes = tot_bytes / args.steps
    gbps = nbytes / (ms * 1e-3) / 1e9
    log(f"[bench] {us:.2f} us/step  {gbps:.1f} GB/s  ({gbps / PEAK_HBM_GBPS * 100:.1f}% of 8 TB/s); "
        f"host {host_us:.2f} us per step to enqueue")

    # the dominant kernel: the decode kernel of K more steps, each launch
    # timed by its own kernel-only timestamps (hipExtLaunchKernel events)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    for e0, e1 in evs:
        e0.record()
        e1.record()
    torch.cuda.synchronize()
    kb = steps_bytes(args.steps, 0)
    for i in range(args.steps):
        ops.time_next_decode_kernel(*evs[i])
        step(i)
    torch.cuda.synchronize()
    kern_ms = sum(e0.elapsed_time(e1) for e0, e1 in evs) / args.steps
    kbytes = kb / args.steps
    kern_gbps = kbytes / (kern_ms * 1e-3) / 1e9
    log(f"[bench] decode_kernel {kern_ms * 1e3:.2f} us (kernel-only timestamps)  {kern_gbps:.1f} GB/s")
    if args.calibrate:
        calibrate_copies(dev)

    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline (torch restatement of the reference path)")
        cpu = cpu_baseline(wl, pool0)
        log(f"[bench] CPU {cpu['value']} us/step on {cpu['cores']} threads")
    line = {
        "metric": METRICS[args.config], "value": round(us, 3), "unit": "µs/decode step", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 6),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp16 I/O; fp32 rotation, QK and softmax; P rounded to fp16 for the fp32-accumulated PV",
        "data": "synthetic (seeded generator, config spec of BASELINE.json)",
        "achieved_hbm_gbps": round(gbps, 1),
        "config": {"workload": f"config{args.config}: {wl.num_q} q / {wl.num_kv} kv heads, dh {wl.dh}, "
                               f"{wl.num_seqs} seq x {max(wl.lengths)} ctx, 16-token pages, tier mix of BASELINE; "
                               f"full decode step: page context + staged tokens + new token, then the append",
                   "num_seqs": wl.num_seqs, "ctx": max(wl.lengths), "pages": wl.plan.num_rows,
                   "rotated_pools": R, "algorithmic_bytes_per_step": round(nbytes),
                   "call": "DecodeTail.runner() (sphkv_step_plan_run)", "host_us_per_step": round(host_us, 2),
                   "kernels_per_step": ["decode_kernel", "decode_tail_kernel"]},
        "roofline": {"bound": "hbm", "achieved": round(kern_gbps, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(kern_gbps / PEAK_HBM_GBPS, 4),
                     "traffic": measured_traffic(args.config, args.layout),
                     "traffic_gbps": counter_gbps(args.config, args.layout, kern_ms),
                     "kernel": "decode_kernel", "kernel_us": round(kern_ms * 1e3, 3),
                     "frac_of": "decode_kernel alone (the step's dominant kernel), kernel-only start / stop "
                                "timestamps of each launch (hipExtLaunchKernel); algorithmic bytes of its launch "
                                "(pages, dense K, V, positions, pointer-table rows)",
                     "traffic_of": "decode_kernel launch, rocprofv3 FETCH_SIZE x2 + WRITE_SIZE "
                                   "(profiles/decode_config2_hbm_traffic.txt); traffic_gbps: those bytes "
                                   "over kernel_us",
                     "whole_step_achieved": round(gbps, 1),
                     "whole_step_frac": round(gbps / PEAK_HBM_GBPS, 4),
                     "whole_step_of": "the headline value: both kernels, HIP events around the steps; algorithmic "
                                      "bytes incl. the staged tokens and the new token"},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--config", type=int, default=2, choices=[1, 2, 3, 4, 5],
                    help="1, 2, 4, 5: decode configs; 3: the encode config (with --path prefill)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--rotate", type=int, default=ROTATE)
    ap.add_argument("--layout", default="default", choices=["default", "sequential"],
                    help="page placement: the config's own (random for configs 2-5) or sequential")
    ap.add_argument("--path", default="step", choices=["step", "pages", "modea", "prefill", "ragged"],
                    help="step: the full Mode-B decode step (page context + staged tokens + new token, then "
                         "the append; the headline); pages: the page-resident decode alone; modea: LayerPool "
                         "decode; prefill: device page plan + fused encode; ragged: fused_decode_ragged")
    ap.add_argument("--page-size", type=int, default=16, help="Mode-A page size (16..128, multiple of 16)")
    ap.add_argument("--rope-tables", default="hf", choices=["hf", "exact"],
                    help="ragged: RoPE tables of the HF construction (fp32 angles) or of exact angles")
    ap.add_argument("--no-rope-fit", action="store_true", help="ragged: read the RoPE tables' rows every call")
    ap.add_argument("--calibrate", action="store_true",
                    help="after timing, run plain device copies of COPY_BYTES (torch copy_), the "
                         "reference kernel of known traffic for FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); the decode "
              f"shards by kv head or context with no exchange inside the kernel, and multi-GPU runs "
              f"are not part of this build.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.path == "modea":
        bench_modea(args, dev)
        return
    if args.path == "prefill":
        bench_prefill(args, dev)
        return
    if args.path == "ragged":
        bench_ragged(args, dev)
        return
    if args.config == 3:
        print("bench.py: config 3 is the encode workload; use --path prefill --config 3", file=sys.stderr)
        sys.exit(2)

    if args.path == "step":
        bench_step(args, dev)
        return

    log(f"[bench] building config{args.config} workload")
    # configs 4 and 5 draw their K / V on the device (gigabytes of rows)
    wl = synth.make_decode_workload(args.config, layout=args.layout,
                                    kv_device=dev if args.config in (4, 5) else None)
    pool0, _, _ = ops.build_pool_gpu(wl, dev)
    pools = [pool0] + [clone_pool(pool0) for _ in range(args.rotate - 1)]
    torch.cuda.synchronize()
    q = torch.as_tensor(wl.q, device=dev)
    out = torch.empty_like(q)
    ws = torch.zeros(max(pool0.workspace_bytes(wl.gqa), 4), dtype=torch.uint8, device=dev)
    nbytes = fmt.decode_bytes(wl.plan)
    log(f"[bench] rows={wl.plan.num_rows} items={pool0.num_items} algorithmic bytes/step={nbytes}")
    # the bound call (one ctypes call of four arguments per step)
    runs = [ops.DecodeRunner(p, wl.gqa, wl.rope_theta, workspace=ws).raw() for p in pools]
    qp, op, R = q.data_ptr(), out.data_ptr(), len(pools)

    settle(lambda i: runs[i % R](qp, op))
    for i in range(args.warmup):
        runs[i % R](qp, op)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    h0 = time.perf_counter()
    for i in range(args.steps):
        runs[i % R](qp, op)
    host_us = (time.perf_counter() - h0) / args.steps * 1e6
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    us = ms * 1e3
    gbps = nbytes / (ms * 1e-3) / 1e9
    log(f"[bench] {us:.2f} us/step  {gbps:.1f} GB/s  ({gbps / PEAK_HBM_GBPS * 100:.1f}% of 8 TB/s); "
        f"host {host_us:.2f} us per call to enqueue")
    # host cost of the checked Python call, for comparison (enqueue only;
    # a few untimed calls first, so one-time costs stay out of short runs)
    for i in range(10):
        ops.decode_paged(pools[i % R], q, wl.gqa, wl.rope_theta, out=out, workspace=ws)
    torch.cuda.synchronize()
    h0 = time.perf_counter()
    for i in range(args.steps):
        ops.decode_paged(pools[i % R], q, wl.gqa, wl.rope_theta, out=out, workspace=ws)
    py_host_us = (time.perf_counter() - h0) / args.steps * 1e6
    torch.cuda.synchronize()
    log(f"[bench] decode_paged (checked Python call): host {py_host_us:.2f} us per call to enqueue")

    # the dominant kernel alone: K decode_kernel launches back to back (the
    # partials phase only), HIP events around them on the stream they run on
    # (the launch gap included).  Kernel-only timestamps of a launch that
    # follows the merge kernel start while that kernel still runs here, so
    # they are not used on this path.
    for i in range(args.warmup):
        ops.decode_paged_partials(pools[i % R], q, wl.gqa, wl.rope_theta, ws)
    torch.cuda.synchronize()
    k0, k1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    k0.record()
    for i in range(args.steps):
        ops.decode_paged_partials(pools[i % R], q, wl.gqa, wl.rope_theta, ws)
    k1.record()
    torch.cuda.synchronize()
    kern_ms = k0.elapsed_time(k1) / args.steps
    kern_gbps = nbytes / (kern_ms * 1e-3) / 1e9
    log(f"[bench] decode_kernel {kern_ms * 1e3:.2f} us (back-to-back launches)  {kern_gbps:.1f} GB/s")

    if args.calibrate:
        calibrate_copies(dev)

    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline (torch restatement of the reference path)")
        cpu = cpu_baseline(wl, pool0)
        log(f"[bench] CPU {cpu['value']} us/step on {cpu['cores']} threads")

    line = {
        "metric": METRICS[args.config], "value": round(us, 3), "unit": "µs/decode step", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 6),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp16 I/O; fp32 rotation, QK and softmax; P rounded to fp16 for the fp32-accumulated PV",
        "data": "synthetic (seeded generator, config spec of BASELINE.json)",
        "achieved_hbm_gbps": round(gbps, 1),
        "config": {"workload": f"config{args.config}: {wl.num_q} q / {wl.num_kv} kv heads, dh {wl.dh}, "
                               f"{wl.num_seqs} seq x {max(wl.lengths)} ctx, 16-token pages, tier mix of BASELINE",
                   "num_seqs": wl.num_seqs, "ctx": max(wl.lengths), "pages": wl.plan.num_rows,
                   "rotated_pools": len(pools), "algorithmic_bytes_per_step": nbytes,
                   "call": "DecodeRunner.raw() (sphkv_decode_plan_run)", "host_us_per_call": round(host_us, 2),
                   "host_us_per_call_decode_paged": round(py_host_us, 2)},
        "roofline": {"bound": "hbm", "achieved": round(kern_gbps, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(kern_gbps / PEAK_HBM_GBPS, 4),
                     "traffic": measured_traffic(args.config, args.layout),
                     "traffic_gbps": counter_gbps(args.config, args.layout, kern_ms),
                     "kernel": "decode_kernel", "kernel_us": round(kern_ms * 1e3, 3),
                     "frac_of": "decode_kernel alone, HIP events around back-to-back launches (launch gap "
                                "included); algorithmic bytes of its launch",
                     "traffic_of": "decode_kernel launch, rocprofv3 FETCH_SIZE x2 + WRITE_SIZE "
                                   "(profiles/decode_config2_hbm_traffic.txt); traffic_gbps: those bytes "
                                   "over kernel_us",
                     "whole_step_achieved": round(gbps, 1),
                     "whole_step_frac": round(gbps / PEAK_HBM_GBPS, 4),
                     "whole_step_of": "the value: decode_kernel + decode_merge_kernel, HIP events around the steps"},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
