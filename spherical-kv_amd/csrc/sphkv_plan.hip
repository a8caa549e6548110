// Device-side page planning: the grouping, sorting, chunking and pointer-table
// construction of _build_per_head_pages (spherical_kv_pipeline.py:1146-1228,
// offsets :1202-1213) for the paged pool, so that prefill builds its plan
// without a host round trip per (layer, head, tier).
//
// The plan equals sphkv_format.plan_pages with logical placement: for each
// (sequence, kv head) the rows of its pages, tiers in order of first
// appearance (the reference's dict insertion order), token indices ascending
// within a tier, chunks of 16; pages placed back to back in row order at
// 16-byte aligned offsets (a dense fp16 page so that its payload after the
// 8-byte header is 16-byte aligned).
//
// Kernels:
//   plan_count_kernel  per (sequence, head): tokens and first index per tier
//   plan_scan_kernel   one thread: row starts and each tier run's byte start
//                      (page i of a run starts at run_start + i * align16(size
//                      of a full page), so a run is placed in O(1))
//   plan_fill_kernel   per (sequence, head): page rows, then each token's
//                      rank within its tier (wave ballots + a block scan) puts
//                      it in its page slot
#include "sphkv_common.h"
#include "sphkv_internal.h"

namespace sphkv {

namespace {

constexpr int kPlanThreads = 256;
constexpr int kHeader = 8;          // config.py:3 HEADER_BYTES

// tier id -> run slot: 1, 2, 3 -> 0, 1, 2; dense (0xFF) -> 3; 0 = dropped (-1); other ids are invalid (-2)
__device__ __forceinline__ int tier_slot(int id) {
  return id == 1 ? 0 : id == 2 ? 1 : id == 3 ? 2 : id == 0xFF ? 3 : id == 0 ? -1 : -2;
}
__device__ __forceinline__ int slot_tier(int k) { return k == 3 ? 0xFF : k + 1; }

// bytes of a page of n tokens (pagebuilder.py:32 concatenation; dense: header + fp16 K)
__device__ __forceinline__ int64_t page_bytes(int k, int n, int dh) {
  if (k == 3) return kHeader + (int64_t)n * dh * 2;
  const int g = tier_g(k + 1), b = tier_b(k + 1), G = dh / g;
  return kHeader + 4 * G + ((int64_t)n * G * b + 7) / 8 + (int64_t)n * G;
}
__device__ __forceinline__ int64_t align16(int64_t x) { return (x + 15) & ~(int64_t)15; }
// placement of a page after byte offset off (sphkv_format.plan_pages)
__device__ __forceinline__ int64_t place(int64_t off, int k) {
  if (k != 3) return align16(off);
  int64_t o = align16(off + kHeader) - kHeader;
  return o < 0 ? o + 16 : o;
}

// per (sequence, head) record in the workspace
enum : int { kCnt = 0, kFirst = 4, kRows = 8, kOrder = 9, kRunStart = 10, kRowStart = 14, kRec = 16 };

}  // namespace

__global__ __launch_bounds__(kPlanThreads) void plan_count_kernel(PlanLaunch a) {
  __shared__ int cnt[4], first[4], bad;
  const int sh = blockIdx.x, s = sh / a.num_kv;
  if (threadIdx.x < 4) { cnt[threadIdx.x] = 0; first[threadIdx.x] = 0x7FFFFFFF; }
  if (threadIdx.x == 0) bad = 0;
  __syncthreads();
  const int L = a.lens[s];
  const uint8_t* t_of = a.tier_of + (int64_t)sh * a.tier_stride;
  for (int t = threadIdx.x; t < L; t += kPlanThreads) {
    const int k = tier_slot(t_of[t]);
    if (k >= 0) {
      atomicAdd(&cnt[k], 1);
      atomicMin(&first[k], t);
    } else if (k == -2) {
      atomicAdd(&bad, 1);
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int32_t* rec = a.work + (int64_t)sh * kRec;
    int order = 0, n_runs = 0, rows = 0;
    bool used[4] = {false, false, false, false};
    for (int r = 0; r < 4; ++r) {               // tiers by first appearance
      int best = -1;
      for (int k = 0; k < 4; ++k)
        if (!used[k] && cnt[k] > 0 && (best < 0 || first[k] < first[best])) best = k;
      if (best < 0) break;
      used[best] = true;
      order |= best << (4 * n_runs);
      ++n_runs;
      rows += (cnt[best] + 15) / 16;
    }
    for (int r = n_runs; r < 4; ++r) order |= 0xF << (4 * r);
    for (int k = 0; k < 4; ++k) { rec[kCnt + k] = cnt[k]; rec[kFirst + k] = first[k]; }
    rec[kRows] = rows;
    rec[kOrder] = order;
    if (bad) atomicAdd(a.totals + 2, bad);
  }
}

__global__ void plan_scan_kernel(PlanLaunch a) {
  if (threadIdx.x != 0) return;
  int64_t off = 0;
  int row = 0;
  for (int sh = 0; sh < a.num_sh; ++sh) {
    int32_t* rec = a.work + (int64_t)sh * kRec;
    rec[kRowStart] = row;
    a.row_start[sh] = row;
    row += rec[kRows];
    for (int r = 0; r < 4; ++r) {
      const int k = (rec[kOrder] >> (4 * r)) & 0xF;
      if (k == 0xF) { rec[kRunStart + r] = -1; continue; }
      const int n = rec[kCnt + k], pages = (n + 15) / 16, last = n - 16 * (pages - 1);
      const int64_t start = place(off, k);
      if (start > 0x7FFFFF00LL) { atomicAdd(a.totals + 3, 1); rec[kRunStart + r] = 0; continue; }
      rec[kRunStart + r] = (int32_t)start;
      off = start + (int64_t)(pages - 1) * align16(page_bytes(k, 16, a.dh)) + page_bytes(k, last, a.dh);
    }
  }
  a.row_start[a.num_sh] = row;
  const int64_t total = align16(off) + 16;
  a.totals[0] = row;
  a.totals[1] = total > 0x7FFFFF00LL ? -1 : (int32_t)total;
}

__global__ __launch_bounds__(kPlanThreads) void plan_fill_kernel(PlanLaunch a) {
  __shared__ int page0[4], run_start[4], base[4], wsum[kPlanThreads / 64][4];
  const int sh = blockIdx.x, s = sh / a.num_kv;
  const int32_t* rec = a.work + (int64_t)sh * kRec;
  const int row0 = rec[kRowStart];
  if (threadIdx.x == 0) {
    int p = 0;
    for (int k = 0; k < 4; ++k) page0[k] = -1;
    for (int r = 0; r < 4; ++r) {
      const int k = (rec[kOrder] >> (4 * r)) & 0xF;
      if (k == 0xF) break;
      page0[k] = p;
      run_start[k] = rec[kRunStart + r];
      p += (rec[kCnt + k] + 15) / 16;
    }
    for (int k = 0; k < 4; ++k) base[k] = 0;
  }
  __syncthreads();
  // page rows: tier, count, pointer-table row, (seq, head), V slot; slots padded with -1
  const int rows = rec[kRows];
  if (row0 < 0 || row0 + rows > a.max_rows) return;       // outputs too small: nothing is written
  for (int j = threadIdx.x; j < rows; j += kPlanThreads) {
    int k = 0;
    for (int kk = 0; kk < 4; ++kk)
      if (page0[kk] >= 0 && j >= page0[kk] && j < page0[kk] + (rec[kCnt + kk] + 15) / 16) k = kk;
    const int i = j - page0[k], n_k = rec[kCnt + k];
    const int n = min(16, n_k - 16 * i);
    const int64_t off = (int64_t)run_start[k] + (int64_t)i * align16(page_bytes(k, 16, a.dh));
    const int row = row0 + j;
    a.tier[row] = slot_tier(k);
    a.count[row] = n;
    a.seq_head[row] = sh;
    a.vslot[row] = row;
    int64_t th, rd;
    if (k == 3) {
      th = off + kHeader;
      rd = th + (int64_t)n * a.dh * 2;
    } else {
      const int g = tier_g(k + 1), b = tier_b(k + 1), G = a.dh / g;
      th = off + kHeader + 4 * G;
      rd = th + ((int64_t)n * G * b + 7) / 8;
    }
    a.ptable[3 * (int64_t)row] = (int32_t)off;
    a.ptable[3 * (int64_t)row + 1] = (int32_t)th;
    a.ptable[3 * (int64_t)row + 2] = (int32_t)rd;
    for (int q = 0; q < 16; ++q) {
      a.tokens[(int64_t)row * 16 + q] = -1;
      a.positions[(int64_t)row * 16 + q] = -1;
      if (a.src_rows) a.src_rows[(int64_t)row * 16 + q] = -1;
    }
  }
  __syncthreads();
  // each kept token's rank within its tier -> (page, slot)
  const int L = a.lens[s];
  const uint8_t* t_of = a.tier_of + (int64_t)sh * a.tier_stride;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t rb = a.row_base ? a.row_base[sh] : 0;
  for (int c0 = 0; c0 < L; c0 += kPlanThreads) {
    const int t = c0 + threadIdx.x;
    const int k = t < L ? tier_slot(t_of[t]) : -1;
    int below = 0;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const uint64_t m = __builtin_amdgcn_ballot_w64(k == kk);
      if (lane == 0) wsum[wave][kk] = __builtin_popcountll(m);
      if (k == kk) below = __builtin_popcountll(m & ((1ull << lane) - 1ull));
    }
    __syncthreads();
    if (k >= 0) {
      int r = base[k] + below;
      for (int w = 0; w < wave; ++w) r += wsum[w][k];
      const int row = row0 + page0[k] + r / 16, q = r % 16;
      a.tokens[(int64_t)row * 16 + q] = t;
      a.positions[(int64_t)row * 16 + q] = a.pos ? a.pos[(int64_t)s * a.pos_stride + t] : t;
      if (a.src_rows) a.src_rows[(int64_t)row * 16 + q] = rb + t;
    }
    __syncthreads();
    if (threadIdx.x < 4)
      for (int w = 0; w < kPlanThreads / 64; ++w) base[threadIdx.x] += wsum[w][threadIdx.x];
    __syncthreads();
  }
}

int launch_plan(const PlanLaunch& L, int phase, hipStream_t stream) {
  if (L.num_sh <= 0) return 0;
  if (phase == 0) {
    hipLaunchKernelGGL(plan_count_kernel, dim3(L.num_sh), dim3(kPlanThreads), 0, stream, L);
    hipLaunchKernelGGL(plan_scan_kernel, dim3(1), dim3(64), 0, stream, L);
  } else {
    hipLaunchKernelGGL(plan_fill_kernel, dim3(L.num_sh), dim3(kPlanThreads), 0, stream, L);
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace sphkv
