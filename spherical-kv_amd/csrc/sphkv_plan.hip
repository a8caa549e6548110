// Device-side page planning: the grouping, sorting, chunking and pointer-table
// construction of _build_per_head_pages (spherical_kv_pipeline.py:1146-1228,
// offsets :1202-1213) for the paged pool, so that prefill builds its plan
// without a host round trip per (layer, head, tier).
//
// The plan equals sphkv_format.plan_pages with logical placement: for each
// (sequence, kv head) the rows of its pages, tiers in order of their smallest
// token index, token indices ascending within a tier, chunks of 16; pages
// placed back to back in row order at 16-byte aligned offsets (a dense fp16
// page so that its payload after the 8-byte header is 16-byte aligned).
//
// The reference orders a head's tiers by first appearance in allocate()'s
// retained list, sinks + recents + the rest (allocation.py:207-217; dict
// insertion order, spherical_kv_pipeline.py:1156-1162).  Smallest index
// gives the same order when every sink and recent token carries token 0's
// tier, as with the protected tier at SINK_TOKENS=4, RECENT_WINDOW=256
// (config.py:14-15); a caller whose recents carry another tier than its
// sinks gets index order.
//
// Kernels (a (sequence, head)'s tokens are cut into chunks of kPlanChunk):
//   plan_count_kernel  per (sequence, head, chunk): tokens and first index
//                      per tier, by wave ballots
//   plan_scan_kernel   one workgroup: per (sequence, head) a wave scans its
//                      chunks' counts into rank bases (64 chunks per load) and
//                      sets the tier order and rows; then the tier runs are
//                      placed back to back by a block-wide scan of placement
//                      maps (below), each thread taking a contiguous span of
//                      (sequence, head) ranges
//
// Placement as a map of the running byte offset x: a run of a compressed
// tier starts at align16(x), a dense run at align16(x + 8) - 8 (payload
// 16-byte aligned after the header); page i of a run starts at run_start +
// i * align16(size of a full page), so the run ends at start + B with B fixed
// by the tier and count.  Each run is therefore x -> 16 ceil((x + a) / 16) +
// b (a = 0 or 8), and so is any chain of runs: (a1, b1) then (a2, b2) is
// (a1, 16 ceil((b1 + a2) / 16) + b2).  The maps form a monoid (with the
// identity for ranges without tokens) and scan in parallel.
//   plan_fill_kernel   per (sequence, head, chunk): its share of the page
//                      rows, then each token's rank within its tier (chunk
//                      base + wave ballots) puts it in its page slot
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

// per (sequence, head) record in the workspace, followed by the chunks' records
enum : int { kCnt = 0, kFirst = 4, kRows = 8, kOrder = 9, kRunStart = 10, kRowStart = 14, kRec = 16 };
// per chunk: counts (then rank bases), first index, invalid ids, sequence-length flag
enum : int { kChCnt = 0, kChFirst = 4, kChBad = 8, kChLen = 9, kChRec = 12 };
constexpr int kPlanChunk = 2048;
constexpr int kScanThreads = 1024;
constexpr int64_t kMaxOff = 0x7FFFFF00LL;   // byte offsets stay int32

// placement map x -> 16 ceil((x + a) / 16) + b, or the identity (id != 0)
struct Place { int64_t b; int a, id; };
__device__ __forceinline__ int64_t ceil16(int64_t v) { return ((v + 15) >> 4) << 4; }
__device__ __forceinline__ Place then(const Place& f, const Place& g) {      // f, then g
  if (f.id) return g;
  if (g.id) return f;
  return Place{ceil16(f.b + g.a) + g.b, f.a, 0};
}
__device__ __forceinline__ int64_t apply(const Place& f, int64_t x) { return f.id ? x : ceil16(x + f.a) + f.b; }
// bytes from a run's start to its end: full pages at align16 strides, then the last page
__device__ __forceinline__ int64_t run_bytes(int k, int n, int dh) {
  const int pages = (n + 15) / 16, last = n - 16 * (pages - 1);
  return (int64_t)(pages - 1) * align16(page_bytes(k, 16, dh)) + page_bytes(k, last, dh);
}
__device__ __forceinline__ Place run_map(int k, int n, int dh) {
  return k == 3 ? Place{run_bytes(k, n, dh) - kHeader, kHeader, 0} : Place{run_bytes(k, n, dh), 0, 0};
}

__device__ __forceinline__ int wave_scan_incl(int v, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int t = __shfl_up(v, d, 64);
    if (lane >= d) v += t;
  }
  return v;
}
__device__ __forceinline__ int wave_min(int v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v = min(v, __shfl_xor(v, d, 64));
  return v;
}
__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
  return v;
}

__device__ __forceinline__ int32_t* sh_rec(const PlanLaunch& a, int sh) { return a.work + (int64_t)sh * kRec; }
__device__ __forceinline__ int32_t* ch_rec(const PlanLaunch& a, int sh, int c) {
  return a.work + (int64_t)a.num_sh * kRec + ((int64_t)sh * a.nchunks + c) * kChRec;
}

}  // namespace

__global__ __launch_bounds__(kPlanThreads) void plan_count_kernel(PlanLaunch a) {
  __shared__ int wc[kPlanThreads / 64][4], wf[kPlanThreads / 64][4], wbad[kPlanThreads / 64];
  const int sh = blockIdx.x / a.nchunks, c = blockIdx.x % a.nchunks, s = sh / a.num_kv;
  const int L = min(a.lens[s], a.max_len), t0 = c * kPlanChunk, t1 = min(L, t0 + kPlanChunk);
  const uint8_t* t_of = a.tier_of + (int64_t)sh * a.tier_stride;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int cnt[4] = {0, 0, 0, 0}, first[4] = {0x7FFFFFFF, 0x7FFFFFFF, 0x7FFFFFFF, 0x7FFFFFFF}, bad = 0;
  for (int b = t0; b < t1; b += kPlanThreads) {        // wave-uniform trip count
    const int t = b + threadIdx.x;
    const int k = t < t1 ? tier_slot(t_of[t]) : -1;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const uint64_t m = __builtin_amdgcn_ballot_w64(k == kk);
      cnt[kk] += __builtin_popcountll(m);
      if (m) first[kk] = min(first[kk], b + 64 * wave + (int)__builtin_ctzll(m));
    }
    bad += __builtin_popcountll(__builtin_amdgcn_ballot_w64(k == -2));
  }
  if (lane == 0) {
    for (int kk = 0; kk < 4; ++kk) { wc[wave][kk] = cnt[kk]; wf[wave][kk] = first[kk]; }
    wbad[wave] = bad;
  }
  __syncthreads();
  if (threadIdx.x < 4) {
    int n = 0, f = 0x7FFFFFFF;
    for (int w = 0; w < kPlanThreads / 64; ++w) { n += wc[w][threadIdx.x]; f = min(f, wf[w][threadIdx.x]); }
    int32_t* r = ch_rec(a, sh, c);
    r[kChCnt + threadIdx.x] = n;
    r[kChFirst + threadIdx.x] = f;
  }
  if (threadIdx.x == 0) {
    int nb = 0;
    for (int w = 0; w < kPlanThreads / 64; ++w) nb += wbad[w];
    int32_t* r = ch_rec(a, sh, c);
    r[kChBad] = nb;
    r[kChLen] = c == 0 && (a.lens[s] > a.max_len || a.lens[s] < 0);
  }
}

// wave-inclusive scan of (map, rows) over the lanes, by shuffles
__device__ __forceinline__ void wave_scan_place(Place& m, int& rows, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int lo = __shfl_up((int)(uint32_t)m.b, d, 64), hi = __shfl_up((int)(m.b >> 32), d, 64);
    const int pa = __shfl_up(m.id ? -1 : m.a, d, 64), pr = __shfl_up(rows, d, 64);
    if (lane >= d) {
      const Place p{(int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo), pa < 0 ? 0 : pa, pa < 0};
      m = then(p, m);
      rows += pr;
    }
  }
}

__global__ __launch_bounds__(kScanThreads) void plan_scan_kernel(PlanLaunch a) {
  // per-range summaries kept for the placement when the ranges fit one per thread
  __shared__ int s_order[kScanThreads], s_rows[kScanThreads], s_cnt[kScanThreads][4];
  __shared__ int64_t w_b[kScanThreads / 64];
  __shared__ int w_a[kScanThreads / 64], w_rows[kScanThreads / 64];
  __shared__ int nbad, nflag;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, t = threadIdx.x;
  const bool cached = a.num_sh <= kScanThreads;
  if (t == 0) { nbad = 0; nflag = 0; }
  __syncthreads();
  // (1) a wave per (sequence, head): its chunks' exclusive rank bases per
  // tier, 64 chunks per step, then totals, first indices, tier order, rows
  for (int sh = wave; sh < a.num_sh; sh += kScanThreads / 64) {
    int carry[4] = {0, 0, 0, 0}, first[4] = {0x7FFFFFFF, 0x7FFFFFFF, 0x7FFFFFFF, 0x7FFFFFFF}, bad = 0, flag = 0;
    for (int c0 = 0; c0 < a.nchunks; c0 += 64) {          // wave-uniform trip count
      const int c = c0 + lane;
      int32_t* r = c < a.nchunks ? ch_rec(a, sh, c) : nullptr;
      int n[4], f[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) { n[k] = r ? r[kChCnt + k] : 0; f[k] = r ? r[kChFirst + k] : 0x7FFFFFFF; }
      if (r) { bad += r[kChBad]; flag |= r[kChLen]; }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int incl = wave_scan_incl(n[k], lane);
        if (r) r[kChCnt + k] = carry[k] + incl - n[k];
        carry[k] += __shfl(incl, 63, 64);
        first[k] = min(first[k], f[k]);
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) first[k] = wave_min(first[k]);
    bad = wave_sum(bad);
    flag = wave_sum(flag);
    if (lane == 0) {
      int order = 0, n_runs = 0, rows = 0;
      bool used[4] = {false, false, false, false};
      for (int q = 0; q < 4; ++q) {                      // tiers by first appearance
        int best = -1;
        for (int k = 0; k < 4; ++k)
          if (!used[k] && carry[k] > 0 && (best < 0 || first[k] < first[best])) best = k;
        if (best < 0) break;
        used[best] = true;
        order |= best << (4 * n_runs);
        ++n_runs;
        rows += (carry[best] + 15) / 16;
      }
      for (int q = n_runs; q < 4; ++q) order |= 0xF << (4 * q);
      int32_t* rec = sh_rec(a, sh);
      for (int k = 0; k < 4; ++k) { rec[kCnt + k] = carry[k]; rec[kFirst + k] = first[k]; }
      rec[kRows] = rows;
      rec[kOrder] = order;
      if (cached) {
        s_order[sh] = order;
        s_rows[sh] = rows;
        for (int k = 0; k < 4; ++k) s_cnt[sh][k] = carry[k];
      }
      if (bad) atomicAdd(&nbad, bad);
      if (flag) atomicAdd(&nflag, flag);
    }
  }
  __syncthreads();                                       // the records above are visible to the whole workgroup
  // (2) placement: thread t takes ranges [s0, s1) (one each when they fit);
  // its runs composed into one map, an exclusive scan of (map, rows) over the
  // threads (shuffles in each wave, then the wave totals), then its runs
  // placed from the scanned offset
  const int per = (a.num_sh + kScanThreads - 1) / kScanThreads;
  const int s0 = min(t * per, a.num_sh), s1 = min(s0 + per, a.num_sh);
  auto summary = [&](int sh, int& order, int& rows, int (&cnt)[4]) {
    if (cached) {
      order = s_order[sh]; rows = s_rows[sh];
      for (int k = 0; k < 4; ++k) cnt[k] = s_cnt[sh][k];
    } else {
      const int32_t* rec = sh_rec(a, sh);
      order = rec[kOrder]; rows = rec[kRows];
      for (int k = 0; k < 4; ++k) cnt[k] = rec[kCnt + k];
    }
  };
  Place m{0, 0, 1};
  int rows = 0;
  for (int sh = s0; sh < s1; ++sh) {
    int order, nr, cnt[4];
    summary(sh, order, nr, cnt);
    rows += nr;
    for (int q = 0; q < 4; ++q) {
      const int k = (order >> (4 * q)) & 0xF;
      if (k != 0xF) m = then(m, run_map(k, cnt[k], a.dh));
    }
  }
  wave_scan_place(m, rows, lane);
  if (lane == 63) { w_b[wave] = m.b; w_a[wave] = m.id ? -1 : m.a; w_rows[wave] = rows; }
  // this thread's exclusive value within its wave: lane - 1's inclusive one
  const int lo = __shfl_up((int)(uint32_t)m.b, 1, 64), hi = __shfl_up((int)(m.b >> 32), 1, 64);
  const int pa = __shfl_up(m.id ? -1 : m.a, 1, 64), pr = __shfl_up(rows, 1, 64);
  __syncthreads();
  int64_t off = 0;
  int row = 0;
  for (int w = 0; w < wave; ++w) {                       // the earlier waves' totals, in order
    off = apply(Place{w_b[w], w_a[w] < 0 ? 0 : w_a[w], w_a[w] < 0}, off);
    row += w_rows[w];
  }
  if (lane > 0) {
    off = apply(Place{(int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo), pa < 0 ? 0 : pa, pa < 0}, off);
    row += pr;
  }
  int ovf = 0;
  for (int sh = s0; sh < s1; ++sh) {
    int order, nr, cnt[4];
    summary(sh, order, nr, cnt);
    int32_t* rec = sh_rec(a, sh);
    rec[kRowStart] = row;
    a.row_start[sh] = row;
    row += nr;
    for (int q = 0; q < 4; ++q) {
      const int k = (order >> (4 * q)) & 0xF;
      if (k == 0xF) { rec[kRunStart + q] = -1; continue; }
      const int64_t start = place(off, k);
      if (start > kMaxOff) ++ovf;
      rec[kRunStart + q] = start > kMaxOff ? 0 : (int32_t)start;
      off = start + run_bytes(k, cnt[k], a.dh);
    }
  }
  if (ovf) atomicAdd(&nflag, ovf);
  __syncthreads();
  if (t == kScanThreads - 1) {                           // holds the last range (or the full scan)
    a.row_start[a.num_sh] = row;
    const int64_t total = align16(off) + 16;
    a.totals[0] = row;
    a.totals[1] = total > kMaxOff ? -1 : (int32_t)total;
    a.totals[2] = nbad;
    a.totals[3] = nflag;
  }
}

__global__ __launch_bounds__(kPlanThreads) void plan_fill_kernel(PlanLaunch a) {
  __shared__ int page0[4], npages[4], run_start[4], base[4], wsum[kPlanThreads / 64][4];
  const int sh = blockIdx.x / a.nchunks, c = blockIdx.x % a.nchunks, s = sh / a.num_kv;
  const int32_t* rec = sh_rec(a, sh);
  const int row0 = rec[kRowStart];
  const int rows = rec[kRows];
  if (row0 < 0 || row0 + rows > a.max_rows) return;       // outputs too small: nothing is written
  if (threadIdx.x == 0) {
    int p = 0;
    for (int k = 0; k < 4; ++k) { page0[k] = -1; npages[k] = 0; }
    for (int q = 0; q < 4; ++q) {
      const int k = (rec[kOrder] >> (4 * q)) & 0xF;
      if (k == 0xF) break;
      page0[k] = p;
      npages[k] = (rec[kCnt + k] + 15) / 16;
      run_start[k] = rec[kRunStart + q];
      p += npages[k];
    }
    const int32_t* cr = ch_rec(a, sh, c);
    for (int k = 0; k < 4; ++k) base[k] = cr[kChCnt + k];
  }
  __syncthreads();
  // this chunk's share of the page rows: tier, count, pointer-table row,
  // (seq, head), V slot; the slots past a page's count are padding (-1)
  const int j0 = (int)((int64_t)rows * c / a.nchunks), j1 = (int)((int64_t)rows * (c + 1) / a.nchunks);
  for (int j = j0 + (int)threadIdx.x; j < j1; j += kPlanThreads) {
    int k = 0;
    for (int kk = 0; kk < 4; ++kk)
      if (page0[kk] >= 0 && j >= page0[kk] && j < page0[kk] + npages[kk]) k = kk;
    const int i = j - page0[k];
    const int n = min(16, rec[kCnt + k] - 16 * i);
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
    for (int q = n; q < 16; ++q) {
      a.tokens[(int64_t)row * 16 + q] = -1;
      a.positions[(int64_t)row * 16 + q] = -1;
      if (a.src_rows) a.src_rows[(int64_t)row * 16 + q] = -1;
    }
  }
  // each kept token of the chunk: rank within its tier -> (page, slot)
  const int L = min(a.lens[s], a.max_len), t0 = c * kPlanChunk, t1 = min(L, t0 + kPlanChunk);
  const uint8_t* t_of = a.tier_of + (int64_t)sh * a.tier_stride;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t rb = a.row_base ? a.row_base[sh] : 0;
  for (int b0 = t0; b0 < t1; b0 += kPlanThreads) {
    const int t = b0 + threadIdx.x;
    const int k = t < t1 ? tier_slot(t_of[t]) : -1;
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

int64_t plan_work_ints(int num_sh, int max_len) {
  const int64_t nch = max_len <= 0 ? 1 : (max_len + kPlanChunk - 1) / kPlanChunk;
  return (int64_t)num_sh * kRec + (int64_t)num_sh * nch * kChRec;
}

int launch_plan(const PlanLaunch& L0, int phase, hipStream_t stream) {
  if (L0.num_sh <= 0) return 0;
  PlanLaunch L = L0;
  L.nchunks = L.max_len <= 0 ? 1 : (L.max_len + kPlanChunk - 1) / kPlanChunk;
  const int64_t grid = (int64_t)L.num_sh * L.nchunks;
  if (grid > 0x7FFFFFFF) return -1;
  if (phase == 0) {
    hipLaunchKernelGGL(plan_count_kernel, dim3((unsigned)grid), dim3(kPlanThreads), 0, stream, L);
    hipLaunchKernelGGL(plan_scan_kernel, dim3(1), dim3(kScanThreads), 0, stream, L);
  } else {
    hipLaunchKernelGGL(plan_fill_kernel, dim3((unsigned)grid), dim3(kPlanThreads), 0, stream, L);
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace sphkv
