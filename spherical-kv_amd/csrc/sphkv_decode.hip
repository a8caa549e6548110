// Angle-domain paged attention decode (gfx950).
//
// Work decomposition: one workgroup (8 waves) per work item = a contiguous
// range of pointer-table rows of one (sequence, kv head).  The workgroup
// stages that head's tier codebooks in LDS once; each wave walks every 8th
// page of the range with its own online-softmax state; the eight states are
// merged in LDS and written as one (m, l, acc) partial.  A second, widely
// parallel kernel merges the partials of each (sequence, kv head) (log-sum-exp)
// and writes the fp16 output.  (Merging in the last-arriving workgroup needs an
// agent-scope release fence per workgroup, which writes back the XCD's L2 and
// measured tens of microseconds on MI355X.)
//
// Page loop, software pipelined per wave: while page p is computed, the
// 512-byte staging window and positions of the wave's next page and the
// pointer-table row of the one after are in flight, and V of page p is loaded
// before its K math.
//
// Per page (16 tokens), lane l = (token t = l % 16, quarter u = l / 16):
//   1. reconstruct k_hat for dims d = 32c + 8u + s (c < DH/32, s < 8):
//      compressed  k_hat_d = r_hat_g * centroid_g[code][d mod g],
//                  r_hat_g = int8 / 127 * scale_g         (pagebuilder.py:17-21)
//      dense       k_hat_d = K[t][d] (fp16)
//   2. rotate by the token's RoPE angle: k_rot = R(pos) k_hat.  The RoPE pair
//      (j, j + DH/2) lives in chunks c and c + DH/64 of the same lane.
//      <R(-pos) q, k_hat> = <q, R(pos) k_hat>, so this equals the reference's
//      back-rotated query (spherical_kv_pipeline.py:2143-2176; its clip of the
//      cosine to [-1, 1] only acts on rounding error).  The phase pos * f_j is
//      formed in fp64 and reduced to [0, 1) turns before the fp32 sin / cos.
//   3. S[h][t] = q_h . k_rot on MFMA (16x16x32 f16): A = q rows (fp16 input,
//      exact), B = k_rot rounded to fp16 (relative error 2^-11 per element).
//   4. online softmax in the log2 domain.  The running reference max of a head
//      only moves when a page's max exceeds it by more than 2^8, so the
//      accumulator rescale is rare; p = 2^(s - m) <= 256 is rounded to fp16 and
//      the same rounded p is summed into l, so the output stays an exact
//      convex combination of V rows.
//   5. O[h][d] += P[h][t] V[t][d] on MFMA (16x16x16 f16), V read token-minor.
#include "sphkv_common.h"
#include "sphkv_internal.h"

namespace sphkv {

struct DecodeArgs {
  const uint8_t* pages;
  int64_t pages_bytes;
  const int32_t* ptable;
  const int32_t* vslot;
  const int32_t* positions;
  const _Float16* v_pool;
  int64_t num_vpages;
  const float* cb[4];
  const int32_t* work;
  const int32_t* work_start;
  const _Float16* q;
  _Float16* out;
  float* partials;
  int32_t num_kv;
  int32_t num_rows;
  float scale_log2;      // sm_scale * log2(e)
  double log2_theta;
};

// Codebooks in LDS: rows padded by 4 floats (g=16 -> 20, g=32 -> 36) so that
// rows of random codes start in different 16-byte bank slots.
template <int DH>
struct CbLayout {
  __host__ __device__ static constexpr int pad(int g) { return g + 4; }
  static constexpr int n1 = (DH / 16) * 64 * 20;   // tier 1 [G][64][20]
  static constexpr int n2 = (DH / 16) * 16 * 20;   // tier 2 [G][16][20]
  static constexpr int n3 = (DH / 32) * 8 * 36;    // tier 3 [G][8][36]
  static constexpr int total = n1 + n2 + n3;
  __host__ __device__ static constexpr int off(int tid) { return tid == 3 ? n1 + n2 : (tid == 2 ? n1 : 0); }
};

constexpr float kRescaleLog2 = 8.0f;   // reference-max hysteresis (log2 units)

// Every per-page load is a buffer load against a resource that covers exactly
// the bytes that page may need; a resource of 0 bytes makes the load return
// zeros without touching memory.  So each loop iteration issues the same
// loads in the same order whatever the page holds, and the vmcnt waits the
// compiler derives are exact (a branch around a load makes them conservative,
// down to waiting for every prefetch in flight).
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kOOB = 0x7FFFFF00;       // offset beyond any resource

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, int64_t bytes) {
  const uint32_t n = bytes <= 0 ? 0u : (bytes > 0x7FFFFFFF ? 0x7FFFFFFFu : (uint32_t)bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, n, 0x00020000);
}

// Pointer-table row of one page (wave-uniform): lanes 0..2 fetch the row,
// lane 3 the V slot; the values are read out (readlane) only when needed.
struct RowLd { int x, y; };
struct Row {
  int64_t page_off, th_off, rad_off, vs;
  bool ok;
};

__device__ __forceinline__ RowLd row_issue(const DecodeArgs& a, int p, int re, int lane) {
  const bool ok = p < re;
  const rsrc_t rp = make_rsrc(a.ptable + 3 * (int64_t)(ok ? p : 0), ok ? 12 : 0);
  const rsrc_t rv = make_rsrc(a.vslot + (ok ? p : 0), ok ? 4 : 0);
  RowLd l;
  l.x = __builtin_amdgcn_raw_buffer_load_b32(rp, lane < 3 ? 4 * lane : kOOB, 0, 0);
  l.y = __builtin_amdgcn_raw_buffer_load_b32(rv, lane == 3 ? 0 : kOOB, 0, 0);
  return l;
}

__device__ __forceinline__ Row row_take(const DecodeArgs& a, const RowLd& l, int p, int re) {
  Row r;
  r.page_off = __builtin_amdgcn_readlane(l.x, 0);
  r.th_off = __builtin_amdgcn_readlane(l.x, 1);
  r.rad_off = __builtin_amdgcn_readlane(l.x, 2);
  r.vs = __builtin_amdgcn_readlane(l.y, 3);
  r.ok = p < re && r.page_off >= 0 && r.page_off + 8 <= a.pages_bytes && (r.page_off & 3) == 0 &&
         r.vs >= 0 && r.vs < a.num_vpages;
  if (!r.ok) { r.page_off = 0; r.th_off = 0; r.rad_off = 0; r.vs = 0; }
  return r;
}

// A dense page's theta section holds n*DH*2 bytes; a compressed page's at most
// ceil(16*G*b/8) < 2*DH.  Used only to decide what to prefetch; the page header
// decides how the page is processed.
template <int DH>
__device__ __forceinline__ bool row_looks_dense(const Row& r) {
  return r.ok && (r.rad_off - r.th_off) >= 2 * DH && (r.th_off & 15) == 0;
}

// 512-byte staging window [page_off & ~15, +512) of a page: lanes < 32 hold 16 bytes each.
__device__ __forceinline__ uint4 load_stage(const DecodeArgs& a, const Row& r, int lane) {
  const int64_t base = r.page_off & ~(int64_t)15;
  const rsrc_t rs = make_rsrc(a.pages + base, r.ok ? (a.pages_bytes - base < 512 ? a.pages_bytes - base : 512) : 0);
  const auto w = __builtin_amdgcn_raw_buffer_load_b128(rs, lane < 32 ? 16 * lane : kOOB, 0, 0);
  return uint4{(uint32_t)w[0], (uint32_t)w[1], (uint32_t)w[2], (uint32_t)w[3]};
}

__device__ __forceinline__ int load_pos(const DecodeArgs& a, const Row& r, int p, int t) {
  const rsrc_t rs = make_rsrc(a.positions + (int64_t)(r.ok ? p : 0) * kTile, r.ok ? 4 * kTile : 0);
  return __builtin_amdgcn_raw_buffer_load_b32(rs, 4 * t, 0, 0);
}

// V page layout ("MFMA order"): element (token 4u+i, dim 16mm+t) at half offset
// ((t*4 + u) * (DH/16) + mm) * 4 + i, so lane (u, t) reads its PV B operands
// for all mm as DH/2 contiguous bytes.
template <int DH>
__device__ __forceinline__ void load_v(const DecodeArgs& a, const Row& r, int t, int u, half4 (&vreg)[DH / 16]) {
  const rsrc_t rs = make_rsrc(a.v_pool + r.vs * DH * kTile, r.ok ? DH * kTile * 2 : 0);
  const int base = (t * 4 + u) * (DH / 16) * 8;     // bytes
#pragma unroll
  for (int m2 = 0; m2 < DH / 32; ++m2) {
    const auto w = __builtin_amdgcn_raw_buffer_load_b128(rs, base + 16 * m2, 0, 0);
    const uint2 lo = {(uint32_t)w[0], (uint32_t)w[1]}, hi = {(uint32_t)w[2], (uint32_t)w[3]};
    vreg[2 * m2] = __builtin_bit_cast(half4, lo);
    vreg[2 * m2 + 1] = __builtin_bit_cast(half4, hi);
  }
}

// Codes and radii of this lane's NC chunks from the staged page (LDS).
template <int DH, int TID>
__device__ __forceinline__ void unpack_page(const uint8_t* st, int rel, int thr, int rdr, int t, int u,
                                            int n, bool ok, int* code, float* rh) {
  constexpr int NC = DH / 32;
  constexpr int g = tier_g(TID), b = tier_b(TID);
  constexpr int G = DH / g;
  const bool live = ok && t < n;
  uint64_t bits = 0;
  uint32_t rad[2] = {0u, 0u};
  if (live) {
    if constexpr (TID == 1 && G == 8) {            // 48 bits per token at byte 6t (2-aligned)
      const uint16_t* p16 = reinterpret_cast<const uint16_t*>(st + thr + 6 * t);
      bits = (uint64_t)p16[0] | ((uint64_t)p16[1] << 16) | ((uint64_t)p16[2] << 32);
    } else if constexpr (TID == 2 && G == 8) {     // 32 bits per token at byte 4t
      bits = *reinterpret_cast<const uint32_t*>(st + thr + 4 * t);
    } else if constexpr (TID == 1 && G == 4) {     // 24 bits per token at byte 3t
      const uint8_t* p8 = st + thr + 3 * t;
      bits = (uint64_t)p8[0] | ((uint64_t)p8[1] << 8) | ((uint64_t)p8[2] << 16);
    } else if constexpr (TID == 2 && G == 4) {     // 16 bits per token at byte 2t
      bits = *reinterpret_cast<const uint16_t*>(st + thr + 2 * t);
    } else {                                       // tier 3: G*3 bits at bit G*3*t
      const int bit0 = t * G * b;
      const uint8_t* p8 = st + thr + (bit0 >> 3);
      bits = ((uint64_t)p8[0] | ((uint64_t)p8[1] << 8) | ((uint64_t)p8[2] << 16)) >> (bit0 & 7);
    }
    if constexpr (G == 8) {
      rad[0] = *reinterpret_cast<const uint32_t*>(st + rdr + 8 * t);
      rad[1] = *reinterpret_cast<const uint32_t*>(st + rdr + 8 * t + 4);
    } else if constexpr (G == 4) {
      rad[0] = *reinterpret_cast<const uint32_t*>(st + rdr + 4 * t);
    } else {
      rad[0] = *reinterpret_cast<const uint16_t*>(st + rdr + 2 * t);
    }
  }
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int gi = (32 * c + 8 * u) / g;
    code[c] = (int)((bits >> (gi * b)) & ((1u << b) - 1));
    const int rc = (int)(int8_t)((rad[gi >> 2] >> (8 * (gi & 3))) & 0xFFu);
    const float sc = live ? *reinterpret_cast<const float*>(st + rel + kHeaderBytes + 4 * gi) : 0.f;
    rh[c] = (float)rc * sc * (1.0f / 127.0f);
  }
}

// LDS offset (floats) of the centroid chunk a lane needs for chunk c, and
// the radius factor, for every chunk of the page.
template <int DH, int TID>
__device__ __forceinline__ void locate_k(const uint8_t* st, int rel, int thr, int rdr, int t, int u, int n,
                                         bool ok, int (&cofs)[DH / 32], float (&rh)[DH / 32]) {
  constexpr int NC = DH / 32;
  constexpr int g = tier_g(TID), C = tier_C(TID);
  int code[NC];
  unpack_page<DH, TID>(st, rel, thr, rdr, t, u, n, ok, code, rh);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int d0 = 32 * c + 8 * u;
    const int gi = d0 / g, off = d0 - gi * g;
    cofs[c] = CbLayout<DH>::off(TID) + (gi * C + code[c]) * CbLayout<DH>::pad(g) + off;
  }
}

constexpr int kWaves = 12;             // waves per decode workgroup (3 per SIMD)
constexpr int kDelta = 64;             // delta-phasor table rows: |pos - page centre| <= 63

// Partial of one work item: [16 floats: m[GQA], l[GQA], pad] [acc: GQA * DH]
template <int DH, int GQA>
__host__ __device__ constexpr int partial_stride() { return 16 + GQA * DH; }

// Reductions over the four 16-lane rows of a wave (lanes l, l^16, l^32, l^48)
// with the gfx950 row-swap instructions (VALU, no LDS round trip).
// v_permlane32_swap a, b: a's upper 32 lanes <-> b's lower 32 lanes;
// v_permlane16_swap a, b: a's odd rows <-> b's even rows.  With a = b = x the
// sum a + b pairs every lane with its partner row.  Issued as inline asm: the
// clang builtin of this toolchain reads the first result twice when both
// inputs are the same value, and the instructions need the s_nop guard
// (measured: results are wrong without it, right with it).
__device__ __forceinline__ void swap32(float& a, float& b) {
  asm volatile("s_nop 4\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 4" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap16(float& a, float& b) {
  asm volatile("s_nop 4\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 4" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ float rows_max(float x) {
  float a = x, b = x;
  swap32(a, b);
  float c = fmaxf(a, b), d = c;
  swap16(c, d);
  return fmaxf(c, d);
}
__device__ __forceinline__ float rows_sum(float x) {
  float a = x, b = x;
  swap32(a, b);
  float c = a + b, d = c;
  swap16(c, d);
  return c + d;
}

// e^{i 2 pi x} with x a phase in turns (fp32 hardware sine/cosine take turns).
__device__ __forceinline__ float2 turn_phasor(double x) {
  const float ph = (float)__builtin_amdgcn_fract(x);
  return float2{__builtin_amdgcn_cosf(ph), __builtin_amdgcn_sinf(ph)};
}

template <int DH, int GQA>
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(3, 3))) void decode_kernel(DecodeArgs a) {
  constexpr int NC = DH / 32;        // 32-dim chunks per lane-token
  constexpr int NP = NC / 2;         // chunks holding the first RoPE half
  constexpr int NM = DH / 16;        // PV MFMA blocks
  constexpr int NJ = DH / 2;         // RoPE frequencies
  using CB = CbLayout<DH>;
  __shared__ __attribute__((aligned(16))) float cb_s[CB::total];
  __shared__ __attribute__((aligned(16))) float2 dtab[kDelta][NJ + 2]; // e^{i 2pi f_j d}; rows padded 16 B
  __shared__ __attribute__((aligned(16))) double ftab[NJ];             // f_j in turns per token
  __shared__ __attribute__((aligned(16))) uint8_t stage[kWaves][512];
  __shared__ __attribute__((aligned(16))) float2 bbuf[kWaves][NJ];     // page base phasors
  __shared__ __attribute__((aligned(16))) _Float16 q_s[16][DH];        // q rows (rows >= GQA zero)

  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int item = blockIdx.x;
  const int sh = a.work[3 * item];
  const int rb = a.work[3 * item + 1];
  const int re = min(a.work[3 * item + 2], a.num_rows);
  const int h = sh % a.num_kv;
  const int seq = sh / a.num_kv;
  const int t = lane & 15;
  const int u = lane >> 4;

  int p = rb + wave;
  // ---- shared tables: codebooks, RoPE frequencies, delta phasors ---------
  for (int tid = 1; tid <= 3; ++tid) {
    const float* src = a.cb[tid];
    if (!src) continue;
    const int g = tier_g(tid), gp = CB::pad(g);
    const int rows = (DH / g) * tier_C(tid);
    const float4* s4 = reinterpret_cast<const float4*>(src + (int64_t)h * rows * g);
    float* dst = cb_s + CB::off(tid);
    for (int i = threadIdx.x; i < rows * g / 4; i += kWaves * 64) {
      const int r = (4 * i) / g, col = (4 * i) % g;
      *reinterpret_cast<float4*>(dst + r * gp + col) = s4[i];
    }
  }
  if (threadIdx.x < NJ)
    ftab[threadIdx.x] = exp2(-(2.0 * threadIdx.x / DH) * a.log2_theta) * 0.15915494309189535;  // / (2 pi)
  __syncthreads();
  for (int i = threadIdx.x; i < kDelta * NJ; i += kWaves * 64)
    dtab[i / NJ][i % NJ] = turn_phasor((double)(i / NJ) * ftab[i % NJ]);
  {
    const _Float16* qh = a.q + ((int64_t)seq * a.num_kv * GQA + (int64_t)h * GQA) * DH;
    for (int i = threadIdx.x; i < 16 * DH / 8; i += kWaves * 64) {
      const int r = i / (DH / 8), c8 = i % (DH / 8);
      half8 v;
      if (r < GQA) v = *reinterpret_cast<const half8*>(qh + r * DH + 8 * c8);
      else for (int s = 0; s < 8; ++s) v[s] = (_Float16)0.f;
      *reinterpret_cast<half8*>(&q_s[r][8 * c8]) = v;
    }
  }
  const double f_lane = ftab[lane % NJ];
  __syncthreads();
  // everything loaded so far is complete before the page pipeline starts, so
  // no wait inside the loop has to account for it
  __builtin_amdgcn_s_waitcnt(0);

  // ---- pipeline prologue: rows of the first two pages, data of the first --
  Row row_c = row_take(a, row_issue(a, p, re, lane), p, re);
  RowLd rl_n = row_issue(a, p + kWaves, re, lane);
  uint4 stg_c = load_stage(a, row_c, lane);
  int pos_c = load_pos(a, row_c, p, t);
  half4 vreg[NM];
  load_v<DH>(a, row_c, t, u, vreg);
  Row row_n = row_take(a, rl_n, p + kWaves, re);

  // online-softmax state of head hl = lane % 16 (replicated over the 4 rows)
  const int hl = lane & 15;
  float m_run = -INFINITY, l_run = 0.f;
  floatx4 acc[NM];
#pragma unroll
  for (int mm = 0; mm < NM; ++mm) acc[mm] = (floatx4){0.f, 0.f, 0.f, 0.f};

  uint8_t* st = stage[wave];
  float2* bb = bbuf[wave];

  for (; p < re; p += kWaves) {
    // Lane-derived addresses are recomputed each iteration (a few VALU ops)
    // instead of being hoisted out of the loop, where they would not fit in
    // the register budget of 3 waves per SIMD and would be spilled.
    int lane_v = lane;
    asm volatile("" : "+v"(lane_v));
    const int t = lane_v & 15;
    const int u = lane_v >> 4;
    // ---- issue: row two pages ahead, stage/positions one page ahead -------
    const RowLd rl_nn = row_issue(a, p + 2 * kWaves, re, lane);
    const uint4 stg_n = load_stage(a, row_n, lane);
    const int pos_n = load_pos(a, row_n, p + kWaves, t);

    // ---- this page's header (lane 0's 16 bytes of the stage) --------------
    const int rel = (int)(row_c.page_off & 15);
    uint32_t hw = rel == 0 ? stg_c.x : (rel == 4 ? stg_c.y : (rel == 8 ? stg_c.z : stg_c.w));
    hw = (uint32_t)__builtin_amdgcn_readfirstlane((int)hw);
    const int tid = row_c.ok ? (int)(hw & 0xFF) : 0;
    const int n = min((int)((hw >> 8) & 0xFF), kTile);
    if (!row_c.ok) pos_c = -1;
    const bool valid = (t < n) && (pos_c >= 0);

    // ---- page base phasors e^{i 2pi f_j t_mid} (one per lane) -------------
    int t_lo = __builtin_amdgcn_readlane(pos_c, 0);
    int t_hi = __builtin_amdgcn_readlane(pos_c, n > 0 ? n - 1 : 0);
    const int t_mid = (t_lo >= 0 && t_hi >= 0) ? (t_lo + t_hi) >> 1 : max(t_lo, 0);
    if (lane < NJ) bb[lane] = turn_phasor((double)t_mid * f_lane);

    // ---- locate this page's keys: dense rows, or centroid offsets + radii --
    const bool dense = tid == kDenseTier;
    uint4 kd[NC];
    int cofs[NC];
    float rh[NC];
    if (dense) {
      const bool ok = (row_c.th_off & 15) == 0;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int64_t src = row_c.th_off + ((int64_t)t * DH + 32 * c + 8 * u) * 2;
        kd[c] = (ok && t < n && src + 16 <= a.pages_bytes) ? *reinterpret_cast<const uint4*>(a.pages + src)
                                                            : uint4{0u, 0u, 0u, 0u};
        cofs[c] = 0;
        rh[c] = 0.f;
      }
    } else {
#pragma unroll
      for (int c = 0; c < NC; ++c) { cofs[c] = 0; rh[c] = 0.f; kd[c] = uint4{0u, 0u, 0u, 0u}; }
      if (tid >= 1 && tid <= 3) {
        if (lane < 32) *reinterpret_cast<uint4*>(st + 16 * lane) = stg_c;
        wave_lds_sync();
        const int64_t base = row_c.page_off & ~(int64_t)15;
        const int64_t thr64 = row_c.th_off - base, rdr64 = row_c.rad_off - base;
        const int g = tier_g(tid), b = tier_b(tid);
        const int G = DH / g;
        const bool ok = thr64 >= 0 && rdr64 >= 0 && rdr64 + n * G <= 512 && thr64 + (n * G * b + 7) / 8 + 2 < 512;
        const int thr = ok ? (int)thr64 : 0, rdr = ok ? (int)rdr64 : 0;
        if (tid == 1) locate_k<DH, 1>(st, rel, thr, rdr, t, u, n, ok, cofs, rh);
        else if (tid == 2) locate_k<DH, 2>(st, rel, thr, rdr, t, u, n, ok, cofs, rh);
        else locate_k<DH, 3>(st, rel, thr, rdr, t, u, n, ok, cofs, rh);
      }
    }
    wave_lds_sync();

    // ---- RoPE per chunk pair (c, c + NP): k_rot = R(pos) k_hat, phasor =
    //      base(t_mid) * delta(pos - t_mid) -> fp16 MFMA operand -------------
    half8 kb[NC];
    {
      const int dl = pos_c - t_mid;
      const int ad = dl < 0 ? -dl : dl;
      const float sg = dl < 0 ? -1.f : 1.f;
      const bool near = valid && ad < kDelta;
#pragma unroll
      for (int c = 0; c < NP; ++c) {
        float k0[8], k1[8];                      // chunks c and c + NP
        if (dense) {
          const half8 h0 = __builtin_bit_cast(half8, kd[c]), h1 = __builtin_bit_cast(half8, kd[c + NP]);
#pragma unroll
          for (int s = 0; s < 8; ++s) { k0[s] = (float)h0[s]; k1[s] = (float)h1[s]; }
        } else {
          const float4* c0 = reinterpret_cast<const float4*>(cb_s + cofs[c]);
          const float4* c1 = reinterpret_cast<const float4*>(cb_s + cofs[c + NP]);
          const float4 a0 = c0[0], a1 = c0[1], b0 = c1[0], b1 = c1[1];
          const float r0 = rh[c], r1 = rh[c + NP];
          k0[0] = r0 * a0.x; k0[1] = r0 * a0.y; k0[2] = r0 * a0.z; k0[3] = r0 * a0.w;
          k0[4] = r0 * a1.x; k0[5] = r0 * a1.y; k0[6] = r0 * a1.z; k0[7] = r0 * a1.w;
          k1[0] = r1 * b0.x; k1[1] = r1 * b0.y; k1[2] = r1 * b0.z; k1[3] = r1 * b0.w;
          k1[4] = r1 * b1.x; k1[5] = r1 * b1.y; k1[6] = r1 * b1.z; k1[7] = r1 * b1.w;
        }
        const float4* bq = reinterpret_cast<const float4*>(bb + 32 * c + 8 * u);
        const float4* dq = reinterpret_cast<const float4*>(&dtab[near ? ad : 0][32 * c + 8 * u]);
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) {
          const float4 b2 = bq[s2];              // two base phasors (j, j+1)
          float zr[2], zi[2];
          if (near) {
            const float4 d2 = dq[s2];
            const float di0 = sg * d2.y, di1 = sg * d2.w;
            zr[0] = b2.x * d2.x - b2.y * di0; zi[0] = b2.x * di0 + b2.y * d2.x;
            zr[1] = b2.z * d2.z - b2.w * di1; zi[1] = b2.z * di1 + b2.w * d2.z;
          } else {
            const double pd = (double)(valid ? pos_c : 0);
            const float2 z0 = turn_phasor(pd * ftab[32 * c + 8 * u + 2 * s2]);
            const float2 z1 = turn_phasor(pd * ftab[32 * c + 8 * u + 2 * s2 + 1]);
            zr[0] = z0.x; zi[0] = z0.y; zr[1] = z1.x; zi[1] = z1.y;
          }
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const int s = 2 * s2 + e;
            kb[c][s] = (_Float16)(k0[s] * zr[e] - k1[s] * zi[e]);
            kb[c + NP][s] = (_Float16)(k1[s] * zr[e] + k0[s] * zi[e]);
          }
        }
      }
    }
    // ---- S^T = K_rot q^T on MFMA: lane (u, hl) gets head hl, tokens 4u..4u+3
    floatx4 S = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const half8 qa = *reinterpret_cast<const half8*>(&q_s[lane & 15][32 * c + 8 * u]);
      S = __builtin_amdgcn_mfma_f32_16x16x32_f16(kb[c], qa, S, 0, 0, 0);
    }

    // ---- online softmax over the page, per head, in the log2 domain -------
    const uint32_t vmask = (uint32_t)__ballot(valid) & 0xFFFFu;
    float x[4];
#pragma unroll
    for (int s = 0; s < 4; ++s)
      x[s] = ((vmask >> (4 * u + s)) & 1u) ? S[s] * a.scale_log2 : -INFINITY;
    const float mx = rows_max(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])));
    const bool upd = mx > m_run + kRescaleLog2;
    const float m_new = upd ? mx : m_run;
    const float alpha = upd ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.f;
    half4 pa;
    float es = 0.f;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const float e = (x[s] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(x[s] - m_new);
      pa[s] = (_Float16)e;
      es += (float)pa[s];
    }
    l_run = alpha * l_run + rows_sum(es);
    m_run = m_new;
    if (__ballot(upd) != 0) {
#pragma unroll
      for (int mm = 0; mm < NM; ++mm) acc[mm] *= alpha;
    }

    // ---- O^T += V^T P^T on MFMA: A[i = dim 16mm + t][k = token 4u + i'] ----
#pragma unroll
    for (int mm = 0; mm < NM; ++mm) {
      half4 av = vreg[mm];
      if (vmask != 0xFFFFu)
        for (int i = 0; i < 4; ++i)
          if (!((vmask >> (4 * u + i)) & 1u)) av[i] = (_Float16)0.f;
      acc[mm] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, pa, acc[mm], 0, 0, 0);
    }

    // ---- issue V / dense K of the next page into the freed registers ------
    load_v<DH>(a, row_n, t, u, vreg);
    wave_lds_sync();

    row_c = row_n;
    row_n = row_take(a, rl_nn, p + 2 * kWaves, re);
    stg_c = stg_n;
    pos_c = pos_n;
  }

  // ---- merge the waves' states in LDS, write this item's partial ----------
  constexpr int PS = partial_stride<DH, GQA>();
  __syncthreads();
  float* mrg = cb_s;                                  // reuse codebook space: [kWaves][GQA][DH]
  float* mrg_ml = mrg + kWaves * GQA * DH;            // [kWaves][GQA][2]
  if (hl < GQA) {
#pragma unroll
    for (int mm = 0; mm < NM; ++mm)
      *reinterpret_cast<floatx4*>(mrg + (wave * GQA + hl) * DH + 16 * mm + 4 * u) = acc[mm];
    if (u == 0) { mrg_ml[(wave * GQA + hl) * 2] = m_run; mrg_ml[(wave * GQA + hl) * 2 + 1] = l_run; }
  }
  __syncthreads();
  float* part = a.partials + (int64_t)item * PS;
  for (int i = threadIdx.x; i < GQA * DH; i += kWaves * 64) {
    const int hh = i / DH, d = i % DH;
    float M = -INFINITY;
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, mrg_ml[(w * GQA + hh) * 2]);
    float L = 0.f, A = 0.f;
    if (M != -INFINITY)
      for (int w = 0; w < kWaves; ++w) {
        const float mw = mrg_ml[(w * GQA + hh) * 2];
        if (mw == -INFINITY) continue;
        const float f = __builtin_amdgcn_exp2f(mw - M);
        L += f * mrg_ml[(w * GQA + hh) * 2 + 1];
        A += f * mrg[(w * GQA + hh) * DH + d];
      }
    part[16 + hh * DH + d] = A;
    if (d == 0) { part[hh] = M; part[GQA + hh] = L; }
  }
}

// Log-sum-exp merge of the partials of each (sequence, kv head).  One
// workgroup per (sequence, kv head, 128-float slice of its GQA*DH output);
// all loads of a thread are independent (issued together) so the merge costs
// about one memory round trip.
template <int DH, int GQA>
__global__ __launch_bounds__(256) void decode_merge_kernel(const float* __restrict__ partials,
                                                           const int32_t* __restrict__ work_start,
                                                           int32_t num_kv, _Float16* __restrict__ out) {
  constexpr int PS = partial_stride<DH, GQA>();
  constexpr int SL = GQA * DH < 128 ? GQA * DH : 128; // floats per output slice
  constexpr int NSL = (GQA * DH) / SL;                // slices per (seq, kv head)
  constexpr int IL = 8;                               // item lanes: 256 threads = 8 x 32 float4 columns
  __shared__ float ml_s[GQA][2];
  __shared__ float4 red[IL][32];
  __shared__ float mred[256];
  const int sh = blockIdx.x / NSL, slice = blockIdx.x % NSL;
  const int ib = work_start[sh], ni = work_start[sh + 1] - ib;
  const int hh0 = (slice * SL) / DH;                  // first head of this slice
  constexpr int HPS = SL / DH > 0 ? SL / DH : 1;      // heads per slice
  // M and L of the slice's heads: 256 threads stride over (item, head)
  for (int k = 0; k < HPS; ++k) {
    const int hh = hh0 + k;
    float mx = -INFINITY;
    for (int it = threadIdx.x; it < ni; it += 256) mx = fmaxf(mx, partials[(int64_t)(ib + it) * PS + hh]);
    mred[threadIdx.x] = mx;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
      if (threadIdx.x < o) mred[threadIdx.x] = fmaxf(mred[threadIdx.x], mred[threadIdx.x + o]);
      __syncthreads();
    }
    const float M = mred[0];
    __syncthreads();
    float ls = 0.f;
    for (int it = threadIdx.x; it < ni; it += 256) {
      const float* pp = partials + (int64_t)(ib + it) * PS;
      const float mi = pp[hh];
      if (mi != -INFINITY) ls += __builtin_amdgcn_exp2f(mi - M) * pp[GQA + hh];
    }
    mred[threadIdx.x] = ls;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
      if (threadIdx.x < o) mred[threadIdx.x] += mred[threadIdx.x + o];
      __syncthreads();
    }
    if (threadIdx.x == 0) { ml_s[hh][0] = M; ml_s[hh][1] = mred[0]; }
    __syncthreads();
  }
  // weighted sum of the slice: thread = (item lane il, float4 column c)
  const int c = threadIdx.x & 31, il = threadIdx.x >> 5;
  const bool col_ok = 4 * c < SL;
  const int f0 = slice * SL + (col_ok ? 4 * c : 0);   // first float of this column in [GQA*DH]
  const int hh = f0 / DH;
  const float M = ml_s[hh][0];
  float4 sum = {0.f, 0.f, 0.f, 0.f};
  constexpr int UN = 8;
  for (int it0 = il; it0 < ni; it0 += IL * UN) {
    float4 v[UN];
    float mi[UN];
#pragma unroll
    for (int k = 0; k < UN; ++k) {
      const int it = it0 + k * IL;
      const float* pp = partials + (int64_t)(ib + (it < ni ? it : 0)) * PS;
      mi[k] = it < ni ? pp[hh] : -INFINITY;
      v[k] = *reinterpret_cast<const float4*>(pp + 16 + f0);
    }
#pragma unroll
    for (int k = 0; k < UN; ++k) {
      const float f = (mi[k] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(mi[k] - M);
      sum.x += f * v[k].x; sum.y += f * v[k].y; sum.z += f * v[k].z; sum.w += f * v[k].w;
    }
  }
  red[il][c] = sum;
  __syncthreads();
  if (il == 0 && col_ok) {
    float4 tot = red[0][c];
    for (int k = 1; k < IL; ++k) {
      const float4 x = red[k][c];
      tot.x += x.x; tot.y += x.y; tot.z += x.z; tot.w += x.w;
    }
    const float L = ml_s[hh][1];
    const float inv = L > 0.f ? 1.f / L : 0.f;
    half4 o;
    o[0] = (_Float16)(tot.x * inv); o[1] = (_Float16)(tot.y * inv);
    o[2] = (_Float16)(tot.z * inv); o[3] = (_Float16)(tot.w * inv);
    const int seq = sh / num_kv, h = sh % num_kv;
    *reinterpret_cast<half4*>(out + ((int64_t)seq * num_kv * GQA + (int64_t)h * GQA) * DH + f0) = o;
  }
}

template <int DH, int GQA>
static int launch_decode_t(const DecodeLaunch& L, hipStream_t stream) {
  DecodeArgs a;
  a.pages = L.pages; a.pages_bytes = L.pages_bytes; a.ptable = L.ptable; a.vslot = L.vslot;
  a.positions = L.positions; a.v_pool = reinterpret_cast<const _Float16*>(L.v_pool);
  a.num_vpages = L.num_vpages; a.cb[0] = nullptr; a.cb[1] = L.cb1; a.cb[2] = L.cb2; a.cb[3] = L.cb3;
  a.work = L.work; a.work_start = L.work_start; a.q = reinterpret_cast<const _Float16*>(L.q);
  a.out = reinterpret_cast<_Float16*>(L.out); a.partials = L.partials;
  a.num_kv = L.num_kv; a.num_rows = L.num_rows;
  a.scale_log2 = L.sm_scale * 1.4426950408889634f;
  a.log2_theta = __builtin_log2(L.rope_theta);
  if (L.num_items > 0) {
    hipLaunchKernelGGL((decode_kernel<DH, GQA>), dim3(L.num_items), dim3(kWaves * 64), 0, stream, a);
    const int nsh = L.num_seqs * L.num_kv;
    hipLaunchKernelGGL((decode_merge_kernel<DH, GQA>), dim3(nsh * ((GQA * DH) / (GQA * DH < 128 ? GQA * DH : 128))), dim3(256), 0, stream,
                       L.partials, L.work_start, L.num_kv, reinterpret_cast<_Float16*>(L.out));
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_decode(const DecodeLaunch& L, hipStream_t stream) {
#define SPHKV_DISPATCH(D, Q) if (L.dh == D && L.gqa == Q) return launch_decode_t<D, Q>(L, stream);
  SPHKV_DISPATCH(128, 1) SPHKV_DISPATCH(128, 2) SPHKV_DISPATCH(128, 4) SPHKV_DISPATCH(128, 8)
  SPHKV_DISPATCH(64, 1) SPHKV_DISPATCH(64, 2) SPHKV_DISPATCH(64, 4) SPHKV_DISPATCH(64, 8)
#undef SPHKV_DISPATCH
  return -1;
}

// ---------------------------------------------------------------------------
// Logits-only ragged kernel (reference contract of fused_decode_ragged).
// One wave per page; lane = (slot t, dim quarter u); pages of one tier; RoPE
// from the caller's HF-layout tables; fp32 VALU dot products with every q head
// of the page's kv head.  Slots are processed 16 at a time.
__global__ __launch_bounds__(256) void ragged_logits_kernel(RaggedLaunch a) {
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int p = blockIdx.x * 4 + wave;
  if (p >= a.num_pages) return;
  const int t16 = lane & 15, u = lane >> 4;
  const int64_t page_off = a.ptable[3 * p];
  const int64_t th_off = a.ptable[3 * p + 1];
  const int64_t rad_off = a.ptable[3 * p + 2];
  const int G = a.groups, g = a.group_size, b = a.b_theta, dh = a.dh;
  int n = (page_off >= 0 && page_off + 2 <= a.pages_bytes) ? (int)a.pages[page_off + 1] : 0;
  if (n > a.page_size) n = a.page_size;
  if (page_off + kHeaderBytes + 4 * G > a.pages_bytes || th_off < 0 || rad_off < 0 ||
      th_off + ((int64_t)n * G * b + 7) / 8 > a.pages_bytes || rad_off + (int64_t)n * G > a.pages_bytes)
    n = 0;
  const int C = 1 << b;
  const int hk = a.head_ids[p];
  const int dq = dh / 4;               // dims per lane
  const int half_dh = dh / 2;
  const int64_t total_slots = (int64_t)a.num_pages * a.page_size;
  for (int t0 = 0; t0 < a.page_size; t0 += 16) {
    const int t = t0 + t16;
    const bool in_page = t < a.page_size;
    const int pos = in_page ? a.positions[(int64_t)p * a.page_size + t] : -1;
    const bool valid = in_page && t < n && pos >= 0 && pos < a.max_pos && hk >= 0 && hk < a.num_kv;
    // lane covers RoPE pairs j = u*dq/2 .. +dq/2 of the first half and their partners
    float kr[64];
    const int j0 = u * (dq / 2);
    for (int jj = 0; jj < dq / 2; ++jj) {
      float x0 = 0.f, x1 = 0.f;
      if (valid) {
        for (int hlf = 0; hlf < 2; ++hlf) {
          const int d = j0 + jj + hlf * half_dh;
          const int gi = d / g, off = d % g;
          const int itm = t * G + gi;
          const int64_t bit = (int64_t)itm * b;
          const int64_t by = th_off + (bit >> 3);
          uint32_t w = a.pages[by];
          if (by + 1 < a.pages_bytes) w |= (uint32_t)a.pages[by + 1] << 8;
          const int code = (int)((w >> (bit & 7)) & (uint32_t)(C - 1));
          const int rc = (int)(int8_t)a.pages[rad_off + itm];
          float sc;
          __builtin_memcpy(&sc, a.pages + page_off + kHeaderBytes + 4 * gi, 4);
          const float x = (float)rc * sc * (1.0f / 127.0f) *
                          a.codebooks[(((int64_t)hk * G + gi) * C + code) * g + off];
          if (hlf == 0) x0 = x; else x1 = x;
        }
        const float cs = a.cos_tbl[(int64_t)pos * dh + j0 + jj];
        const float sn = a.sin_tbl[(int64_t)pos * dh + j0 + jj];
        kr[jj] = x0 * cs - x1 * sn;
        kr[dq / 2 + jj] = x1 * cs + x0 * sn;
      } else {
        kr[jj] = 0.f;
        kr[dq / 2 + jj] = 0.f;
      }
    }
    for (int i = 0; i < a.grp; ++i) {
      float sacc = 0.f;
      if (hk >= 0 && hk < a.num_kv) {
        const float* qr = a.q + ((int64_t)hk * a.grp + i) * dh;
        for (int jj = 0; jj < dq / 2; ++jj)
          sacc += qr[j0 + jj] * kr[jj] + qr[j0 + jj + half_dh] * kr[dq / 2 + jj];
      }
      sacc += shfl_xor(sacc, 16);
      sacc += shfl_xor(sacc, 32);
      if (u == 0 && in_page)
        a.logits_out[(int64_t)i * total_slots + (int64_t)p * a.page_size + t] =
            valid ? sacc * (1.0f / __builtin_sqrtf((float)dh)) : -INFINITY;
    }
  }
}

int launch_ragged(const RaggedLaunch& L, hipStream_t stream) {
  if (L.num_pages > 0)
    hipLaunchKernelGGL(ragged_logits_kernel, dim3((L.num_pages + 3) / 4), dim3(256), 0, stream, L);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace sphkv
