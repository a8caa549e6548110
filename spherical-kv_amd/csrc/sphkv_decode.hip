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

template <int DH>
struct CbLayout {
  static constexpr int n1 = (DH / 16) * 64 * 16;   // tier 1 [G][64][16]
  static constexpr int n2 = (DH / 16) * 16 * 16;   // tier 2 [G][16][16]
  static constexpr int n3 = (DH / 32) * 8 * 32;    // tier 3 [G][8][32]
  static constexpr int total = n1 + n2 + n3;
  __host__ __device__ static constexpr int off(int tid) { return tid == 3 ? n1 + n2 : (tid == 2 ? n1 : 0); }
};

constexpr float kRescaleLog2 = 8.0f;   // reference-max hysteresis (log2 units)

// Pointer-table row of one page, wave-uniform.
struct Row {
  int64_t page_off, th_off, rad_off, vs;
  bool ok;
};

__device__ __forceinline__ Row load_row(const DecodeArgs& a, int p, int re) {
  Row r;
  r.ok = p < re;
  if (r.ok) {
    r.page_off = a.ptable[3 * p];
    r.th_off = a.ptable[3 * p + 1];
    r.rad_off = a.ptable[3 * p + 2];
    r.vs = a.vslot[p];
    r.ok = r.page_off >= 0 && r.page_off + 8 <= a.pages_bytes && (r.page_off & 3) == 0 &&
           r.vs >= 0 && r.vs < a.num_vpages;
  }
  if (!r.ok) { r.page_off = 0; r.th_off = 0; r.rad_off = 0; r.vs = 0; }
  return r;
}

// 512-byte staging window [page_off & ~15, +512) of a page: lanes < 32 hold 16 bytes each.
__device__ __forceinline__ uint4 load_stage(const DecodeArgs& a, const Row& r, int lane) {
  uint4 w = {0u, 0u, 0u, 0u};
  if (r.ok && lane < 32) {
    const int64_t src = (r.page_off & ~(int64_t)15) + 16 * lane;
    if (src + 16 <= a.pages_bytes) w = *reinterpret_cast<const uint4*>(a.pages + src);
  }
  return w;
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

template <int DH, int TID>
__device__ __forceinline__ void gather_k(const float* cb_s, const uint8_t* st, int rel, int thr, int rdr,
                                         int t, int u, int n, bool ok, float (&k)[DH / 32][8]) {
  constexpr int NC = DH / 32;
  constexpr int g = tier_g(TID), C = tier_C(TID);
  int code[NC];
  float rh[NC];
  unpack_page<DH, TID>(st, rel, thr, rdr, t, u, n, ok, code, rh);
  const float* cbt = cb_s + CbLayout<DH>::off(TID);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int d0 = 32 * c + 8 * u;
    const int gi = d0 / g, off = d0 - gi * g;
    const float4* cen = reinterpret_cast<const float4*>(cbt + (gi * C + code[c]) * g + off);
    const float4 c0 = cen[0], c1 = cen[1];
    k[c][0] = rh[c] * c0.x; k[c][1] = rh[c] * c0.y; k[c][2] = rh[c] * c0.z; k[c][3] = rh[c] * c0.w;
    k[c][4] = rh[c] * c1.x; k[c][5] = rh[c] * c1.y; k[c][6] = rh[c] * c1.z; k[c][7] = rh[c] * c1.w;
  }
}

constexpr int kWaves = 8;              // waves per decode workgroup

// Partial of one work item: [16 floats: m[GQA], l[GQA], pad] [acc: GQA * DH]
template <int DH, int GQA>
__host__ __device__ constexpr int partial_stride() { return 16 + GQA * DH; }

template <int DH, int GQA>
__global__ __launch_bounds__(kWaves * 64) void decode_kernel(DecodeArgs a) {
  constexpr int NC = DH / 32;        // 32-dim chunks per lane-token
  constexpr int NP = NC / 2;         // chunks holding the first RoPE half
  constexpr int NM = DH / 16;        // PV MFMA blocks
  constexpr int RG = (GQA + 3) / 4;  // 16-lane row groups holding heads
  using CB = CbLayout<DH>;
  __shared__ __attribute__((aligned(16))) float cb_s[CB::total];
  __shared__ __attribute__((aligned(16))) uint8_t stage[kWaves][512];
  __shared__ __attribute__((aligned(16))) _Float16 pbuf[kWaves][16 * 16];

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

  // ---- pipeline prologue: rows of the first two pages, stage of the first --
  int p = rb + wave;
  Row row_c = load_row(a, p, re);
  Row row_n = load_row(a, p + kWaves, re);
  uint4 stg_c = load_stage(a, row_c, lane);
  int pos_c = row_c.ok ? a.positions[(int64_t)p * kTile + t] : -1;

  // ---- stage this head's codebooks -----------------------------------------
  for (int tid = 1; tid <= 3; ++tid) {
    const float* src = a.cb[tid];
    if (!src) continue;
    const int n = tid == 1 ? CB::n1 : (tid == 2 ? CB::n2 : CB::n3);
    const float4* s4 = reinterpret_cast<const float4*>(src + (int64_t)h * n);
    float4* d4 = reinterpret_cast<float4*>(cb_s + CB::off(tid));
    for (int i = threadIdx.x; i < n / 4; i += kWaves * 64) d4[i] = s4[i];
  }
  for (int i = threadIdx.x; i < kWaves * 16 * 16; i += kWaves * 64) (&pbuf[0][0])[i] = (_Float16)0.f;

  // ---- per-lane constants: query A operand, RoPE frequencies (turns/token) -
  half8 qa[NC];
  {
    const int hr = lane & 15;
    const _Float16* qrow = a.q + ((int64_t)seq * a.num_kv * GQA + (int64_t)h * GQA + hr) * DH;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      if (hr < GQA) qa[c] = *reinterpret_cast<const half8*>(qrow + 32 * c + 8 * u);
      else for (int s = 0; s < 8; ++s) qa[c][s] = (_Float16)0.f;
    }
  }
  double fturn[NP][8];
#pragma unroll
  for (int c = 0; c < NP; ++c)
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int j = 32 * c + 8 * u + s;
      fturn[c][s] = exp2(-(2.0 * j / DH) * a.log2_theta) * 0.15915494309189535;  // / (2 pi)
    }
  __syncthreads();

  float m_run[4], l_run[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) { m_run[s] = -INFINITY; l_run[s] = 0.f; }
  floatx4 acc[NM];
#pragma unroll
  for (int mm = 0; mm < NM; ++mm) acc[mm] = (floatx4){0.f, 0.f, 0.f, 0.f};

  uint8_t* st = stage[wave];
  _Float16* pb = pbuf[wave];

  for (; p < re; p += kWaves) {
    // ---- issue: V of this page, stage/positions of p+4, row of p+8 --------
    half4 vreg[NM];
    {
      const _Float16* vp = a.v_pool + (row_c.vs * DH + t) * kTile + 4 * u;
#pragma unroll
      for (int mm = 0; mm < NM; ++mm) vreg[mm] = *reinterpret_cast<const half4*>(vp + mm * 16 * kTile);
    }
    const uint4 stg_n = load_stage(a, row_n, lane);
    const int pos_n = row_n.ok ? a.positions[(int64_t)(p + kWaves) * kTile + t] : -1;
    const Row row_nn = load_row(a, p + 2 * kWaves, re);

    // ---- this page's header (in lane 0's 16 bytes of the stage) -----------
    const int rel = (int)(row_c.page_off & 15);
    uint32_t hw = rel == 0 ? stg_c.x : (rel == 4 ? stg_c.y : (rel == 8 ? stg_c.z : stg_c.w));
    hw = (uint32_t)__builtin_amdgcn_readfirstlane((int)hw);
    const int tid = row_c.ok ? (int)(hw & 0xFF) : 0;
    const int n = min((int)((hw >> 8) & 0xFF), kTile);
    const bool valid = (t < n) && (pos_c >= 0);

    float k[NC][8];
    if (tid == kDenseTier) {
      const bool ok = (row_c.th_off & 15) == 0 && row_c.th_off + (int64_t)n * DH * 2 <= a.pages_bytes;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        half8 kv;
        if (ok && t < n) kv = *reinterpret_cast<const half8*>(a.pages + row_c.th_off + ((int64_t)t * DH + 32 * c + 8 * u) * 2);
        else for (int s = 0; s < 8; ++s) kv[s] = (_Float16)0.f;
        for (int s = 0; s < 8; ++s) k[c][s] = (float)kv[s];
      }
    } else if (tid >= 1 && tid <= 3) {
      if (lane < 32) *reinterpret_cast<uint4*>(st + 16 * lane) = stg_c;
      wave_lds_sync();
      const int64_t base = row_c.page_off & ~(int64_t)15;
      const int64_t thr64 = row_c.th_off - base, rdr64 = row_c.rad_off - base;
      const int g = tier_g(tid), b = tier_b(tid);
      const int G = DH / g;
      const bool ok = thr64 >= 0 && rdr64 >= 0 && rdr64 + n * G <= 512 && thr64 + (n * G * b + 7) / 8 + 2 < 512;
      const int thr = ok ? (int)thr64 : 0, rdr = ok ? (int)rdr64 : 0;
      if (tid == 1) gather_k<DH, 1>(cb_s, st, rel, thr, rdr, t, u, n, ok, k);
      else if (tid == 2) gather_k<DH, 2>(cb_s, st, rel, thr, rdr, t, u, n, ok, k);
      else gather_k<DH, 3>(cb_s, st, rel, thr, rdr, t, u, n, ok, k);
    } else {
#pragma unroll
      for (int c = 0; c < NC; ++c)
        for (int s = 0; s < 8; ++s) k[c][s] = 0.f;
    }

    // ---- RoPE: k_rot = R(pos) k_hat, then fp16 B operand -------------------
    half8 kb[NC];
    {
      const double pd = (double)(valid ? pos_c : 0);
#pragma unroll
      for (int c = 0; c < NP; ++c)
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const float ph = (float)__builtin_amdgcn_fract(pd * fturn[c][s]);
          const float sn = __builtin_amdgcn_sinf(ph);
          const float cs = __builtin_amdgcn_cosf(ph);
          const float x0 = k[c][s], x1 = k[c + NP][s];
          kb[c][s] = (_Float16)(x0 * cs - x1 * sn);
          kb[c + NP][s] = (_Float16)(x1 * cs + x0 * sn);
        }
    }
    floatx4 S = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NC; ++c) S = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[c], kb[c], S, 0, 0, 0);

    // ---- online softmax (lane row group u holds heads 4u + s, column t) ----
    float pv[4];
    float alpha[4];
    bool any_upd = false;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const float x = valid ? S[s] * a.scale_log2 : -INFINITY;
      float mx = x;
      for (int o = 1; o < 16; o <<= 1) mx = fmaxf(mx, shfl_xor(mx, o));
      const bool upd = mx > m_run[s] + kRescaleLog2;
      const float m_new = upd ? mx : m_run[s];
      alpha[s] = upd ? __builtin_amdgcn_exp2f(m_run[s] - m_new) : 1.f;
      any_upd |= upd;
      const float e = (x == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(x - m_new);
      const _Float16 e16 = (_Float16)e;
      float es = (float)e16;
      pv[s] = es;
      for (int o = 1; o < 16; o <<= 1) es += shfl_xor(es, o);
      l_run[s] = alpha[s] * l_run[s] + es;
      m_run[s] = m_new;
    }
    if (__ballot(any_upd) != 0) {
#pragma unroll
      for (int mm = 0; mm < NM; ++mm)
#pragma unroll
        for (int s = 0; s < 4; ++s) acc[mm][s] *= alpha[s];
    }

    // ---- P^T through LDS into the A-operand layout -----------------------
    if (u < RG) {
#pragma unroll
      for (int s = 0; s < 4; ++s)
        if (4 * u + s < GQA) pb[(4 * u + s) * 16 + t] = (_Float16)pv[s];
    }
    wave_lds_sync();
    const half4 pa = *reinterpret_cast<const half4*>(pb + (lane & 15) * 16 + 4 * u);

    // ---- O += P V on MFMA: B[k = token 4u + i][n = dim 16mm + t] --------
    const uint32_t vmask = (uint32_t)__ballot(valid) & 0xFFFFu;
#pragma unroll
    for (int mm = 0; mm < NM; ++mm) {
      half4 bv = vreg[mm];
      if (vmask != 0xFFFFu)
        for (int i = 0; i < 4; ++i)
          if (!((vmask >> (4 * u + i)) & 1u)) bv[i] = (_Float16)0.f;
      acc[mm] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, bv, acc[mm], 0, 0, 0);
    }
    wave_lds_sync();

    row_c = row_n; row_n = row_nn; stg_c = stg_n; pos_c = pos_n;
  }

  // ---- merge the waves' states in LDS, write this item's partial ----------
  constexpr int PS = partial_stride<DH, GQA>();
  __syncthreads();
  float* mrg = cb_s;                                  // reuse codebook space: [kWaves][GQA][DH]
  float* mrg_ml = mrg + kWaves * GQA * DH;            // [kWaves][GQA][2]
  if (u < RG) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int hh = 4 * u + s;
      if (hh >= GQA) continue;
      for (int mm = 0; mm < NM; ++mm) mrg[(wave * GQA + hh) * DH + 16 * mm + t] = acc[mm][s];
      if (t == 0) { mrg_ml[(wave * GQA + hh) * 2] = m_run[s]; mrg_ml[(wave * GQA + hh) * 2 + 1] = l_run[s]; }
    }
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
