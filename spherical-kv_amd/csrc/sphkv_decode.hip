// Angle-domain paged attention decode (gfx950).
//
// Work decomposition: one workgroup (4 waves) per work item = a contiguous
// range of pointer-table rows of one (sequence, kv head).  The workgroup
// stages that head's tier codebooks in LDS once; each wave walks every 4th
// page of the range with its own online-softmax state; the four states are
// merged in LDS and written as one (m, l, acc) partial.  A second kernel
// merges the partials of each (sequence, q head) (log-sum-exp) and writes fp16.
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
//      cosine to [-1, 1] only acts on rounding error).
//   3. S[h][t] = q_h . k_rot on MFMA (16x16x32 f16): A = q rows (fp16 input,
//      exact), B = k_rot split into fp16 hi + lo parts (two MFMAs per chunk),
//      so the product carries ~22 bits.
//   4. online softmax in the log2 domain over the page, p rounded to fp16 and
//      the same rounded p summed into l, so the output stays an exact convex
//      combination of V rows.
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
  const _Float16* q;
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

template <int DH, int GQA>
__global__ __launch_bounds__(256) void decode_split_kernel(DecodeArgs a) {
  constexpr int NC = DH / 32;        // 32-dim chunks per lane-token
  constexpr int NP = NC / 2;         // chunks holding the first RoPE half
  constexpr int NM = DH / 16;        // PV MFMA blocks
  constexpr int RG = (GQA + 3) / 4;  // 16-lane row groups holding heads
  using CB = CbLayout<DH>;
  __shared__ __attribute__((aligned(16))) float cb_s[CB::total];
  __shared__ __attribute__((aligned(16))) uint8_t stage[4][512];
  __shared__ __attribute__((aligned(16))) _Float16 pbuf[4][16 * 16];

  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int item = blockIdx.x;
  const int sh = a.work[3 * item];
  const int rb = a.work[3 * item + 1];
  const int re = min(a.work[3 * item + 2], a.num_rows);
  const int h = sh % a.num_kv;
  const int seq = sh / a.num_kv;

  // ---- stage this head's codebooks -----------------------------------------
  for (int tid = 1; tid <= 3; ++tid) {
    const float* src = a.cb[tid];
    if (!src) continue;
    const int n = tid == 1 ? CB::n1 : (tid == 2 ? CB::n2 : CB::n3);
    const float4* s4 = reinterpret_cast<const float4*>(src + (int64_t)h * n);
    float4* d4 = reinterpret_cast<float4*>(cb_s + CB::off(tid));
    for (int i = threadIdx.x; i < n / 4; i += 256) d4[i] = s4[i];
  }
  for (int i = threadIdx.x; i < 4 * 16 * 16; i += 256) (&pbuf[0][0])[i] = (_Float16)0.f;
  __syncthreads();

  const int t = lane & 15;
  const int u = lane >> 4;

  // ---- per-lane constants: query A operand, RoPE frequencies (turns/token) -
  half8 qa[NC];
  {
    const int hr = lane & 15;
    const _Float16* qrow = a.q + ((int64_t)seq * a.num_kv * GQA + (int64_t)h * GQA + hr) * DH;
    for (int c = 0; c < NC; ++c) {
      if (hr < GQA) qa[c] = *reinterpret_cast<const half8*>(qrow + 32 * c + 8 * u);
      else for (int s = 0; s < 8; ++s) qa[c][s] = (_Float16)0.f;
    }
  }
  double fturn[NP][8];
  for (int c = 0; c < NP; ++c)
    for (int s = 0; s < 8; ++s) {
      const int j = 32 * c + 8 * u + s;
      fturn[c][s] = exp2(-(2.0 * j / DH) * a.log2_theta) * 0.15915494309189535;  // / (2 pi)
    }

  // ---- online-softmax state (rows 4u + s of this lane's row group) --------
  float m_run[4], l_run[4];
  for (int s = 0; s < 4; ++s) { m_run[s] = -INFINITY; l_run[s] = 0.f; }
  floatx4 acc[NM];
  for (int mm = 0; mm < NM; ++mm) acc[mm] = (floatx4){0.f, 0.f, 0.f, 0.f};

  uint8_t* st = stage[wave];
  _Float16* pb = pbuf[wave];

  for (int p = rb + wave; p < re; p += 4) {
    const int64_t page_off = a.ptable[3 * p];
    const int64_t th_off = a.ptable[3 * p + 1];
    const int64_t rad_off = a.ptable[3 * p + 2];
    const int64_t vs = a.vslot[p];
    if (page_off < 0 || page_off + 8 > a.pages_bytes || (page_off & 3) || vs < 0 || vs >= a.num_vpages)
      continue;
    const uint32_t hdr = *reinterpret_cast<const uint32_t*>(a.pages + page_off);
    const int tid = uniform(hdr & 0xFF);
    const int n = min(uniform((hdr >> 8) & 0xFF), kTile);
    const int pos = a.positions[(int64_t)p * kTile + t];
    const bool valid = (t < n) && (pos >= 0);

    float k[NC][8];
    if (tid == kDenseTier) {
      const bool ok = (th_off & 15) == 0 && th_off + (int64_t)n * DH * 2 <= a.pages_bytes;
      for (int c = 0; c < NC; ++c) {
        half8 kv;
        if (ok && t < n) kv = *reinterpret_cast<const half8*>(a.pages + th_off + ((int64_t)t * DH + 32 * c + 8 * u) * 2);
        else for (int s = 0; s < 8; ++s) kv[s] = (_Float16)0.f;
        for (int s = 0; s < 8; ++s) k[c][s] = (float)kv[s];
      }
    } else if (tid >= 1 && tid <= 3) {
      // stage [page_off & ~15, +512) in LDS (header, scales, codes, radii)
      const int64_t base = page_off & ~(int64_t)15;
      if (lane < 32) {
        const int64_t src = base + 16 * lane;
        uint4 w = {0u, 0u, 0u, 0u};
        if (src + 16 <= a.pages_bytes) w = *reinterpret_cast<const uint4*>(a.pages + src);
        *reinterpret_cast<uint4*>(st + 16 * lane) = w;
      }
      wave_lds_sync();
      const int g = tier_g(tid), b = tier_b(tid), C = tier_C(tid);
      const int G = DH / g;
      const int rel = (int)(page_off - base);
      const int thr = (int)(th_off - base);
      const int rdr = (int)(rad_off - base);
      const bool ok = thr >= 0 && rdr >= 0 && rdr + n * G <= 512 && thr + (n * G * b + 7) / 8 < 512;
      const float* cbt = cb_s + CB::off(tid);
      for (int c = 0; c < NC; ++c) {
        const int d0 = 32 * c + 8 * u;
        const int gi = d0 / g;
        const int off = d0 - gi * g;
        const int itm = t * G + gi;
        int code = 0;
        float rh = 0.f;
        if (ok && t < n) {
          const int bit = itm * b;
          const int by = thr + (bit >> 3);
          const uint32_t w = (uint32_t)st[by] | ((uint32_t)st[by + 1] << 8);
          code = (int)((w >> (bit & 7)) & (uint32_t)(C - 1));
          const int rc = (int)(int8_t)st[rdr + itm];
          const float sc = *reinterpret_cast<const float*>(st + rel + kHeaderBytes + 4 * gi);
          rh = (float)rc * sc * (1.0f / 127.0f);
        }
        const float4* cen = reinterpret_cast<const float4*>(cbt + (gi * C + code) * g + off);
        const float4 c0 = cen[0], c1 = cen[1];
        k[c][0] = rh * c0.x; k[c][1] = rh * c0.y; k[c][2] = rh * c0.z; k[c][3] = rh * c0.w;
        k[c][4] = rh * c1.x; k[c][5] = rh * c1.y; k[c][6] = rh * c1.z; k[c][7] = rh * c1.w;
      }
    } else {
      continue;
    }

    // ---- RoPE: k_rot = R(pos) k_hat ----------------------------------------
    {
      const double pd = (double)(valid ? pos : 0);
      for (int c = 0; c < NP; ++c)
        for (int s = 0; s < 8; ++s) {
          double ph = pd * fturn[c][s];
          ph -= __builtin_floor(ph);
          const float phf = (float)ph;
          const float sn = __builtin_amdgcn_sinf(phf);
          const float cs = __builtin_amdgcn_cosf(phf);
          const float x0 = k[c][s], x1 = k[c + NP][s];
          k[c][s] = x0 * cs - x1 * sn;
          k[c + NP][s] = x1 * cs + x0 * sn;
        }
    }

    // ---- S = q . k_rot on MFMA, k split into fp16 hi + lo ----------------
    floatx4 S = {0.f, 0.f, 0.f, 0.f};
    for (int c = 0; c < NC; ++c) {
      half8 bh, bl;
      for (int s = 0; s < 8; ++s) {
        const float x = valid ? k[c][s] : 0.f;
        const _Float16 hi = (_Float16)x;
        bh[s] = hi;
        bl[s] = (_Float16)(x - (float)hi);
      }
      S = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[c], bh, S, 0, 0, 0);
      S = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[c], bl, S, 0, 0, 0);
    }

    // ---- online softmax (lanes of row group u hold heads 4u + s) ----------
    // S[s] at lane l is row 4u + s, column (token) t.
    float pv[4];
    float alpha[4];
    for (int s = 0; s < 4; ++s) {
      const float x = valid ? S[s] * a.scale_log2 : -INFINITY;
      float mx = x;
      for (int o = 1; o < 16; o <<= 1) mx = fmaxf(mx, shfl_xor(mx, o));
      const float m_new = fmaxf(m_run[s], mx);
      const float al = (m_new == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(m_run[s] - m_new);
      const float e = (x == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(x - m_new);
      const _Float16 e16 = (_Float16)e;
      float es = (float)e16;
      pv[s] = es;
      for (int o = 1; o < 16; o <<= 1) es += shfl_xor(es, o);
      l_run[s] = al * l_run[s] + es;
      m_run[s] = m_new;
      alpha[s] = al;
    }
    for (int mm = 0; mm < NM; ++mm)
      for (int s = 0; s < 4; ++s) acc[mm][s] *= alpha[s];

    // ---- P^T through LDS into the A-operand layout -----------------------
    if (u < RG)
      for (int s = 0; s < 4; ++s)
        if (4 * u + s < GQA) pb[(4 * u + s) * 16 + t] = (_Float16)pv[s];
    wave_lds_sync();
    const half4 pa = *reinterpret_cast<const half4*>(pb + (lane & 15) * 16 + 4 * u);

    // ---- O += P V on MFMA: B[k = token 4u + i][n = dim 16mm + t] --------
    const uint32_t vmask = (uint32_t)__ballot(valid) & 0xFFFFu;
    const _Float16* vp = a.v_pool + (vs * DH + t) * kTile + 4 * u;
    for (int mm = 0; mm < NM; ++mm) {
      half4 bv = *reinterpret_cast<const half4*>(vp + (int64_t)mm * 16 * kTile);
      if (vmask != 0xFFFFu)
        for (int i = 0; i < 4; ++i)
          if (!((vmask >> (4 * u + i)) & 1u)) bv[i] = (_Float16)0.f;
      acc[mm] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, bv, acc[mm], 0, 0, 0);
    }
    wave_lds_sync();
  }

  // ---- merge the four waves' states in LDS, write one partial -------------
  __syncthreads();
  float* mrg = cb_s;                                  // reuse codebook space
  float* mrg_ml = mrg + 4 * GQA * DH;                 // [4][GQA][2]
  if (u < RG) {
    for (int s = 0; s < 4; ++s) {
      const int hh = 4 * u + s;
      if (hh >= GQA) continue;
      for (int mm = 0; mm < NM; ++mm) mrg[(wave * GQA + hh) * DH + 16 * mm + t] = acc[mm][s];
      if (t == 0) { mrg_ml[(wave * GQA + hh) * 2] = m_run[s]; mrg_ml[(wave * GQA + hh) * 2 + 1] = l_run[s]; }
    }
  }
  __syncthreads();
  float* part = a.partials + (int64_t)item * GQA * (DH + 2);
  for (int i = threadIdx.x; i < GQA * DH; i += 256) {
    const int hh = i / DH, d = i % DH;
    float M = -INFINITY;
    for (int w = 0; w < 4; ++w) M = fmaxf(M, mrg_ml[(w * GQA + hh) * 2]);
    float L = 0.f, A = 0.f;
    if (M != -INFINITY)
      for (int w = 0; w < 4; ++w) {
        const float mw = mrg_ml[(w * GQA + hh) * 2];
        if (mw == -INFINITY) continue;
        const float f = __builtin_amdgcn_exp2f(mw - M);
        L += f * mrg_ml[(w * GQA + hh) * 2 + 1];
        A += f * mrg[(w * GQA + hh) * DH + d];
      }
    part[hh * (DH + 2) + 2 + d] = A;
    if (d == 0) { part[hh * (DH + 2)] = M; part[hh * (DH + 2) + 1] = L; }
  }
}

// Log-sum-exp merge of the partials of each (sequence, q head).
template <int DH, int GQA>
__global__ __launch_bounds__(DH) void decode_merge_kernel(const float* __restrict__ partials,
                                                          const int32_t* __restrict__ work_start,
                                                          int32_t num_kv, _Float16* __restrict__ out) {
  const int qh = blockIdx.x;            // seq * num_kv * GQA + head * GQA + i
  const int sh = qh / GQA, i = qh % GQA;
  const int d = threadIdx.x;
  const int b = work_start[sh], e = work_start[sh + 1];
  float M = -INFINITY;
  for (int it = b; it < e; ++it) M = fmaxf(M, partials[((int64_t)it * GQA + i) * (DH + 2)]);
  float L = 0.f, A = 0.f;
  if (M != -INFINITY)
    for (int it = b; it < e; ++it) {
      const float* pp = partials + ((int64_t)it * GQA + i) * (DH + 2);
      if (pp[0] == -INFINITY) continue;
      const float f = __builtin_amdgcn_exp2f(pp[0] - M);
      L += f * pp[1];
      A += f * pp[2 + d];
    }
  out[(int64_t)qh * DH + d] = (_Float16)(L > 0.f ? A / L : 0.f);
}

template <int DH, int GQA>
static int launch_decode_t(const DecodeLaunch& L, hipStream_t stream) {
  DecodeArgs a;
  a.pages = L.pages; a.pages_bytes = L.pages_bytes; a.ptable = L.ptable; a.vslot = L.vslot;
  a.positions = L.positions; a.v_pool = reinterpret_cast<const _Float16*>(L.v_pool);
  a.num_vpages = L.num_vpages; a.cb[0] = nullptr; a.cb[1] = L.cb1; a.cb[2] = L.cb2; a.cb[3] = L.cb3;
  a.work = L.work; a.q = reinterpret_cast<const _Float16*>(L.q); a.partials = L.partials;
  a.num_kv = L.num_kv; a.num_rows = L.num_rows;
  a.scale_log2 = L.sm_scale * 1.4426950408889634f;
  a.log2_theta = __builtin_log2(L.rope_theta);
  if (L.num_items > 0)
    hipLaunchKernelGGL((decode_split_kernel<DH, GQA>), dim3(L.num_items), dim3(256), 0, stream, a);
  const int nq = L.num_seqs * L.num_kv * GQA;
  if (nq > 0)
    hipLaunchKernelGGL((decode_merge_kernel<DH, GQA>), dim3(nq), dim3(DH), 0, stream, L.partials,
                       L.work_start, L.num_kv, reinterpret_cast<_Float16*>(L.out));
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
