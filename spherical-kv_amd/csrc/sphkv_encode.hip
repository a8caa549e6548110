// Fused encode + bitpack + page build + V placement (gfx950).
//
// One 8-wave workgroup per four consecutive pages: one lane per token, one
// wave per group in the nearest-centroid phase, then one wave per page for
// the page build and one per page for its V placement.  Per (token, group)
// the radius, direction and code reproduce torch CPU's operation order of
// _encode_keys_with_codebooks (spherical_kv_pipeline.py:1136-1144) bit for
// bit:
//   r    = sqrtf(sum over 8 lanes of fmaf(x, x, .) chains, lanes summed in order)
//   dir  = x / (r + 1e-8f)                     (IEEE division)
//   code = first index of the maximum similarity, where the similarity is
//          scored in the order of the torch path the page's size selects
//          (code_sim / code_sim_m1 below).
// The g = 16 tiers (1, 2) first rank all codes on v_mfma_f32_16x16x16_f16
// with fp16 copies of the direction and the codebook rows (LDS); only the
// codes within a proven error bound of the approximate maximum are then scored
// exactly.  The g = 32 tier (3) scores every code exactly with the codebook
// rows as scalar operands.  The page of pagebuilder.py:8-33 (header, fp32
// scales, LSB-first theta codes, int8 radius codes) is built in LDS and
// stored.  This file is compiled with -ffp-contract=off so no multiply/add
// pair is fused except where fmaf is written.
#include "sphkv_common.h"
#include "sphkv_internal.h"

namespace sphkv {

struct EncodeArgs {
  const void* k;
  int32_t k_is_fp32;
  const __half* v;
  int64_t num_src_rows;
  const int64_t* src_rows;
  const int32_t* tier;
  const int32_t* count;
  const int32_t* ptable;
  const int32_t* vslot;
  const int32_t* seq_head;
  int32_t num_pages;
  int32_t num_kv;
  const float* cb[4];
  uint8_t* pages;
  int64_t pages_bytes;
  __half* v_pool;
  int64_t num_vpages;
  float* r_out;
  int32_t* code_out;
  const int32_t* order_n;   // per page: N of the torch call whose summation order applies (NULL: count)
  int32_t codes_only;       // 1: write r_out / code_out only (no pages, no V)
};

template <int DH>
__device__ __forceinline__ void load_group(const EncodeArgs& a, int64_t row, int col0, int g, float* x) {
  if (a.k_is_fp32) {
    const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(a.k) + row * DH + col0);
    for (int i = 0; i < g / 4; ++i) {
      float4 v4 = src[i];
      x[4 * i] = v4.x; x[4 * i + 1] = v4.y; x[4 * i + 2] = v4.z; x[4 * i + 3] = v4.w;
    }
  } else {
    const half8* src = reinterpret_cast<const half8*>(static_cast<const __half*>(a.k) + row * DH + col0);
    for (int i = 0; i < g / 8; ++i) {
      half8 h = src[i];
      for (int j = 0; j < 8; ++j) x[8 * i + j] = (float)h[j];
    }
  }
}

typedef const float __attribute__((address_space(4)))* cb_ptr;   // read through the scalar cache

constexpr int kEncWaves = 8;       // waves per workgroup: one per group in the argmax phase
constexpr int kEncPages = 4;       // pages per workgroup: one lane per token of four pages
constexpr int kEncMaxG = 8;        // groups per token (dh / g)

constexpr int kCbRow = 20;         // floats per staged codebook row (16 + pad)

template <int DH>
struct EncodeLds {
  float r[kEncPages * kTile][kEncMaxG];        // radius of (token, group)
  int32_t code[kEncPages * kTile][kEncMaxG];   // code of (token, group)
  union {
    struct {                                   // argmax phase, per wave (group)
      float cb[kEncWaves][64][kCbRow];                  // the group's codebook rows (g = 16 tiers)
      _Float16 dh[kEncWaves][kEncPages * kTile][20];    // fp16 direction, token-major (rows padded)
    } arg;
    struct {                                   // build phase
      uint8_t stage[kEncPages][512];           // page images
      _Float16 vt[kEncPages][DH * kTile];      // V pages, dim-major
    } build;
  } u;
};

// Nearest-centroid search of the g = 16 tiers in two stages, with the
// group's codebook rows staged in LDS once per (tier, kv head) run.
//  1. Approximate similarities of 16 tokens x 16 codes per
//     v_mfma_f32_16x16x16_f16, from fp16 copies of the direction and the
//     codebook rows.  Both are unit vectors, so |approx - s| <= 2^-10 from the
//     two fp16 roundings (sum_i |d_i c_i| <= |d| |c| <= 1), plus at most
//     16 * 2^-14 if the unit flushes fp16 denormals, plus the fp32 rounding of
//     the chains (< 1e-5): eps < 2.1e-3, where s is the exact fp32 score.
//  2. Every code c with approx_c >= max_approx - kCandSlack (>= 2 eps) is
//     scored exactly (the torch-order chain below), in ascending order; the
//     first maximum among them is the first maximum over all codes, because
//     every code whose exact score equals the exact maximum passes the test.
//     No candidate (NaN similarities) falls back to scoring every code.
constexpr float kCandSlack = 5e-3f;
// The bound above scales with |c|: it holds, inside the slack, for rows with
// |c|^2 within kUnitTol of 1.  A staged codebook with any other row (scaled
// or unnormalised rows: _encode_keys_with_codebooks accepts any codebook,
// only codebook_loader.py:43-44 normalises) is scored exactly over every
// code.
constexpr float kUnitTol = 0.1f;

// Does any staged row (lane < C: its 16 values) leave the unit-row bound?
__device__ __forceinline__ bool rows_not_unit(const float4 (&row)[4], int lane, int C) {
  float n2 = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) n2 += row[i].x * row[i].x + row[i].y * row[i].y + row[i].z * row[i].z + row[i].w * row[i].w;
  return __builtin_amdgcn_ballot_w64(lane < C && !(fabsf(n2 - 1.f) <= kUnitTol)) != 0;   // NaN: not unit
}

// Nearest centroid of one (token, group) against the codebook rows cbg[c * GG ..]
// (wave-uniform, so every centroid coordinate is a scalar operand): the fmaf
// chain over i of torch's batched path, or its separate multiply and add when
// the page is small (N*g*C < 400); first index of the maximum, codes scored in
// ascending order.
template <int GG, bool NAIVE>
__device__ __forceinline__ float code_sim(const float* dir, const float* w) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < GG; ++i) {
    if (NAIVE) s = __fadd_rn(s, __fmul_rn(dir[i], w[i]));
    else s = __builtin_fmaf(dir[i], w[i], s);
  }
  return s;
}

// torch's N = 1 path for a contraction of 16 with C = 64 (tier 1, one token:
// N*g*C >= 400 with M = 1) runs MKL's M = 1 sgemm kernel, whose order is
//   s01 = fmaf(d1, c1, d0*c0); L_l = d_{l+2}c_{l+2} + d_{l+10}c_{l+10} (l < 6);
//   L_6 = d8 c8; L_7 = d9 c9 + s01; M_l = L_l + L_{l+4}; (M_0 + M_2) + (M_1 + M_3)
// (identified with exact power-of-two probes against torch 2.10 / oneMKL
// 2024.2 and pinned by near-tie single-token fixtures).
__device__ __forceinline__ float code_sim_m1(const float* d, const float* c) {
  float L[8];
  const float s01 = __builtin_fmaf(d[1], c[1], __fmul_rn(d[0], c[0]));
#pragma unroll
  for (int l = 0; l < 6; ++l) L[l] = __fadd_rn(__fmul_rn(d[l + 2], c[l + 2]), __fmul_rn(d[l + 10], c[l + 10]));
  L[6] = __fmul_rn(d[8], c[8]);
  L[7] = __fadd_rn(__fmul_rn(d[9], c[9]), s01);
  float M[4];
#pragma unroll
  for (int l = 0; l < 4; ++l) M[l] = __fadd_rn(L[l], L[l + 4]);
  return __fadd_rn(__fadd_rn(M[0], M[2]), __fadd_rn(M[1], M[3]));
}

// Codes are scored in batches of NB rows (NB * GG = 64 floats, the scalar
// registers one batch holds): scalar loads return in any order, so a batch's
// rows are waited for together and their NB chains run side by side.
template <int GG, bool NAIVE>
__device__ __forceinline__ int argmax_codes(const float* dir, cb_ptr cbg, int C) {
  constexpr int NB = 64 / GG;
  float best_sim = 0.f;
  int best = 0;
  for (int c = 0; c < C; c += NB) {
    float w[NB][GG];
#pragma unroll
    for (int q = 0; q < NB; ++q)
#pragma unroll
      for (int i = 0; i < GG; ++i) w[q][i] = cbg[(c + q) * GG + i];
    float sim[NB];
#pragma unroll
    for (int q = 0; q < NB; ++q) sim[q] = code_sim<GG, NAIVE>(dir, w[q]);
#pragma unroll
    for (int q = 0; q < NB; ++q)
      if (c + q == 0 || sim[q] > best_sim) { best_sim = sim[q]; best = c + q; }
  }
  return best;
}

// Radius (torch_norm) and code of the group of GG values at element kofs of K.
template <int GG>
__device__ __forceinline__ void encode_group(const EncodeArgs& a, int64_t kofs, bool naive, cb_ptr cbg, int C,
                                             float& r_out, int& code_out) {
  float x[GG];
  if (a.k_is_fp32) {
    const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(a.k) + kofs);
#pragma unroll
    for (int i = 0; i < GG / 4; ++i) {
      const float4 v4 = src[i];
      x[4 * i] = v4.x; x[4 * i + 1] = v4.y; x[4 * i + 2] = v4.z; x[4 * i + 3] = v4.w;
    }
  } else {
    const half8* src = reinterpret_cast<const half8*>(static_cast<const __half*>(a.k) + kofs);
#pragma unroll
    for (int i = 0; i < GG / 8; ++i) {
      const half8 hv = src[i];
#pragma unroll
      for (int e = 0; e < 8; ++e) x[8 * i + e] = (float)hv[e];
    }
  }
  const float r = torch_norm(x, GG);
  const float den = __fadd_rn(r, 1e-8f);
  float dir[GG];
  group_directions<GG>(x, den, !a.k_is_fp32, dir);
  r_out = r;
  code_out = naive ? argmax_codes<GG, true>(dir, cbg, C) : argmax_codes<GG, false>(dir, cbg, C);
}

// One workgroup per four consecutive pages; lane = token (page slot j =
// lane / 16, token t = lane % 16).  Argmax phase: wave w encodes group w of
// every token, with the codebook of a (tier, kv head) as scalar operands; the
// lanes whose page shares the first unhandled page's (tier, head) go
// together, so four pages of one run take one pass.  Build phase: wave j < 4
// builds page j in LDS (header, scales, LSB-first codes, int8 radius codes;
// pagebuilder.py:8-33) and stores it, or copies a dense page's fp16 K rows;
// wave 4 + j places page j's V rows dim-major.
template <int DH>
__global__ __launch_bounds__(kEncWaves * 64) void encode_pages_kernel(EncodeArgs a) {
  __shared__ EncodeLds<DH> sm;
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int p0 = blockIdx.x * kEncPages;                          // the workgroup's first page

  // ---- argmax phase: group `wave` of this lane's token ---------------------
  {
    const int j = lane >> 4, t = lane & 15;
    const int p = p0 + j;
    const bool p_ok = p < a.num_pages;
    // the token's source row is loaded together with the page's metadata (its
    // address does not depend on them) and masked by the count afterwards
    const int64_t row_raw = p_ok ? a.src_rows[(int64_t)p * kTile + t] : -1;
    const int tid_l = p_ok ? a.tier[p] : 0;
    const int n_l = p_ok ? min(max(a.count[p], 0), kTile) : 0;
    // the summation order follows torch's call over ord_l tokens: the page's
    // own count, or the caller's N (a whole head's tokens in one call)
    const int ord_l = p_ok ? (a.order_n ? max(a.order_n[p], 1) : n_l) : 0;
    const int sh_l = p_ok ? a.seq_head[p] : -1;
    const int head_l = sh_l >= 0 ? sh_l % a.num_kv : 0;
    int64_t row = t < n_l ? row_raw : -1;
    if (row >= a.num_src_rows) row = -1;
    // a page is encoded only with its tier's codebook and a valid (seq, head)
    const bool comp_l = tid_l >= 1 && tid_l <= 3 && wave < DH / tier_g(tid_l) && sh_l >= 0 &&
                        a.cb[tid_l >= 1 && tid_l <= 3 ? tid_l : 0] != nullptr;
    const int gi = wave;
    // ---- g = 16 tiers (1, 2): MFMA similarities, exact scores for candidates
    const bool m16_l = comp_l && tier_g(tid_l) == 16;
    const uint64_t m16 = __builtin_amdgcn_ballot_w64(m16_l);
    if (m16) {
      const bool live = m16_l && row >= 0;
      const int tl = lane & 15, kg = lane >> 4;
      float (*cbs)[kCbRow] = sm.u.arg.cb[wave];
      // codebook rows of the first g = 16 page's (tier, head), loaded before K
      const int j0 = (int)__builtin_ctzll(m16) >> 4;
      const int tid0 = uniform(__builtin_amdgcn_readlane(tid_l, 16 * j0));
      const int h0 = uniform(__builtin_amdgcn_readlane(head_l, 16 * j0));
      const int C0 = tier_C(tid0);                                  // 64 or 16
      float4 crow[4];
      {
        const float* cbg = a.cb[tid0] + ((int64_t)h0 * (DH / 16) + gi) * C0 * 16;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          crow[i] = lane < C0 ? *reinterpret_cast<const float4*>(cbg + lane * 16 + 4 * i) : float4{0.f, 0.f, 0.f, 0.f};
      }
      bool exact_all = rows_not_unit(crow, lane, C0);
      // do all g = 16 pages of the workgroup use (tid0, h0)?
      bool same = true;
#pragma unroll
      for (int jj = 0; jj < kEncPages; ++jj)
        if ((m16 >> (16 * jj)) & 0xFFFFull)
          same = same && __builtin_amdgcn_readlane(tid_l, 16 * jj) == tid0 &&
                 __builtin_amdgcn_readlane(head_l, 16 * jj) == h0;
      float dir[16];
      float r = 0.f;
      {
        float x[16];
        if (live) {
          const int64_t kofs = row * DH + gi * 16;
          if (a.k_is_fp32) {
            const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(a.k) + kofs);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float4 v4 = src[i];
              x[4 * i] = v4.x; x[4 * i + 1] = v4.y; x[4 * i + 2] = v4.z; x[4 * i + 3] = v4.w;
            }
          } else {
            const half8* src = reinterpret_cast<const half8*>(static_cast<const __half*>(a.k) + kofs);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
              const half8 hv = src[i];
#pragma unroll
              for (int e = 0; e < 8; ++e) x[8 * i + e] = (float)hv[e];
            }
          }
        } else {
#pragma unroll
          for (int i = 0; i < 16; ++i) x[i] = 0.f;
        }
        r = live ? torch_norm(x, 16) : 0.f;
        const float den = __fadd_rn(r, 1e-8f);
        group_directions<16>(x, den, !a.k_is_fp32, dir);         // x = 0 (dir = +0) where not live
      }
      {
        _Float16* d = sm.u.arg.dh[wave][lane];
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4)
          *reinterpret_cast<half4*>(d + 4 * q4) = half4{(_Float16)dir[4 * q4], (_Float16)dir[4 * q4 + 1],
                                                        (_Float16)dir[4 * q4 + 2], (_Float16)dir[4 * q4 + 3]};
      }
      if (lane < C0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) *reinterpret_cast<float4*>(&cbs[lane][4 * i]) = crow[i];
      }
      wave_lds_sync();
      // candidate codes of 16 tokens of page jj against the staged rows (A
      // operands, codes 16 b + row); lane (tl, kg) ends with token tl's mask
      auto page_masks = [&](int jj, int C, const half4 (&A)[4], uint32_t& lo, uint32_t& hi) {
        const half4 B = *reinterpret_cast<const half4*>(sm.u.arg.dh[wave][16 * jj + tl] + 4 * kg);
        floatx4 D[4];
        float mloc = -INFINITY;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          if (16 * b < C) {
            D[b] = __builtin_amdgcn_mfma_f32_16x16x16f16(A[b], B, (floatx4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) mloc = fmaxf(mloc, D[b][i]);    // D[b][i]: code 16 b + 4 kg + i, token tl
          }
        }
        const float thr = rows_max(mloc) - kCandSlack;
        lo = 0u;
        hi = 0u;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          if (16 * b < C) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int c = 16 * b + 4 * kg + i;
              if (D[b][i] >= thr) {
                if (c < 32) lo |= 1u << c;
                else hi |= 1u << (c - 32);
              }
            }
          }
        }
        lo = rows_or(lo);
        hi = rows_or(hi);
      };
      auto load_A = [&](int C, half4 (&A)[4]) {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const float4 cv = 16 * b < C ? *reinterpret_cast<const float4*>(&cbs[16 * b + tl][4 * kg]) : float4{0.f, 0.f, 0.f, 0.f};
          A[b] = half4{(_Float16)cv.x, (_Float16)cv.y, (_Float16)cv.z, (_Float16)cv.w};
        }
      };
      // exact scores of this lane's token over the codes of mask (lo, hi)
      auto score = [&](uint32_t lo, uint32_t hi, int C) {
        uint64_t mk = (uint64_t)lo | ((uint64_t)hi << 32);
        if (C < 64) mk &= (1ull << C) - 1;
        if (mk == 0 || exact_all) mk = C == 64 ? ~0ull : ((1ull << C) - 1);   // NaN similarities or
                                                                                // non-unit rows: every code
        const bool naive = ord_l * 16 * C < 400;                     // torch's own small-bmm loop
        const bool m1 = !naive && ord_l == 1;                        // MKL's M = 1 kernel
        float best_sim = 0.f;
        int best = -1;
        while (mk) {
          const int c = (int)__builtin_ctzll(mk);
          mk &= mk - 1;
          float w[16];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float4 v4 = *reinterpret_cast<const float4*>(&cbs[c][4 * i]);
            w[4 * i] = v4.x; w[4 * i + 1] = v4.y; w[4 * i + 2] = v4.z; w[4 * i + 3] = v4.w;
          }
          const float sc = naive ? code_sim<16, true>(dir, w) : (m1 ? code_sim_m1(dir, w) : code_sim<16, false>(dir, w));
          if (best < 0 || sc > best_sim) { best_sim = sc; best = c; }
        }
        return best;
      };
      if (same) {
        // one set of A operands and one exact pass for all four pages
        half4 A[4];
        load_A(C0, A);
        uint32_t mlo = 0u, mhi = 0u;
#pragma unroll
        for (int jj = 0; jj < kEncPages; ++jj) {
          if (((m16 >> (16 * jj)) & 0xFFFFull) == 0) continue;
          uint32_t lo, hi;
          page_masks(jj, C0, A, lo, hi);
          if ((lane >> 4) == jj) { mlo = lo; mhi = hi; }               // lane 16 jj + t: token t of page jj
        }
        if (live) {
          sm.r[lane][gi] = r;
          sm.code[lane][gi] = score(mlo, mhi, C0);
        }
      } else {
        // pages of several (tier, head) runs: one page at a time, restaging
        int st_tid = tid0, st_h = h0;
        for (int jj = 0; jj < kEncPages; ++jj) {
          if (((m16 >> (16 * jj)) & 0xFFFFull) == 0) continue;
          const int tid = uniform(__builtin_amdgcn_readlane(tid_l, 16 * jj));
          const int h = uniform(__builtin_amdgcn_readlane(head_l, 16 * jj));
          const int C = tier_C(tid);
          if (tid != st_tid || h != st_h) {
            wave_lds_sync();
            const float* cbg = a.cb[tid] + ((int64_t)h * (DH / 16) + gi) * C * 16;
            float4 row[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
              row[i] = lane < C ? *reinterpret_cast<const float4*>(cbg + lane * 16 + 4 * i) : float4{0.f, 0.f, 0.f, 0.f};
            if (lane < C) {
#pragma unroll
              for (int i = 0; i < 4; ++i) *reinterpret_cast<float4*>(&cbs[lane][4 * i]) = row[i];
            }
            exact_all = rows_not_unit(row, lane, C);
            st_tid = tid;
            st_h = h;
            wave_lds_sync();
          }
          half4 A[4];
          load_A(C, A);
          uint32_t lo, hi;
          page_masks(jj, C, A, lo, hi);
          if (live && (lane >> 4) == jj) {
            sm.r[lane][gi] = r;
            sm.code[lane][gi] = score(lo, hi, C);
          }
        }
      }
      if (m16_l && !live) {
        sm.r[lane][gi] = 0.f;
        sm.code[lane][gi] = 0;
      }
    }
    // ---- other tiers (g = 32): exact scan with scalar codebook rows
    uint64_t todo = __builtin_amdgcn_ballot_w64(comp_l && !m16_l);
    while (todo) {
      const int lead = (int)__builtin_ctzll(todo);                 // first lane not yet encoded
      const int tid = uniform(__builtin_amdgcn_readlane(tid_l, lead));
      const int h = uniform(__builtin_amdgcn_readlane(head_l, lead));
      const bool mine = comp_l && !m16_l && tid_l == tid && head_l == h;
      todo &= ~__builtin_amdgcn_ballot_w64(mine);
      const int g = uniform(tier_g(tid)), C = uniform(tier_C(tid)), G = DH / g;
      const uint64_t cba = (uint64_t)(a.cb[tid] + ((int64_t)h * G + gi) * C * g);
      const cb_ptr cbg = (cb_ptr)(((uint64_t)(uint32_t)uniform((int)(cba >> 32)) << 32) |
                                  (uint32_t)uniform((int)(uint32_t)cba));
      if (mine) {
        const bool naive = ord_l * g * C < 400;                   // torch's own small-bmm loop
        float r = 0.f;
        int code = 0;
        if (row >= 0) {
          if (g == 16) encode_group<16>(a, row * DH + gi * 16, naive, cbg, C, r, code);
          else encode_group<32>(a, row * DH + gi * 32, naive, cbg, C, r, code);
        }
        sm.r[lane][gi] = r;
        sm.code[lane][gi] = code;
      }
    }
  }
  __syncthreads();

  if (a.codes_only) {
    // radii and codes of every (token, group) of the workgroup's compressed
    // pages, [page][slot][DH / 16]
    const int j = threadIdx.x >> 4 & 3, t = threadIdx.x & 15, gbase = threadIdx.x >> 6;
    const int p = p0 + j;
    if (p >= a.num_pages) return;
    const int tid = a.tier[p];
    if (tid < 1 || tid > 3 || t >= min(max(a.count[p], 0), kTile)) return;
    for (int gi = gbase; gi < DH / tier_g(tid); gi += kEncWaves) {
      const int64_t o = ((int64_t)p * kTile + t) * (DH / 16) + gi;
      if (a.r_out) a.r_out[o] = sm.r[16 * j + t][gi];
      if (a.code_out) a.code_out[o] = sm.code[16 * j + t][gi];
    }
    return;
  }

  const int j = wave & 3;
  const int p = p0 + j;
  if (p >= a.num_pages) return;
  const int tid = a.tier[p];
  const int n = min(max(a.count[p], 0), kTile);
  const int t = lane & 15, gs = lane >> 4;
  const bool tok_ok = t < n;

  if (wave >= kEncPages) {
    // ---- V of page j: lane (token t, quarter gs) loads DH / 4 dims of its
    // row into LDS dim-major (element (token k, dim d) at d * 16 + k), then
    // the wave stores whole 32-byte dim rows
    const int64_t vs = a.vslot[p];
    if (vs < 0 || vs >= a.num_vpages) return;
    _Float16* vt = sm.u.build.vt[j];
    int64_t vr = tok_ok ? a.src_rows[(int64_t)p * kTile + t] : -1;
    if (vr >= a.num_src_rows) vr = -1;
    constexpr int QD = DH / 4;
#pragma unroll
    for (int c8 = 0; c8 < QD / 8; ++c8) {
      const int d0 = gs * QD + c8 * 8;
      half8 hv;
      if (vr >= 0) {
        hv = *reinterpret_cast<const half8*>(a.v + vr * DH + d0);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) hv[e] = (_Float16)0.f;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) vt[(d0 + e) * kTile + t] = hv[e];
    }
    wave_lds_sync();
    half8* dst = reinterpret_cast<half8*>(a.v_pool + vs * DH * kTile);
    for (int i = lane; i < DH * kTile / 8; i += kWave) dst[i] = *reinterpret_cast<const half8*>(vt + 8 * i);
    return;
  }

  // ---- page j ---------------------------------------------------------------
  const int64_t page_off = a.ptable[3 * p];
  const int64_t th_off = a.ptable[3 * p + 1];
  if (tid == kDenseTier) {
    // header: tier id, count, six zero bytes; payload fp16 [n, DH] at a
    // 16-byte aligned theta offset.  A pointer-table row that does not place
    // the whole page inside the byte pool (negative or misaligned offsets
    // included) writes nothing, as a compressed page's does.
    if (page_off < 0 || page_off + 8 > a.pages_bytes || th_off < page_off + 8 || (th_off & 15) != 0 ||
        th_off + (int64_t)n * DH * 2 > a.pages_bytes)
      return;
    if (lane < 8) a.pages[page_off + lane] = lane == 0 ? (uint8_t)kDenseTier : (lane == 1 ? (uint8_t)n : 0);
    for (int i = lane; i < n * DH / 8; i += kWave) {
      const int tt = i / (DH / 8), c8 = i % (DH / 8);
      const int64_t rr = a.src_rows[(int64_t)p * kTile + tt];
      half8 hv;
      if (rr >= 0 && rr < a.num_src_rows) {
        if (a.k_is_fp32) {
          const float* src = static_cast<const float*>(a.k) + rr * DH + c8 * 8;
          for (int e = 0; e < 8; ++e) hv[e] = (_Float16)src[e];
        } else {
          hv = *reinterpret_cast<const half8*>(static_cast<const __half*>(a.k) + rr * DH + c8 * 8);
        }
      } else {
        for (int e = 0; e < 8; ++e) hv[e] = (_Float16)0.f;
      }
      *reinterpret_cast<half8*>(a.pages + th_off + ((int64_t)tt * DH + c8 * 8) * 2) = hv;
    }
    return;
  }
  if (tid < 1 || tid > 3) return;

  const int g = tier_g(tid), b = tier_b(tid);
  const int G = DH / g;
  const int nk = (G + 3) / 4;                   // groups per lane (2 for g=16, 1 for g=32 at DH=128)
  float rr_[2] = {0.f, 0.f};
  int best_[2] = {0, 0};
  for (int k = 0; k < nk; ++k) {
    const int gi = gs + 4 * k;
    if (gi < G) { rr_[k] = sm.r[16 * j + t][gi]; best_[k] = sm.code[16 * j + t][gi]; }
  }
  // radius scale per group: max over the page's tokens (lanes of one 16-row)
  float scale_[2];
  for (int k = 0; k < 2; ++k) {
    float m = tok_ok ? rr_[k] : 0.f;
    for (int o = 1; o < 16; o <<= 1) m = fmaxf(m, shfl_xor(m, o));
    scale_[k] = m;
  }
  uint8_t* st = sm.u.build.stage[j];
  const int nG = n * G;
  const int tb = (nG * b + 7) / 8;
  const int hdr = kHeaderBytes + 4 * G;
  const int size = hdr + tb + nG;
  if (lane < kHeaderBytes) st[lane] = lane == 0 ? (uint8_t)tid : (lane == 1 ? (uint8_t)n : 0);
  for (int k = 0; k < nk; ++k) {
    const int gi = gs + 4 * k;
    if (t == 0 && gi < G) *reinterpret_cast<float*>(st + kHeaderBytes + 4 * gi) = scale_[k];
  }
  // LSB-first bit stream (bitpacking.py:14-27): bit j of item i = (token t,
  // group gi), i = t*G + gi, at bit i*b + j.  The theta section's dwords (hdr
  // = 8 + 4G is a multiple of 4) are cleared, then every item ORs its b bits
  // into the one or two dwords they fall in.
  uint32_t* thw = reinterpret_cast<uint32_t*>(st + hdr);
  for (int w = lane; w < (tb + 3) / 4; w += kWave) thw[w] = 0u;
  wave_lds_sync();
  for (int k = 0; k < nk; ++k) {
    const int gi = gs + 4 * k;
    if (!tok_ok || gi >= G) continue;
    const uint32_t c = (uint32_t)best_[k];
    const int o = (t * G + gi) * b, w = o >> 5, sh = o & 31;
    __hip_atomic_fetch_or(thw + w, c << sh, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (sh + b > 32) __hip_atomic_fetch_or(thw + w + 1, c >> (32 - sh), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  // the radius codes, after the ORs (the first radius bytes can share the
  // last theta dword)
  wave_lds_sync();
  for (int k = 0; k < nk; ++k) {
    const int gi = gs + 4 * k;
    if (!tok_ok || gi >= G) continue;
    const int item = t * G + gi;
    const float safe = scale_[k] < 1e-8f ? 1e-8f : scale_[k];
    float qv = __fmul_rn(__fdiv_rn(rr_[k], safe), 127.0f);
    qv = __builtin_rintf(qv);
    qv = fminf(fmaxf(qv, -127.f), 127.f);
    st[hdr + tb + item] = (uint8_t)(int8_t)(int)qv;
    if (a.r_out) a.r_out[((int64_t)p * kTile + t) * (DH / 16) + gi] = rr_[k];
    if (a.code_out) a.code_out[((int64_t)p * kTile + t) * (DH / 16) + gi] = best_[k];
  }
  wave_lds_sync();
  if (page_off >= 0 && page_off + size <= a.pages_bytes) {
    // whole dwords where the page is 4-byte aligned, then its last bytes
    // (the next page may start right after it)
    const int nw = (page_off & 3) == 0 ? size >> 2 : 0;
    uint32_t* dw = reinterpret_cast<uint32_t*>(a.pages + page_off);
    for (int i = lane; i < nw; i += kWave) dw[i] = reinterpret_cast<const uint32_t*>(st)[i];
    for (int i = 4 * nw + lane; i < size; i += kWave) a.pages[page_off + i] = st[i];
  }
}

int launch_encode(const EncodeLaunch& L, hipStream_t stream) {
  EncodeArgs a;
  a.k = L.k; a.k_is_fp32 = L.k_is_fp32; a.v = reinterpret_cast<const __half*>(L.v);
  a.num_src_rows = L.num_src_rows; a.src_rows = L.src_rows; a.tier = L.tier; a.count = L.count;
  a.ptable = L.ptable; a.vslot = L.vslot; a.seq_head = L.seq_head; a.num_pages = L.num_pages;
  a.num_kv = L.num_kv; a.cb[0] = nullptr; a.cb[1] = L.cb1; a.cb[2] = L.cb2; a.cb[3] = L.cb3;
  a.pages = L.pages; a.pages_bytes = L.pages_bytes; a.v_pool = reinterpret_cast<__half*>(L.v_pool);
  a.num_vpages = L.num_vpages; a.r_out = L.r_out; a.code_out = L.code_out;
  a.order_n = L.order_n; a.codes_only = L.codes_only;
  const dim3 grid((L.num_pages + kEncPages - 1) / kEncPages), block(kEncWaves * 64);
  if (L.dh == 128) hipLaunchKernelGGL(encode_pages_kernel<128>, grid, block, 0, stream, a);
  else hipLaunchKernelGGL(encode_pages_kernel<64>, grid, block, 0, stream, a);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace sphkv
