// Fused encode + bitpack + page build + V placement (gfx950).
//
// One workgroup per four consecutive pages, one lane per token and one wave
// per group; the codebook of a (tier, kv head) is read as scalar operands.
// Per (token, group) it reproduces the torch CPU
// operation order of _encode_keys_with_codebooks
// (spherical_kv_pipeline.py:1136-1144) so that radii and codes are bit-exact:
//   r   = sqrtf(sum over 8 lanes of fmaf(x, x, .) chains, lanes summed in order)
//   dir = x / (r + 1e-8f)                     (IEEE division)
//   sim = fmaf chain over i (torch's naive small-bmm path, N*g*C < 400:
//         separate multiply and add)
//   code = first index of the maximum similarity
// then builds the page of pagebuilder.py:8-33 in LDS (header, fp32 scales,
// LSB-first theta codes, int8 radius codes) and stores it.  This file is
// compiled with -ffp-contract=off so no multiply/add pair is fused.
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

// torch CPU fp32 L2 norm of a contiguous group (ATen vectorised last-dim
// reduction, 8 lanes, fused multiply-add accumulation, lanes summed in order).
__device__ __forceinline__ float torch_norm(const float* x, int g) {
  float acc[8];
  for (int l = 0; l < 8; ++l) acc[l] = 0.f;
  for (int d = 0; d < g; d += 8)
    for (int l = 0; l < 8; ++l) acc[l] = __builtin_fmaf(x[d + l], x[d + l], acc[l]);
  float b = acc[0];
  for (int l = 1; l < 8; ++l) b = __fadd_rn(b, acc[l]);
  return __builtin_sqrtf(b);  // correctly rounded expansion (v_sqrt_f32 alone is not)
}

typedef const float __attribute__((address_space(4)))* cb_ptr;   // read through the scalar cache

constexpr int kEncWaves = 8;       // waves per workgroup: one per group in the argmax phase
constexpr int kEncPages = 4;       // pages per workgroup: one lane per token of four pages
constexpr int kEncMaxG = 8;        // groups per token (dh / g)

template <int DH>
struct EncodeLds {
  float r[kEncPages * kTile][kEncMaxG];        // radius of (token, group)
  int32_t code[kEncPages * kTile][kEncMaxG];   // code of (token, group)
  uint8_t stage[kEncPages][512];               // page images
  int32_t cs[kEncPages][kTile * kEncMaxG];     // a page's codes, token-major
  _Float16 vt[kEncPages][DH * kTile];          // V pages, dim-major
};

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
#pragma unroll
  for (int i = 0; i < GG; ++i) dir[i] = __fdiv_rn(x[i], den);
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
    const int tid_l = p_ok ? a.tier[p] : 0;
    const int n_l = p_ok ? min(max(a.count[p], 0), kTile) : 0;
    const int head_l = p_ok ? a.seq_head[p] % a.num_kv : 0;
    int64_t row = (p_ok && t < n_l) ? a.src_rows[(int64_t)p * kTile + t] : -1;
    if (row >= a.num_src_rows) row = -1;
    const bool comp_l = tid_l >= 1 && tid_l <= 3 && wave < DH / tier_g(tid_l);
    const int gi = wave;
    uint64_t todo = __builtin_amdgcn_ballot_w64(comp_l);
    while (todo) {
      const int lead = (int)__builtin_ctzll(todo);                 // first lane not yet encoded
      const int tid = uniform(__builtin_amdgcn_readlane(tid_l, lead));
      const int h = uniform(__builtin_amdgcn_readlane(head_l, lead));
      const bool mine = comp_l && tid_l == tid && head_l == h;
      todo &= ~__builtin_amdgcn_ballot_w64(mine);
      const int g = uniform(tier_g(tid)), C = uniform(tier_C(tid)), G = DH / g;
      const uint64_t cba = (uint64_t)(a.cb[tid] + ((int64_t)h * G + gi) * C * g);
      const cb_ptr cbg = (cb_ptr)(((uint64_t)(uint32_t)uniform((int)(cba >> 32)) << 32) |
                                  (uint32_t)uniform((int)(uint32_t)cba));
      if (mine) {
        const bool naive = n_l * g * C < 400;                     // torch's own small-bmm loop
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
    _Float16* vt = sm.vt[j];
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
    // header: tier id, count, six zero bytes; payload fp16 [n, DH]
    if (lane < 8 && page_off + 8 <= a.pages_bytes)
      a.pages[page_off + lane] = lane == 0 ? (uint8_t)kDenseTier : (lane == 1 ? (uint8_t)n : 0);
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
      const int64_t dst = th_off + ((int64_t)tt * DH + c8 * 8) * 2;
      if (dst + 16 <= a.pages_bytes) *reinterpret_cast<half8*>(a.pages + dst) = hv;
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
  uint8_t* st = sm.stage[j];
  int32_t* cs = sm.cs[j];
  const int nG = n * G;
  const int tb = (nG * b + 7) / 8;
  const int hdr = kHeaderBytes + 4 * G;
  const int size = hdr + tb + nG;
  if (lane < kHeaderBytes) st[lane] = lane == 0 ? (uint8_t)tid : (lane == 1 ? (uint8_t)n : 0);
  for (int k = 0; k < nk; ++k) {
    const int gi = gs + 4 * k;
    if (t == 0 && gi < G) *reinterpret_cast<float*>(st + kHeaderBytes + 4 * gi) = scale_[k];
  }
  for (int k = 0; k < nk; ++k) {
    const int gi = gs + 4 * k;
    if (!tok_ok || gi >= G) continue;
    const int item = t * G + gi;
    cs[item] = best_[k];
    const float safe = scale_[k] < 1e-8f ? 1e-8f : scale_[k];
    float qv = __fmul_rn(__fdiv_rn(rr_[k], safe), 127.0f);
    qv = __builtin_rintf(qv);
    qv = fminf(fmaxf(qv, -127.f), 127.f);
    st[hdr + tb + item] = (uint8_t)(int8_t)(int)qv;
    if (a.r_out) a.r_out[((int64_t)p * kTile + t) * (DH / 16) + gi] = rr_[k];
    if (a.code_out) a.code_out[((int64_t)p * kTile + t) * (DH / 16) + gi] = best_[k];
  }
  wave_lds_sync();
  // LSB-first bit stream (bitpacking.py:14-27): bit j of item i at bit i*b + j
  for (int byte = lane; byte < tb; byte += kWave) {
    uint32_t v = 0;
    for (int bit = 0; bit < 8; ++bit) {
      const int gb = byte * 8 + bit;
      const int item = gb / b;
      if (item < nG) v |= (uint32_t)((cs[item] >> (gb - item * b)) & 1) << bit;
    }
    st[hdr + byte] = (uint8_t)v;
  }
  wave_lds_sync();
  if (page_off >= 0 && page_off + size <= a.pages_bytes)
    for (int i = lane; i < size; i += kWave) a.pages[page_off + i] = st[i];
}

int launch_encode(const EncodeLaunch& L, hipStream_t stream) {
  EncodeArgs a;
  a.k = L.k; a.k_is_fp32 = L.k_is_fp32; a.v = reinterpret_cast<const __half*>(L.v);
  a.num_src_rows = L.num_src_rows; a.src_rows = L.src_rows; a.tier = L.tier; a.count = L.count;
  a.ptable = L.ptable; a.vslot = L.vslot; a.seq_head = L.seq_head; a.num_pages = L.num_pages;
  a.num_kv = L.num_kv; a.cb[0] = nullptr; a.cb[1] = L.cb1; a.cb[2] = L.cb2; a.cb[3] = L.cb3;
  a.pages = L.pages; a.pages_bytes = L.pages_bytes; a.v_pool = reinterpret_cast<__half*>(L.v_pool);
  a.num_vpages = L.num_vpages; a.r_out = L.r_out; a.code_out = L.code_out;
  const dim3 grid((L.num_pages + kEncPages - 1) / kEncPages), block(kEncWaves * 64);
  if (L.dh == 128) hipLaunchKernelGGL(encode_pages_kernel<128>, grid, block, 0, stream, a);
  else hipLaunchKernelGGL(encode_pages_kernel<64>, grid, block, 0, stream, a);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace sphkv
