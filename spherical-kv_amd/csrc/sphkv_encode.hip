// Fused encode + bitpack + page build + V placement (gfx950).
//
// One wave per page.  For a compressed page, lane l owns token t = l % 16 and
// the groups gi = l/16 + 4k.  Per (token, group) it reproduces the torch CPU
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

template <int DH>
__global__ __launch_bounds__(256) void encode_pages_kernel(EncodeArgs a) {
  __shared__ uint8_t stage[4][512];
  __shared__ int32_t codes_s[4][kTile * 8];
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int p = blockIdx.x * 4 + wave;
  if (p >= a.num_pages) return;

  const int tid = a.tier[p];
  const int n = min(max(a.count[p], 0), kTile);
  const int64_t page_off = a.ptable[3 * p];
  const int64_t th_off = a.ptable[3 * p + 1];
  const int64_t vs = a.vslot[p];
  const int t = lane & 15;
  const int gs = lane >> 4;
  const bool tok_ok = t < n;
  int64_t row = tok_ok ? a.src_rows[(int64_t)p * kTile + t] : -1;
  if (row >= a.num_src_rows) row = -1;

  // ---- V placement, dim-major: element (token k, dim d) of page vs at half
  //      d * 16 + k, so one dim's 16 tokens are 32 contiguous bytes ---------
  if (vs >= 0 && vs < a.num_vpages) {
    constexpr int DPL = DH / 64;  // dims per lane
    for (int dd = 0; dd < DPL; ++dd) {
      const int d = lane + 64 * dd;
      half8 h[2];
      for (int tok = 0; tok < kTile; ++tok) {
        int64_t rr = -1;
        if (tok < n) rr = a.src_rows[(int64_t)p * kTile + tok];
        _Float16 val = (_Float16)0.f;
        if (rr >= 0 && rr < a.num_src_rows) {
          __half hv = a.v[rr * DH + d];
          val = *reinterpret_cast<_Float16*>(&hv);
        }
        h[tok >> 3][tok & 7] = val;
      }
      half8* dst = reinterpret_cast<half8*>(a.v_pool + vs * DH * kTile + d * kTile);
      dst[0] = h[0];
      dst[1] = h[1];
    }
  }

  if (tid == kDenseTier) {
    // header: tier id, count, six zero bytes; payload fp16 [n, DH]
    if (lane < 8 && page_off + 8 <= a.pages_bytes)
      a.pages[page_off + lane] = lane == 0 ? (uint8_t)kDenseTier : (lane == 1 ? (uint8_t)n : 0);
    for (int i = lane; i < n * DH / 8; i += kWave) {
      const int tt = i / (DH / 8), c8 = i % (DH / 8);
      int64_t rr = a.src_rows[(int64_t)p * kTile + tt];
      half8 hv;
      if (rr >= 0 && rr < a.num_src_rows) {
        if (a.k_is_fp32) {
          const float* src = static_cast<const float*>(a.k) + rr * DH + c8 * 8;
          for (int j = 0; j < 8; ++j) hv[j] = (_Float16)src[j];
        } else {
          hv = *reinterpret_cast<const half8*>(static_cast<const __half*>(a.k) + rr * DH + c8 * 8);
        }
      } else {
        for (int j = 0; j < 8; ++j) hv[j] = (_Float16)0.f;
      }
      const int64_t dst = th_off + ((int64_t)tt * DH + c8 * 8) * 2;
      if (dst + 16 <= a.pages_bytes) *reinterpret_cast<half8*>(a.pages + dst) = hv;
    }
    return;
  }
  if (tid < 1 || tid > 3) return;

  const int g = tier_g(tid), b = tier_b(tid), C = tier_C(tid);
  const int G = DH / g;
  const int h = a.seq_head[p] % a.num_kv;
  const float* cbh = a.cb[tid] + (int64_t)h * G * C * g;
  const bool naive = n * g * C < 400;  // torch's own small-bmm loop
  uint8_t* st = stage[wave];
  int32_t* cs = codes_s[wave];

  float rr_[2];
  int best_[2];
  const int nk = (G + 3) / 4;  // groups per lane (2 for g=16, 1 for g=32 at DH=128)
  for (int k = 0; k < 2; ++k) {
    rr_[k] = 0.f;
    best_[k] = 0;
    if (k >= nk) break;
    const int gi = gs + 4 * k;
    if (gi >= G || row < 0) continue;
    float x[32];
    load_group<DH>(a, row, gi * g, g, x);
    const float r = torch_norm(x, g);
    const float den = __fadd_rn(r, 1e-8f);
    float dir[32];
    for (int i = 0; i < g; ++i) dir[i] = __fdiv_rn(x[i], den);
    const float* cbg = cbh + (int64_t)gi * C * g;
    float best_sim = 0.f;
    int best = 0;
    for (int c = 0; c < C; ++c) {
      const float4* row4 = reinterpret_cast<const float4*>(cbg + c * g);
      float s = 0.f;
      for (int i4 = 0; i4 < g / 4; ++i4) {
        const float4 w = row4[i4];
        if (naive) {
          s = __fadd_rn(s, __fmul_rn(dir[4 * i4], w.x));
          s = __fadd_rn(s, __fmul_rn(dir[4 * i4 + 1], w.y));
          s = __fadd_rn(s, __fmul_rn(dir[4 * i4 + 2], w.z));
          s = __fadd_rn(s, __fmul_rn(dir[4 * i4 + 3], w.w));
        } else {
          s = __builtin_fmaf(dir[4 * i4], w.x, s);
          s = __builtin_fmaf(dir[4 * i4 + 1], w.y, s);
          s = __builtin_fmaf(dir[4 * i4 + 2], w.z, s);
          s = __builtin_fmaf(dir[4 * i4 + 3], w.w, s);
        }
      }
      if (c == 0 || s > best_sim) { best_sim = s; best = c; }
    }
    rr_[k] = r;
    best_[k] = best;
  }

  // radius scale per group: max over the page's tokens (lanes of one 16-row)
  float scale_[2];
  for (int k = 0; k < 2; ++k) {
    float m = tok_ok ? rr_[k] : 0.f;
    for (int o = 1; o < 16; o <<= 1) m = fmaxf(m, shfl_xor(m, o));
    scale_[k] = m;
  }

  const int nG = n * G;
  const int tb = (nG * b + 7) / 8;
  const int hdr = kHeaderBytes + 4 * G;
  const int size = hdr + tb + nG;
  // header + scales
  if (lane < kHeaderBytes) st[lane] = lane == 0 ? (uint8_t)tid : (lane == 1 ? (uint8_t)n : 0);
  for (int k = 0; k < nk; ++k) {
    const int gi = gs + 4 * k;
    if (t == 0 && gi < G) *reinterpret_cast<float*>(st + kHeaderBytes + 4 * gi) = scale_[k];
  }
  // codes to LDS, int8 radius codes into the page image
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
  const dim3 grid((L.num_pages + 3) / 4), block(256);
  if (L.dh == 128) hipLaunchKernelGGL(encode_pages_kernel<128>, grid, block, 0, stream, a);
  else hipLaunchKernelGGL(encode_pages_kernel<64>, grid, block, 0, stream, a);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace sphkv
