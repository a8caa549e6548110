// Mode-A (LayerPool) kernels: the unpacked-pool decode path of the reference's
// fused_decode.py / sphkv_lut.py / new_fused_decode.py, built for gfx950.
//
// Pools (sphkv_lut.py:71-80): theta_codes / radius_codes uint8
// [n_pages, page_size, G_max], r_scales fp32 [n_pages, G_max], v_pool fp16
// [n_pages, page_size, dh] (token-major); per kv head a block table (logical
// page -> pool page, -1 = none) and a bits table (logical page -> tier index);
// cb_flat fp32 [num_kv, num_tiers, G_max, cb_max, g_max] (zero padded).
// Radii are uint8 with r_hat = r_scale * code / 255 (decode_kernel.cu:183).
// There is no RoPE in Mode A: q and the keys behind the codes are post-RoPE,
// so a per-query table LUT[g][c] = <q_g, centroid_g[c]> is exact and a key's
// logit is sum_g r_hat_g * LUT[g][code_g].
//
// Kernels:
//   append_kernel      sphkv_encode_append (decode_kernel.cu:10-84): one
//                      workgroup per kv head; every (group, code) similarity in
//                      parallel, then per group the first-max argmax and the
//                      running-max radius scale.  Bit-exact with the reference
//                      arithmetic as nvcc compiles it (a*b + c contracted to
//                      fmaf, IEEE sqrt and divide, roundf).
//   modea_split_kernel Mode-A decode (decode_kernel.cu:108-218): one
//                      workgroup per (kv head, range of logical pages); the
//                      kv head's q heads share every page read; per page and q
//                      head it writes the reference's (m, l) into
//                      partial_scratch[..., 0:2] (read by the omega-EMA update,
//                      spherical_kv_pipeline.py:1690-1701); per range one
//                      online-softmax partial (m, l, acc[dh]).
//   modea_fast_kernel  the same for G_max 4 or 8 with vector loads and a
//                      two-deep tile prefetch ring (the common case).
//   modea_merge_kernel log-sum-exp merge of the ranges (decode_kernel.cu:221-246):
//                      out = acc / (l + 1e-8).
//   qlut_kernel        the per-query LUT [num_q, num_tiers, G_max, cb_max].
//   lut_logits_kernel  logits from a given LUT (new_fused_decode.py:22-43).
#include "sphkv_common.h"
#include "sphkv_internal.h"

namespace sphkv {

// ---------------------------------------------------------------------------
// encode + append
// ---------------------------------------------------------------------------
constexpr int kAppendThreads = 256;
constexpr int kAppendMaxDh = 256;
constexpr int kAppendMaxSims = 4096;     // G * C

__global__ __launch_bounds__(kAppendThreads) void append_kernel(AppendLaunch a) {
  const int h = blockIdx.x;
  const int tid = threadIdx.x;
  __shared__ __attribute__((aligned(16))) float s_k[kAppendMaxDh];
  __shared__ float s_norm[kAppendMaxDh], s_inv[kAppendMaxDh], s_ratio[kAppendMaxDh];
  __shared__ int s_code[kAppendMaxDh], s_resc[kAppendMaxDh];
  __shared__ float s_sim[kAppendMaxSims];
  const int64_t pid = a.pids[h];
  // k and v do not depend on the page: their loads share pid's round trip
  const float kx = tid < a.dh ? a.k_post[(int64_t)h * a.dh + tid] : 0.f;
  const float vx = tid < a.dh ? a.v_new[(int64_t)h * a.dh + tid] : 0.f;
  if (pid < 0 || pid >= a.num_pages) return;        // no such pool page: nothing is written
  const int64_t row = pid * a.page_size + a.slot;   // (page, slot)
  const float prev = tid < a.G && !a.is_new_page ? a.r_scales[pid * a.G_max + tid] : 0.f;   // running scale
  if (tid < a.dh) {
    s_k[tid] = kx;
    a.v_pool[row * a.dh + tid] = (_Float16)vx;      // round to nearest even
  }
  __syncthreads();
  // decode_kernel.cu:38-42: norm = sqrt(sum k^2 + 1e-16), inv = 1 / (norm + 1e-8)
  if (tid < a.G) {
    const float* kg = s_k + tid * a.g;
    float nsq = 0.f;
    for (int d = 0; d < a.g; ++d) nsq = __builtin_fmaf(kg[d], kg[d], nsq);
    const float nrm = __builtin_sqrtf(nsq + 1e-16f);
    s_norm[tid] = nrm;
    s_inv[tid] = 1.0f / (nrm + 1e-8f);
  }
  __syncthreads();
  // decode_kernel.cu:45-55: sim_c = sum_d (k_d * inv) * cb[c][d], in d order
  const int nsim = a.G * a.C;
  for (int i = tid; i < nsim; i += kAppendThreads) {
    const int grp = i / a.C, c = i - grp * a.C;
    const float* kg = s_k + grp * a.g;
    const float inv = s_inv[grp];
    const float* cb = a.decode_cb + (((int64_t)h * a.G + grp) * a.C + c) * a.g;
    float sim = 0.f;
    if (a.g == 16 && ((uintptr_t)cb & 15) == 0) {  // the row as four 16-byte loads, same d order
      floatx4 cv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) cv[j] = reinterpret_cast<const floatx4*>(cb)[j];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) sim = __builtin_fmaf(kg[4 * j + e] * inv, cv[j][e], sim);
    } else {
      for (int d = 0; d < a.g; ++d) sim = __builtin_fmaf(kg[d] * inv, cb[d], sim);
    }
    s_sim[i] = sim;
  }
  __syncthreads();
  // argmax per group, one wave per group: each lane keeps the first maximum of
  // its codes (c = lane, lane + 64, ...), then the lanes agree on the largest
  // value and, among equal values, the smallest code -- the first maximum of
  // the ascending scan (decode_kernel.cu:47-55); NaN and values <= -1e30 never win
  const int lane = tid & 63;
  for (int grp = tid >> 6; grp < a.G; grp += kAppendThreads / 64) {
    float best = -1e30f;
    int code = -1;
    for (int c = lane; c < a.C; c += 64) {
      const float v = s_sim[grp * a.C + c];
      if (v > best) { best = v; code = c; }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const float ob = __shfl_xor(best, o, 64);
      const int oc = __shfl_xor(code, o, 64);
      if (ob > best || (ob == best && (unsigned)oc < (unsigned)code)) { best = ob; code = oc; }
    }
    if (lane == 0) s_code[grp] = code < 0 ? 0 : code;
  }
  __syncthreads();
  // decode_kernel.cu:59-82: per-page running-max radius scale
  if (tid < a.G) {
    const int grp = tid;
    a.theta_codes[row * a.G_max + grp] = (uint8_t)s_code[grp];
    const float nrm = s_norm[grp];
    float* rs = a.r_scales + pid * a.G_max + grp;
    float r_scale;
    int resc = 0;
    if (a.is_new_page) {
      *rs = nrm;
      r_scale = nrm;
    } else if (nrm > prev) {
      s_ratio[grp] = prev / (nrm + 1e-8f);
      resc = 1;
      *rs = nrm;
      r_scale = nrm;
    } else {
      r_scale = prev;
    }
    s_resc[grp] = resc;
    float rq = roundf(nrm / (r_scale + 1e-8f) * 255.0f);
    rq = fminf(fmaxf(rq, 0.f), 255.f);
    a.radius_codes[row * a.G_max + grp] = (uint8_t)rq;
  }
  __syncthreads();
  // a rescaled group's earlier radius codes, one thread per (token, group)
  for (int i = tid; i < a.slot * a.G; i += kAppendThreads) {
    const int t = i / a.G, grp = i - t * a.G;
    if (!s_resc[grp]) continue;
    uint8_t* rc = a.radius_codes + (pid * a.page_size + t) * a.G_max + grp;
    float x = (float)(*rc) * s_ratio[grp];
    x = fminf(fmaxf(roundf(x), 0.f), 255.f);
    *rc = (uint8_t)x;
  }
}

int launch_append(const AppendLaunch& L, hipStream_t stream) {
  if (L.num_kv > 0)
    hipLaunchKernelGGL(append_kernel, dim3(L.num_kv), dim3(kAppendThreads), 0, stream, L);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// ---------------------------------------------------------------------------
// per-query LUT: lut[hq][tier][g][c] = sum_{d < g_t} q[hq][g g_t + d] cb[hkv][tier][g][c][d]
// for g < G_t (tier's group count), else 0.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float lut_entry(const ModeALaunch& a, int hq, int tier, int g, int c,
                                           const int* tG, const int* tg) {
  const int Gt = tG[tier], gt = tg[tier];
  if (g >= Gt || c >= a.cb_max) return 0.f;
  const int hkv = hq / a.kv_groups;
  const float* qg = a.q + (int64_t)hq * a.dh + g * gt;
  const float* cb = a.cb_flat + ((((int64_t)hkv * a.num_tiers + tier) * a.G_max + g) * a.cb_max + c) * a.g_max;
  float dot = 0.f;
  if (gt == 16 && (((uintptr_t)qg | (uintptr_t)cb) & 15) == 0) {   // both rows as four 16-byte loads
    float4 qv[4], cv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      qv[j] = reinterpret_cast<const float4*>(qg)[j];
      cv[j] = reinterpret_cast<const float4*>(cb)[j];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {                   // the same d order as the loop below
      dot = __builtin_fmaf(qv[j].x, cv[j].x, dot);
      dot = __builtin_fmaf(qv[j].y, cv[j].y, dot);
      dot = __builtin_fmaf(qv[j].z, cv[j].z, dot);
      dot = __builtin_fmaf(qv[j].w, cv[j].w, dot);
    }
    return dot;
  }
  for (int d = 0; d < gt; ++d) dot = __builtin_fmaf(qg[d], cb[d], dot);   // decode_kernel.cu:187-189 order
  return dot;
}

// Tier geometry checked on the device: a tier index outside [0, num_tiers) or
// a geometry that does not fit the tables makes the page count as absent.
__device__ __forceinline__ bool tier_ok(const ModeALaunch& a, int tier, const int* tG, const int* tg) {
  return tier >= 0 && tier < a.num_tiers && tG[tier] >= 1 && tG[tier] <= a.G_max && tg[tier] >= 1 &&
         tg[tier] <= a.g_max && tG[tier] * tg[tier] <= a.dh;
}

__global__ __launch_bounds__(256) void qlut_kernel(ModeALaunch a, float* lut) {
  __shared__ int tG[kModeAMaxTiers], tg[kModeAMaxTiers];
  if (threadIdx.x < a.num_tiers) { tG[threadIdx.x] = a.tier_G[threadIdx.x]; tg[threadIdx.x] = a.tier_g[threadIdx.x]; }
  __syncthreads();
  const int64_t per_q = (int64_t)a.num_tiers * a.G_max * a.cb_max;
  const int64_t total = (int64_t)a.num_q * per_q;
  if (total < ((int64_t)1 << 31)) {                 // 32-bit index arithmetic (the usual table size)
    const int pq = (int)per_q, per_t = a.G_max * a.cb_max;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < (int)total; i += gridDim.x * blockDim.x) {
      const int hq = i / pq;
      int r = i - hq * pq;
      const int tier = r / per_t;
      r -= tier * per_t;
      const int g = r / a.cb_max, c = r - g * a.cb_max;
      lut[i] = tier_ok(a, tier, tG, tg) ? lut_entry(a, hq, tier, g, c, tG, tg) : 0.f;
    }
    return;
  }
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int hq = (int)(i / per_q);
    int64_t r = i - hq * per_q;
    const int tier = (int)(r / ((int64_t)a.G_max * a.cb_max));
    r -= (int64_t)tier * a.G_max * a.cb_max;
    const int g = (int)(r / a.cb_max), c = (int)(r - (int64_t)g * a.cb_max);
    lut[i] = tier_ok(a, tier, tG, tg) ? lut_entry(a, hq, tier, g, c, tG, tg) : 0.f;
  }
}

// ---------------------------------------------------------------------------
// Mode-A decode, split over ranges of logical pages.
// Workgroup = 4 waves; lane l = (token t16 = l % 16, head row hr = l / 16) when
// scoring a 16-token tile; q heads hkv*kv_groups + hr + 4 hp, hp < NHP.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float mdpp(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float rmax16(float x) {
  x = fmaxf(x, mdpp<0xB1>(x));
  x = fmaxf(x, mdpp<0x4E>(x));
  x = fmaxf(x, mdpp<0x141>(x));
  return fmaxf(x, mdpp<0x140>(x));
}
__device__ __forceinline__ float rsum16(float x) {
  x = x + mdpp<0xB1>(x);
  x = x + mdpp<0x4E>(x);
  x = x + mdpp<0x141>(x);
  return x + mdpp<0x140>(x);
}

// exp(x) as the reference's __expf computes it: 2^(x * log2 e) on the
// hardware exp2.
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

// First logical page of range s of a kv head's block table (ranges split the
// table as evenly as integers allow; every range holds >= 2 pages when
// nsplit > 1, so a range's partial fits in the free part of two page entries).
__device__ __forceinline__ int range_begin(const ModeALaunch& a, int s) {
  return (int)((int64_t)s * a.max_blocks / a.nsplit);
}

template <int DH, int NHP>
__global__ __launch_bounds__(256) void modea_split_kernel(ModeALaunch a) {
  constexpr int NH = 4 * NHP;              // q-head rows (padded)
  constexpr int DPL = DH / 16;             // dims per lane in P V (16 lanes cover a token row)
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int wave = uniform(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int hkv = blockIdx.x / a.nsplit, s = blockIdx.x % a.nsplit;
  const int pb = range_begin(a, s), pe = range_begin(a, s + 1);
  const int P = a.page_size, NT = P / 16;
  const int lut_n = NH * a.num_tiers * a.G_max * a.cb_max;
  float* lut = reinterpret_cast<float*>(smem);                           // [NH][tier][G_max][cb_max]
  float* pw = lut + lut_n;                                                // per wave: p [P][NH]
  float* red = pw + 4 * P * NH;                                           // merge: [4][NH][DH + 2]
  __shared__ int tG[kModeAMaxTiers], tg[kModeAMaxTiers];
  if (threadIdx.x < a.num_tiers) { tG[threadIdx.x] = a.tier_G[threadIdx.x]; tg[threadIdx.x] = a.tier_g[threadIdx.x]; }
  __syncthreads();
  for (int i = threadIdx.x; i < lut_n; i += 256) {
    const int hr = i / (a.num_tiers * a.G_max * a.cb_max);
    int r = i - hr * (a.num_tiers * a.G_max * a.cb_max);
    const int tier = r / (a.G_max * a.cb_max);
    r -= tier * a.G_max * a.cb_max;
    const int g = r / a.cb_max, c = r - g * a.cb_max;
    lut[i] = (hr < a.kv_groups && tier_ok(a, tier, tG, tg))
                 ? lut_entry(a, hkv * a.kv_groups + hr, tier, g, c, tG, tg) : 0.f;
  }
  __syncthreads();

  const int t16 = lane & 15, hr = lane >> 4;
  const int dg = lane & 15, tq = lane >> 4;     // P V: dims [DPL dg, DPL dg + DPL) of token 4 i + tq
  float* pwv = pw + wave * P * NH;
  float M[NH], Lr[NH];                          // running max / sum per q-head row (wave-uniform)
  float acc[NH][DPL];
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    M[h] = -INFINITY;
    Lr[h] = 0.f;
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc[h][j] = 0.f;
  }
  for (int p = pb + wave; p < pe; p += 4) {
    const int phys = a.block_table[(int64_t)hkv * a.max_blocks + p];
    const int tier = a.bits_table[(int64_t)hkv * a.max_blocks + p];
    const bool live = phys >= 0 && phys < a.num_pages && tier_ok(a, tier, tG, tg);
    float mp[NHP], lp[NHP];
    if (!live) {                                // decode_kernel.cu:139-144
#pragma unroll
      for (int hp = 0; hp < NHP; ++hp) { mp[hp] = -INFINITY; lp[hp] = 0.f; }
    } else {
      const int Gt = tG[tier];
      // logits of the page: lane (t16, hr) keeps tile k's logit for each head pass
      float lg[8][NHP];
      const float* rsc = a.r_scales + (int64_t)phys * a.G_max;
      const float* lt = lut + ((int64_t)hr * a.num_tiers + tier) * a.G_max * a.cb_max;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        if (k >= NT) break;
        const int t = 16 * k + t16;
        const uint8_t* th = a.theta_codes + ((int64_t)phys * P + t) * a.G_max;
        const uint8_t* rd = a.radius_codes + ((int64_t)phys * P + t) * a.G_max;
        float sum[NHP];
#pragma unroll
        for (int hp = 0; hp < NHP; ++hp) sum[hp] = 0.f;
        for (int g = 0; g < Gt; ++g) {
          const int code = th[g];
          const float rh = rsc[g] * (float)rd[g] / 255.0f;          // decode_kernel.cu:183
#pragma unroll
          for (int hp = 0; hp < NHP; ++hp) {
            const float v = code < a.cb_max ? lt[(int64_t)hp * 4 * a.num_tiers * a.G_max * a.cb_max + g * a.cb_max + code] : 0.f;
            sum[hp] = __builtin_fmaf(rh, v, sum[hp]);
          }
        }
#pragma unroll
        for (int hp = 0; hp < NHP; ++hp) lg[k][hp] = (sum[hp] == 0.f) ? -1e9f : sum[hp] * a.sm_scale;   // :183
      }
      // page softmax per head row (a head row = one 16-lane DPP row)
#pragma unroll
      for (int hp = 0; hp < NHP; ++hp) {
        float mx = lg[0][hp];
#pragma unroll
        for (int k = 1; k < 8; ++k)
          if (k < NT) mx = fmaxf(mx, lg[k][hp]);
        mx = rmax16(mx);
        float ls = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          if (k >= NT) break;
          const float e = fast_exp(lg[k][hp] - mx);
          ls += e;
          pwv[(16 * k + t16) * NH + hr + 4 * hp] = e;
        }
        mp[hp] = mx;
        lp[hp] = rsum16(ls);
      }
    }
    // the reference's per-page (m, l) of each q head
#pragma unroll
    for (int hp = 0; hp < NHP; ++hp)
      if (t16 == 0 && hr + 4 * hp < a.kv_groups) {
        float* pt = a.partial + ((int64_t)(hkv * a.kv_groups + hr + 4 * hp) * a.max_blocks + p) * (a.dh + 2);
        pt[0] = mp[hp];
        pt[1] = lp[hp];
      }
    if (!live) continue;
    wave_lds_sync();
    // running state update per head row: values of row hr live in lanes 16 hr ..
    float f_old[NH], f_new[NH];
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      const float mph = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mp[h / 4]), 16 * (h % 4)));
      const float lph = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lp[h / 4]), 16 * (h % 4)));
      const float mn = fmaxf(M[h], mph);
      f_old[h] = (M[h] == -INFINITY) ? 0.f : fast_exp(M[h] - mn);
      f_new[h] = fast_exp(mph - mn);
      Lr[h] = Lr[h] * f_old[h] + lph * f_new[h];
      M[h] = mn;
    }
    float pv[NH][DPL];
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
      for (int j = 0; j < DPL; ++j) pv[h][j] = 0.f;
    const _Float16* vp = a.v_pool + (int64_t)phys * P * DH + DPL * dg;
    for (int t = tq; t < P; t += 4) {
      float v[DPL];
      if constexpr (DPL == 8) {
        const half8 w = *reinterpret_cast<const half8*>(vp + (int64_t)t * DH);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = (float)w[j];
      } else {
        const half4 w = *reinterpret_cast<const half4*>(vp + (int64_t)t * DH);
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = (float)w[j];
      }
      const float* pr = pwv + t * NH;
#pragma unroll
      for (int h = 0; h < NH; ++h) {
        const float ph = pr[h];
#pragma unroll
        for (int j = 0; j < DPL; ++j) pv[h][j] = __builtin_fmaf(ph, v[j], pv[h][j]);
      }
    }
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
      for (int j = 0; j < DPL; ++j) acc[h][j] = acc[h][j] * f_old[h] + pv[h][j] * f_new[h];
    wave_lds_sync();
  }
  // combine the four token rows of each wave (lanes dg, dg+16, dg+32, dg+48)
#pragma unroll
  for (int h = 0; h < NH; ++h)
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      float x = acc[h][j];
      x += __shfl_xor(x, 16, 64);
      x += __shfl_xor(x, 32, 64);
      acc[h][j] = x;
    }
  // merge the four waves in LDS, then write this range's partial
  float* rw = red + (int64_t)wave * NH * (DH + 2);
  if (tq == 0)
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
      for (int j = 0; j < DPL; ++j) rw[h * (DH + 2) + 2 + DPL * dg + j] = acc[h][j];
  if (lane == 0)
#pragma unroll
    for (int h = 0; h < NH; ++h) { rw[h * (DH + 2)] = M[h]; rw[h * (DH + 2) + 1] = Lr[h]; }
  __syncthreads();
  for (int i = threadIdx.x; i < a.kv_groups * DH; i += 256) {
    const int h = i / DH, d = i - h * DH;
    float Mx = -INFINITY;
    for (int w = 0; w < 4; ++w) Mx = fmaxf(Mx, red[(w * NH + h) * (DH + 2)]);
    float Ls = 0.f, A = 0.f;
    if (Mx != -INFINITY)
      for (int w = 0; w < 4; ++w) {
        const float mw = red[(w * NH + h) * (DH + 2)];
        if (mw == -INFINITY) continue;
        const float f = fast_exp(mw - Mx);
        Ls += f * red[(w * NH + h) * (DH + 2) + 1];
        A += f * red[(w * NH + h) * (DH + 2) + 2 + d];
      }
    const int hq = hkv * a.kv_groups + h;
    if (a.nsplit == 1) {
      a.out[(int64_t)hq * DH + d] = A / (Ls + 1e-8f);                    // decode_kernel.cu:244-245
    } else {
      // range partial in the free part of partial_scratch: acc in page entry
      // pb, (m, l) in page entry pb + 1 (every range holds >= 2 pages)
      float* e0 = a.partial + ((int64_t)hq * a.max_blocks + pb) * (a.dh + 2);
      e0[2 + d] = A;
      if (d == 0) {
        float* e1 = e0 + (a.dh + 2);
        e1[2] = Mx;
        e1[3] = Ls;
      }
    }
  }
}

// Log-sum-exp merge of the ranges' partials (decode_kernel.cu:221-246):
// workgroup = (q head, 64-dim chunk); wave w folds ranges w, w + 8, ... into a
// running (m, l, acc) with four ranges' loads in flight at a time, then wave 0
// folds the eight waves and writes out = acc / (l + 1e-8).
constexpr int kMergeWaves = 8;
__global__ __launch_bounds__(64 * kMergeWaves) void modea_merge_kernel(ModeALaunch a) {
  const int nch = (a.dh + 63) / 64;
  const int hq = blockIdx.x / nch, ch = blockIdx.x - hq * nch;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int d = ch * 64 + lane;
  const bool dv = d < a.dh;
  const int64_t E = a.dh + 2;
  const float* base = a.partial + (int64_t)hq * a.max_blocks * E;
  float m = -INFINITY, L = 0.f, A = 0.f;
  for (int s0 = wave; s0 < a.nsplit; s0 += 4 * kMergeWaves) {
    float ms[4], ls[4], as[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int s = s0 + u * kMergeWaves;
      const bool ok = s < a.nsplit;
      const float* e0 = base + (int64_t)(ok ? range_begin(a, s) : 0) * E;
      ms[u] = ok ? e0[E + 2] : -INFINITY;
      ls[u] = ok ? e0[E + 3] : 0.f;
      as[u] = ok && dv ? e0[2 + d] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (ms[u] == -INFINITY) continue;
      const float mn = fmaxf(m, ms[u]);
      const float fo = m == -INFINITY ? 0.f : fast_exp(m - mn), fn = fast_exp(ms[u] - mn);
      L = L * fo + ls[u] * fn;
      A = A * fo + as[u] * fn;
      m = mn;
    }
  }
  __shared__ float sm[kMergeWaves][66];
  sm[wave][2 + lane] = A;
  if (lane == 0) { sm[wave][0] = m; sm[wave][1] = L; }
  __syncthreads();
  if (wave == 0 && dv) {
    float Mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kMergeWaves; ++w) Mx = fmaxf(Mx, sm[w][0]);
    float Ls = 0.f, As = 0.f;
    if (Mx != -INFINITY)
#pragma unroll
      for (int w = 0; w < kMergeWaves; ++w) {
        if (sm[w][0] == -INFINITY) continue;
        const float f = fast_exp(sm[w][0] - Mx);
        Ls += f * sm[w][1];
        As += f * sm[w][2 + lane];
      }
    a.out[(int64_t)hq * a.dh + d] = As / (Ls + 1e-8f);
  }
}

// ---------------------------------------------------------------------------
// Mode-A decode, vector-load kernel (G_max 4 or 8: a token's code row is one
// 4- or 8-byte load).  Workgroup = kFastWaves waves on one kv head and one
// range of logical pages; the range's 16-token tiles are split evenly over
// the waves (a page of P tokens is P / 16 tiles, so pages of 16 and of 128
// spread the same way).
//
// Per wave, tiles stream through a two-deep register ring: while tile k is
// scored and accumulated, the loads of tile k + 2 are in flight.  Every load
// is a buffer load against a resource covering exactly the tile's page (0
// bytes for an absent page or a tile past the end), so each ring step issues
// the same loads whatever the page holds and the compiler's vmcnt waits stay
// exact.  The first two tiles are issued before the workgroup builds its
// lookup table, so their HBM latency overlaps that work.
//
// Lanes score a tile as (token t16 = lane % 16, head row hr = lane / 16) and
// accumulate P V as (dims [DPL dg, DPL dg + DPL), dg = lane % 16; tokens
// tq + 4 j, tq = lane / 16).  The table holds <q_g, c> * sm_scale * log2(e) /
// 255, so a logit in log2 units is sum_g r_scale_g * rcode_g * T[g][code_g]
// and softmax runs on the hardware exp2.  Each tile's (max, sum) per q head
// goes to LDS; after the loop the tiles of each page are combined into the
// reference's per-page (m, l) (decode_kernel.cu:198-215, in natural units).
// ---------------------------------------------------------------------------
constexpr int kFastWaves = 16;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegLogit2 = -1e9f * kLog2e;     // the reference's -1e9 logit (decode_kernel.cu:194), log2 units

// LDS carve-up of the vector-load kernel (floats unless noted).
struct FastLds {
  int lut, q, p, ts, tbl, red, total;             // offsets in 4-byte words; total bytes
};
__host__ __device__ inline FastLds fast_lds(int dh, int nhp, int num_tiers, int G_max, int cb_max, int max_pages,
                                            int page_size) {
  const int NH = 4 * nhp;
  FastLds f;
  f.lut = 0;
  f.q = f.lut + NH * num_tiers * G_max * (cb_max + 1);
  f.p = f.q + NH * dh;
  f.ts = f.p + kFastWaves * 128;                 // per wave a [16][16] fp16 MFMA operand
  f.tbl = f.ts + 2 * NH * max_pages * (page_size / 16);
  f.red = f.tbl + 2 * max_pages;
  f.total = 4 * (f.red + kFastWaves * NH * (dh + 2));
  return f;
}

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int GV, int DPL>
struct FastTile {
  int live, tier, slot;                 // wave-uniform: page present, tier, workgroup-local tile index
  uint32_t th[GV / 4], rd[GV / 4];      // this lane's token: theta and radius code bytes
  uint32_t rs;                          // lane g < G_tier: r_scales[g]
  uint32_t v[4][DPL / 2];               // fp16 V: 4 tokens x DPL dims
};

template <int DH, int NHP, int GV>
__global__ __launch_bounds__(64 * kFastWaves) void modea_fast_kernel(ModeALaunch a) {
  constexpr int NH = 4 * NHP;
  constexpr int DPL = DH / 16;
  constexpr int W = kFastWaves;
  constexpr int NTH = 64 * W;
  extern __shared__ __attribute__((aligned(16))) float fsm[];
  __shared__ int tG[kModeAMaxTiers], tg[kModeAMaxTiers];
  const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
  const int hkv = blockIdx.x / a.nsplit, s = blockIdx.x % a.nsplit;
  const int rb = range_begin(a, s), npg = range_begin(a, s + 1) - rb;
  const int P = a.page_size, TPP = P / 16;
  const int max_pages = (a.max_blocks + a.nsplit - 1) / a.nsplit;
  const FastLds lay = fast_lds(DH, NHP, a.num_tiers, a.G_max, a.cb_max, max_pages, P);
  float* lut = fsm + lay.lut;                     // [NH][tier][G_max][cb_max + 1], entry cb_max = 0
  float* qs = fsm + lay.q;
  _Float16* pa = reinterpret_cast<_Float16*>(fsm + lay.p) + wave * 256;   // P as the MFMA A operand, [16][16] fp16
  float* ts = fsm + lay.ts;                       // [tile][NH] (max, sum), log2 units
  int* tbl = reinterpret_cast<int*>(fsm + lay.tbl);   // [page] (phys, tier)
  float* red = fsm + lay.red;
  const int T = a.num_tiers, GM = a.G_max, CM = a.cb_max, CMP = CM + 1;
  const int U = T * GM * CM;                      // lookup-table entries per head row

  // ---- 1. this thread's first lookup-table entry (u = tid): its centroid row's
  // first 16 coordinates, loaded before anything is staged
  const bool vec = (a.g_max & 3) == 0;
  floatx4 cv0[4];
  {
    const int tier = tid / (GM * CM), r = tid - tier * GM * CM, g = r / CM, c = r - g * CM;
    const bool in = tid < U && vec;
    const float* row = in ? a.cb_flat + ((((int64_t)hkv * T + tier) * GM + g) * CM + c) * a.g_max : a.cb_flat;
    const int last = in ? a.g_max - 4 : 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) cv0[i] = *reinterpret_cast<const floatx4*>(row + (4 * i < last ? 4 * i : last));
  }

  // ---- 2. stage: tier geometry, block table range, scaled q, tile stats = (-inf, 0), P rows = 0.
  // The first slice of each staged array is loaded into registers before any
  // is written, so the loads share one round trip.
  const int64_t tb0 = (int64_t)hkv * a.max_blocks + rb;
  const int tgv0 = tid < T ? a.tier_G[tid] : 0, tgv1 = tid < T ? a.tier_g[tid] : 0;
  const int bt0 = tid < npg ? a.block_table[tb0 + tid] : 0, bb0 = tid < npg ? a.bits_table[tb0 + tid] : 0;
  const int qh0 = tid / DH;
  const float qv0 = tid < NH * DH && qh0 < a.kv_groups ? a.q[((int64_t)hkv * a.kv_groups + qh0) * DH + (tid - qh0 * DH)] : 0.f;
  const float qscale = a.sm_scale * kLog2e / 255.0f;
  if (tid < T) { tG[tid] = tgv0; tg[tid] = tgv1; }
  if (tid < npg) { tbl[2 * tid] = bt0; tbl[2 * tid + 1] = bb0; }
  if (tid < NH * DH) qs[tid] = qv0 * qscale;
  for (int i = tid + NTH; i < npg; i += NTH) {
    tbl[2 * i] = a.block_table[tb0 + i];
    tbl[2 * i + 1] = a.bits_table[tb0 + i];
  }
  for (int i = tid + NTH; i < NH * DH; i += NTH) {
    const int h = i / DH;
    qs[i] = h < a.kv_groups ? a.q[((int64_t)hkv * a.kv_groups + h) * DH + (i - h * DH)] * qscale : 0.f;
  }
  for (int i = tid; i < npg * TPP * NH; i += NTH) { ts[2 * i] = -INFINITY; ts[2 * i + 1] = 0.f; }
  for (int i = tid; i < W * 128; i += NTH) reinterpret_cast<uint32_t*>(fsm + lay.p)[i] = 0u;
  for (int i = tid; i < NH * T * GM; i += NTH) lut[i * CMP + CM] = 0.f;
  __syncthreads();

  const int t16 = lane & 15, hr = lane >> 4;
  const int dg = lane & 15, tq = lane >> 4;
  const int ntile = npg * TPP;
  const int k_begin = (int)((int64_t)ntile * wave / W), k_end = (int)((int64_t)ntile * (wave + 1) / W);
  const int nt = k_end - k_begin;
  const int tsh = (TPP & (TPP - 1)) == 0 ? __builtin_ctz(TPP) : -1;   // tiles per page as a shift

  // ---- 3. this wave's block-table entries, 64 pages at a time, one per lane
  int cbase = uniform(k_begin / TPP);
  int cph = cbase + lane < npg ? tbl[2 * (cbase + lane)] : -1;
  int ctr = cbase + lane < npg ? tbl[2 * (cbase + lane) + 1] : -1;

  // issue the loads of workgroup-local tile k (k >= k_end: nothing is read)
  auto issue = [&](FastTile<GV, DPL>& b, int k) {
    const bool in = k < k_end;
    const int kc = in ? k : k_begin;
    const int pl = uniform(tsh >= 0 ? kc >> tsh : kc / TPP), ti = kc - pl * TPP;
    if (pl - cbase >= 64) {
      cbase = pl;
      cph = cbase + lane < npg ? tbl[2 * (cbase + lane)] : -1;
      ctr = cbase + lane < npg ? tbl[2 * (cbase + lane) + 1] : -1;
    }
    const int phys = __builtin_amdgcn_readlane(cph, (pl - cbase) & 63), tier = __builtin_amdgcn_readlane(ctr, (pl - cbase) & 63);
    const bool tok = tier >= 0 && tier < T && tG[tier] >= 1 && tG[tier] <= GM && tg[tier] >= 1 &&
                     tg[tier] <= a.g_max && tG[tier] * tg[tier] <= DH;
    const bool live = in && phys >= 0 && phys < a.num_pages && tok;
    const int Gt = live ? tG[tier] : 0;
    b.live = live;
    b.tier = live ? tier : 0;
    b.slot = kc;
    const int64_t pg = live ? phys : 0;
    const rsrc_t rth = make_rsrc(a.theta_codes + pg * P * GM, live ? (int64_t)P * GM : 0);
    const rsrc_t rrd = make_rsrc(a.radius_codes + pg * P * GM, live ? (int64_t)P * GM : 0);
    const rsrc_t rrs = make_rsrc(a.r_scales + pg * GM, live ? (int64_t)GM * 4 : 0);
    const rsrc_t rv = make_rsrc(a.v_pool + pg * P * DH, live ? (int64_t)P * DH * 2 : 0);
    const int row = (ti * 16 + t16) * GV;
    if constexpr (GV == 8) {
      const u32x2 x = __builtin_amdgcn_raw_buffer_load_b64(rth, row, 0, 0);
      const u32x2 y = __builtin_amdgcn_raw_buffer_load_b64(rrd, row, 0, 0);
      b.th[0] = x[0]; b.th[1] = x[1]; b.rd[0] = y[0]; b.rd[1] = y[1];
    } else {
      b.th[0] = __builtin_amdgcn_raw_buffer_load_b32(rth, row, 0, 0);
      b.rd[0] = __builtin_amdgcn_raw_buffer_load_b32(rrd, row, 0, 0);
    }
    b.rs = __builtin_amdgcn_raw_buffer_load_b32(rrs, lane < Gt ? 4 * lane : kOOB, 0, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int off = ((ti * 16 + tq + 4 * j) * DH + DPL * dg) * 2;
      if constexpr (DPL == 8) {
        const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0);
        b.v[j][0] = w[0]; b.v[j][1] = w[1]; b.v[j][2] = w[2]; b.v[j][3] = w[3];
      } else {
        const u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(rv, off, 0, 0);
        b.v[j][0] = w[0]; b.v[j][1] = w[1];
      }
    }
  };

  // ---- 4. the first two tiles
  FastTile<GV, DPL> b0, b1;
  issue(b0, k_begin);
  issue(b1, k_begin + 1);

  // ---- 5. lookup table: entry u = (tier, g, c) holds <q_h,g, centroid> for
  // every head row h, one head row at a time
  auto entry_finish = [&](int tier, int g, int c, const floatx4 (&first)[4]) {
    const int gt = tg[tier];
    const float* row = a.cb_flat + ((((int64_t)hkv * T + tier) * GM + g) * CM + c) * a.g_max;
    const float* qg = qs + g * gt;
    float* dst = lut + (tier * GM + g) * CMP + c;
    for (int d0 = 0; d0 < gt; d0 += 16) {
      floatx4 cv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (d0 == 0) cv[i] = first[i];
        else cv[i] = *reinterpret_cast<const floatx4*>(row + (d0 + 4 * i < gt ? d0 + 4 * i : gt - 4));
        if (d0 + 4 * i + 4 > gt)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (d0 + 4 * i + e >= gt) cv[i][e] = 0.f;
      }
#pragma unroll 1
      for (int h = 0; h < NH; ++h) {
        float dot = d0 == 0 ? 0.f : dst[h * T * GM * CMP];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int dq = d0 + 4 * i + 4 <= gt ? d0 + 4 * i : 0;
          const floatx4 qv = *reinterpret_cast<const floatx4*>(qg + h * DH + dq);
#pragma unroll
          for (int e = 0; e < 4; ++e) dot = __builtin_fmaf(qv[e], cv[i][e], dot);
        }
        dst[h * T * GM * CMP] = dot;
      }
    }
  };
  auto do_entry = [&](int u, bool first_loaded) {
    if (u >= U) return;
    const int tier = u / (GM * CM), r = u - tier * GM * CM, g = r / CM, c = r - g * CM;
    const bool ok = tier_ok(a, tier, tG, tg) && g < tG[tier];
    if (ok && vec) {
      if (first_loaded) {
        entry_finish(tier, g, c, cv0);
      } else {
        const float* row = a.cb_flat + ((((int64_t)hkv * T + tier) * GM + g) * CM + c) * a.g_max;
        floatx4 cv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) cv[i] = *reinterpret_cast<const floatx4*>(row + (4 * i < a.g_max - 4 ? 4 * i : a.g_max - 4));
        entry_finish(tier, g, c, cv);
      }
    } else if (ok) {
      const int gt = tg[tier];
      const float* row = a.cb_flat + ((((int64_t)hkv * T + tier) * GM + g) * CM + c) * a.g_max;
      const float* qg = qs + g * gt;
      for (int h = 0; h < NH; ++h) {
        float dot = 0.f;
        for (int d = 0; d < gt; ++d) dot = __builtin_fmaf(qg[h * DH + d], row[d], dot);
        lut[((h * T + tier) * GM + g) * CMP + c] = dot;
      }
    } else {
      for (int h = 0; h < NH; ++h) lut[((h * T + tier) * GM + g) * CMP + c] = 0.f;
    }
  };
  do_entry(tid, true);
  for (int u = tid + NTH; u < U; u += NTH) do_entry(u, false);
  __syncthreads();

  // running (max, sum) of this lane's head rows (log2 units); P V accumulators
  // in the MFMA D layout: acc[j][i] = out[head 4 (lane / 16) + i][dim DPL (lane % 16) + j]
  float Mw[NHP], Lw[NHP];
  floatx4 acc[DPL];
#pragma unroll
  for (int hp = 0; hp < NHP; ++hp) { Mw[hp] = -INFINITY; Lw[hp] = 0.f; }
#pragma unroll
  for (int j = 0; j < DPL; ++j) acc[j] = floatx4{0.f, 0.f, 0.f, 0.f};

  auto process = [&](const FastTile<GV, DPL>& b) {
    if (!b.live) return;
    // logits of (token t16, head row hr + 4 hp); a code >= cb_max reads the
    // row's zero entry
    float lg[NHP];
#pragma unroll
    for (int hp = 0; hp < NHP; ++hp) {
      const float* lt = lut + ((hr + 4 * hp) * T + b.tier) * GM * CMP;
      float sum = 0.f;
#pragma unroll
      for (int g = 0; g < GV; ++g) {
        const uint32_t code = (b.th[g / 4] >> (8 * (g % 4))) & 0xFFu;
        const float rc = (float)((b.rd[g / 4] >> (8 * (g % 4))) & 0xFFu);
        const float rsg = __builtin_bit_cast(float, __builtin_amdgcn_readlane((int)b.rs, g));
        const float v = lt[g * CMP + (code < (uint32_t)CM ? code : (uint32_t)CM)];
        sum = __builtin_fmaf(rsg * rc, v, sum);
      }
      lg[hp] = sum == 0.f ? kNegLogit2 : sum;                               // decode_kernel.cu:194
    }
    bool grow = false;
    float fo[NHP];
#pragma unroll
    for (int hp = 0; hp < NHP; ++hp) {
      const float mt = rmax16(lg[hp]);
      const float e = __builtin_amdgcn_exp2f(lg[hp] - mt);
      const float ls = rsum16(e);
      if (t16 == 0) { ts[2 * (b.slot * NH + hr + 4 * hp)] = mt; ts[2 * (b.slot * NH + hr + 4 * hp) + 1] = ls; }
      const float mn = fmaxf(Mw[hp], mt);
      const float fn = __builtin_amdgcn_exp2f(mt - mn);
      fo[hp] = __builtin_amdgcn_exp2f(Mw[hp] - mn);
      grow |= mn > Mw[hp];
      Lw[hp] = Lw[hp] * fo[hp] + ls * fn;
      Mw[hp] = mn;
      // A operand row (head), k = 4 (t16 % 4) + t16 / 4 <-> token t16
      pa[(hr + 4 * hp) * 16 + 4 * (t16 & 3) + (t16 >> 2)] = (_Float16)(e * fn);
    }
    if (__builtin_amdgcn_ballot_w64(grow)) {
      float f[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f[i] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, fo[0]), 16 * i));
        if constexpr (NHP == 2) {
          const float f2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, fo[NHP - 1]), 16 * i));
          if (lane >= 16) f[i] = f2;
        }
      }
#pragma unroll
      for (int j = 0; j < DPL; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[j][i] *= f[i];
    }
    wave_lds_sync();
    // P (A: row = lane % 16, k = 4 (lane / 16) + i <-> token lane / 16 + 4 i)
    const half4 pA = *reinterpret_cast<const half4*>(pa + (lane & 15) * 16 + 4 * (lane >> 4));
    // V (B: column = lane % 16 <-> dim DPL (lane % 16) + j, k as above): this
    // lane's four token rows tq + 4 i, one dim per MFMA
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
      const uint32_t lo = __builtin_amdgcn_perm(b.v[1][j / 2], b.v[0][j / 2], sel);
      const uint32_t hi = __builtin_amdgcn_perm(b.v[3][j / 2], b.v[2][j / 2], sel);
      const half4 vB = __builtin_bit_cast(half4, (u32x2){lo, hi});
      acc[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(pA, vB, acc[j], 0, 0, 0);
    }
    wave_lds_sync();
  };

  for (int k = 0; k < nt; k += 2) {
    process(b0);
    issue(b0, k_begin + k + 2);
    if (k + 1 < nt) process(b1);
    issue(b1, k_begin + k + 3);
  }

  // ---- this wave's partial -> LDS
  float* rw = red + wave * NH * (DH + 2);
  if ((lane >> 4) < NHP)
#pragma unroll
    for (int j = 0; j < DPL; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) rw[(4 * (lane >> 4) + i) * (DH + 2) + 2 + DPL * dg + j] = acc[j][i];
  if (t16 == 0)
#pragma unroll
    for (int hp = 0; hp < NHP; ++hp) {
      rw[(hr + 4 * hp) * (DH + 2)] = Mw[hp];
      rw[(hr + 4 * hp) * (DH + 2) + 1] = Lw[hp];
    }
  __syncthreads();

  // ---- per-page (m, l) of each q head from its tiles (decode_kernel.cu:198-215)
  for (int i = tid; i < npg * a.kv_groups; i += 64 * W) {
    const int pl = i / a.kv_groups, h = i - pl * a.kv_groups;
    float m = -INFINITY;
    for (int t = 0; t < TPP; ++t) m = fmaxf(m, ts[2 * ((pl * TPP + t) * NH + h)]);
    float l = 0.f;
    if (m != -INFINITY)
      for (int t = 0; t < TPP; ++t) {
        const float mt = ts[2 * ((pl * TPP + t) * NH + h)];
        if (mt != -INFINITY) l += ts[2 * ((pl * TPP + t) * NH + h) + 1] * __builtin_amdgcn_exp2f(mt - m);
      }
    float* pt = a.partial + ((int64_t)(hkv * a.kv_groups + h) * a.max_blocks + rb + pl) * (DH + 2);
    pt[0] = m * kLn2;
    pt[1] = l;
  }
  // ---- merge the waves; write out (one range) or this range's partial
  for (int i = tid; i < a.kv_groups * DH; i += 64 * W) {
    const int h = i / DH, d = i - h * DH;
    float Mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < W; ++w) Mx = fmaxf(Mx, red[(w * NH + h) * (DH + 2)]);
    float Ls = 0.f, A = 0.f;
    if (Mx != -INFINITY)
#pragma unroll
      for (int w = 0; w < W; ++w) {
        const float mw = red[(w * NH + h) * (DH + 2)];
        if (mw == -INFINITY) continue;
        const float f = __builtin_amdgcn_exp2f(mw - Mx);
        Ls += f * red[(w * NH + h) * (DH + 2) + 1];
        A += f * red[(w * NH + h) * (DH + 2) + 2 + d];
      }
    const int hq = hkv * a.kv_groups + h;
    if (a.nsplit == 1) {
      a.out[(int64_t)hq * DH + d] = A / (Ls + 1e-8f);                    // decode_kernel.cu:244-245
    } else {
      float* e0 = a.partial + ((int64_t)hq * a.max_blocks + rb) * (DH + 2);
      e0[2 + d] = A;
      if (d == 0) {
        e0[(DH + 2) + 2] = Mx * kLn2;
        e0[(DH + 2) + 3] = Ls;
      }
    }
  }
}

static int64_t general_lds_bytes(int dh, int nhp, int num_tiers, int G_max, int cb_max, int page_size) {
  const int NH = 4 * nhp;
  return 4LL * ((int64_t)NH * num_tiers * G_max * cb_max + 4LL * page_size * NH + 4LL * NH * (dh + 2));
}

int64_t modea_configure(ModeALaunch& L) {
  const int nhp = L.kv_groups <= 4 ? 1 : 2;
  const int mb = L.max_blocks > 0 ? L.max_blocks : 1;
  L.fast = (L.G_max == 4 || L.G_max == 8) ? 1 : 0;
  // one 16-wave workgroup (fast) or eight 4-wave workgroups (general) per CU
  const int target = L.fast ? 256 : 2048;
  int nsplit = L.num_kv > 0 ? (target + L.num_kv - 1) / L.num_kv : 1;
  if (nsplit > mb / 2) nsplit = mb / 2;
  if (nsplit < 1) nsplit = 1;
  if (L.fast) {
    // the range's block table and tile stats live in LDS: split finer until they fit
    auto bytes = [&](int ns) {
      return (int64_t)fast_lds(L.dh, nhp, L.num_tiers, L.G_max, L.cb_max, (mb + ns - 1) / ns, L.page_size).total;
    };
    while (bytes(nsplit) > 160 * 1024 && nsplit < mb / 2) nsplit = nsplit * 2 <= mb / 2 ? nsplit * 2 : mb / 2;
    L.nsplit = nsplit;
    const int64_t b = bytes(nsplit);
    if (b <= 160 * 1024) return b;
    L.fast = 0;
  }
  L.nsplit = nsplit;
  return general_lds_bytes(L.dh, nhp, L.num_tiers, L.G_max, L.cb_max, L.page_size);
}

template <typename K>
static int launch_split(K kernel, const ModeALaunch& L, int threads, int64_t lds, hipStream_t stream) {
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)lds) != hipSuccess)
    return -1;
  hipLaunchKernelGGL(kernel, dim3(L.num_kv * L.nsplit), dim3(threads), (size_t)lds, stream, L);
  if (L.nsplit > 1)
    hipLaunchKernelGGL(modea_merge_kernel, dim3(L.num_q * ((L.dh + 63) / 64)), dim3(64 * kMergeWaves), 0, stream, L);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_modea(const ModeALaunch& L0, hipStream_t stream) {
  if (L0.num_kv <= 0 || L0.max_blocks <= 0) return 0;
  ModeALaunch L = L0;
  const int64_t lds = modea_configure(L);
  if (lds > 160 * 1024) return -1;
  const int nhp = L.kv_groups <= 4 ? 1 : 2;
  const int ft = 64 * kFastWaves;
  if (L.fast) {
    if (L.dh == 128 && nhp == 1) return L.G_max == 8 ? launch_split(&modea_fast_kernel<128, 1, 8>, L, ft, lds, stream)
                                                     : launch_split(&modea_fast_kernel<128, 1, 4>, L, ft, lds, stream);
    if (L.dh == 128 && nhp == 2) return L.G_max == 8 ? launch_split(&modea_fast_kernel<128, 2, 8>, L, ft, lds, stream)
                                                     : launch_split(&modea_fast_kernel<128, 2, 4>, L, ft, lds, stream);
    if (L.dh == 64 && nhp == 1) return L.G_max == 8 ? launch_split(&modea_fast_kernel<64, 1, 8>, L, ft, lds, stream)
                                                    : launch_split(&modea_fast_kernel<64, 1, 4>, L, ft, lds, stream);
    if (L.dh == 64 && nhp == 2) return L.G_max == 8 ? launch_split(&modea_fast_kernel<64, 2, 8>, L, ft, lds, stream)
                                                    : launch_split(&modea_fast_kernel<64, 2, 4>, L, ft, lds, stream);
    return -1;
  }
  if (L.dh == 128 && nhp == 1) return launch_split(&modea_split_kernel<128, 1>, L, 256, lds, stream);
  if (L.dh == 128 && nhp == 2) return launch_split(&modea_split_kernel<128, 2>, L, 256, lds, stream);
  if (L.dh == 64 && nhp == 1) return launch_split(&modea_split_kernel<64, 1>, L, 256, lds, stream);
  if (L.dh == 64 && nhp == 2) return launch_split(&modea_split_kernel<64, 2>, L, 256, lds, stream);
  return -1;
}

int launch_qlut(const ModeALaunch& L, float* lut, hipStream_t stream) {
  const int64_t total = (int64_t)L.num_q * L.num_tiers * L.G_max * L.cb_max;
  if (total > 0) {
    const int blocks = (int)((total + 255) / 256 < 4096 ? (total + 255) / 256 : 4096);
    hipLaunchKernelGGL(qlut_kernel, dim3(blocks), dim3(256), 0, stream, L, lut);
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// ---------------------------------------------------------------------------
// Logits from a precomputed LUT (new_fused_decode.py:22-43): logits_out fp32
// [num_q, max_ctx]; token n of kv head hkv lives in logical page n / P, slot
// n % P; n >= ctx_lens[hkv] or an absent page gives -inf.  One thread per
// (q head, token).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void lut_logits_kernel(LutLogitsLaunch a) {
  const int64_t total = (int64_t)a.num_q * a.max_ctx;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int hq = (int)(i / a.max_ctx);
    const int n = (int)(i - (int64_t)hq * a.max_ctx);
    const int hkv = hq / a.kv_groups;
    float out = -INFINITY;
    const int lb = n / a.page_size, slot = n - lb * a.page_size;
    if (hkv < a.num_kv && n < a.ctx_lens[hkv] && lb < a.max_blocks) {
      const int phys = a.block_table[(int64_t)hkv * a.max_blocks + lb];
      const int tier = a.bits_table[(int64_t)hkv * a.max_blocks + lb];
      if (phys >= 0 && phys < a.num_pages && tier >= 0 && tier < a.num_tiers) {
        const uint8_t* th = a.theta_codes + ((int64_t)phys * a.page_size + slot) * a.G_max;
        const uint8_t* rd = a.radius_codes + ((int64_t)phys * a.page_size + slot) * a.G_max;
        const float* rsc = a.r_scales + (int64_t)phys * a.G_max;
        const float* lt = a.q_lut + (((int64_t)hq * a.num_tiers + tier) * a.G_max) * a.cb_size_max;
        float sum = 0.f;
        for (int g = 0; g < a.G_max; ++g) {
          const int code = th[g];
          const float rh = rsc[g] * (float)rd[g] / 255.0f;
          const float v = code < a.cb_size_max ? lt[g * a.cb_size_max + code] : 0.f;
          sum = __builtin_fmaf(rh, v, sum);
        }
        out = sum * a.sm_scale;
      }
    }
    a.logits_out[i] = out;
  }
}

// The same logits, one thread per (kv head, token) serving all kv_groups q
// heads of that kv head: the token's codes and radius bytes are read once (8
// bytes each at G_max = 8), the page's scales once, and the kv head's
// q_lut rows are staged in LDS for the lookups.  A workgroup takes kLutTok
// tokens of one kv head.  Same arithmetic, in the same order, per (q head,
// token) as lut_logits_kernel.
constexpr int kLutTok = 256;
template <int GM>
__global__ __launch_bounds__(256) void lut_logits_group_kernel(LutLogitsLaunch a) {
  extern __shared__ float lut_s[];                     // [kv_groups][num_tiers][GM][cb_size_max]
  const int nb = (a.max_ctx + kLutTok - 1) / kLutTok;
  const int hkv = blockIdx.x / nb, n0 = (blockIdx.x % nb) * kLutTok;
  const int cb = a.cb_size_max, T = a.num_tiers, kg = a.kv_groups;
  const int rows = kg * T * GM * cb;
  const float* src = a.q_lut + (int64_t)hkv * kg * T * GM * cb;   // q heads hkv * kg .. + kg - 1
  for (int i = threadIdx.x; i < rows; i += 256) lut_s[i] = src[i];
  __syncthreads();
  const int ctx = a.ctx_lens[hkv];
  // the thread's kLutTok / 256 tokens, their loads issued together
  constexpr int NT = kLutTok / 256;
  int phys[NT], tier[NT];
  bool ok[NT];
#pragma unroll
  for (int k = 0; k < NT; ++k) {
    const int n = n0 + threadIdx.x + 256 * k, lb = n / a.page_size;
    ok[k] = n < a.max_ctx && n < ctx && lb < a.max_blocks;
    const int64_t bi = (int64_t)hkv * a.max_blocks + (ok[k] ? lb : 0);
    phys[k] = a.block_table[bi];
    tier[k] = a.bits_table[bi];
  }
  uint32_t tw[NT][GM / 4], rw[NT][GM / 4];
  float rsc[NT][GM];
#pragma unroll
  for (int k = 0; k < NT; ++k) {
    ok[k] = ok[k] && phys[k] >= 0 && phys[k] < a.num_pages && tier[k] >= 0 && tier[k] < T;
    const int n = n0 + threadIdx.x + 256 * k;
    const int slot = n - (n / a.page_size) * a.page_size;
    const int64_t pg = ok[k] ? phys[k] : 0;
    const int64_t e = (pg * a.page_size + slot) * GM;
#pragma unroll
    for (int w = 0; w < GM / 4; ++w) {
      tw[k][w] = *reinterpret_cast<const uint32_t*>(a.theta_codes + e + 4 * w);
      rw[k][w] = *reinterpret_cast<const uint32_t*>(a.radius_codes + e + 4 * w);
    }
#pragma unroll
    for (int g4 = 0; g4 < GM / 4; ++g4) {
      const float4 v = *reinterpret_cast<const float4*>(a.r_scales + pg * GM + 4 * g4);
      rsc[k][4 * g4] = v.x; rsc[k][4 * g4 + 1] = v.y; rsc[k][4 * g4 + 2] = v.z; rsc[k][4 * g4 + 3] = v.w;
    }
  }
#pragma unroll
  for (int k = 0; k < NT; ++k) {
    const int n = n0 + threadIdx.x + 256 * k;
    if (n >= a.max_ctx) continue;
    for (int j = 0; j < kg; ++j) {
      float out = -INFINITY;
      if (ok[k]) {
        const float* lt = lut_s + ((j * T + tier[k]) * GM) * cb;
        float sum = 0.f;
#pragma unroll
        for (int g = 0; g < GM; ++g) {
          const int code = (int)((tw[k][g >> 2] >> (8 * (g & 3))) & 0xFF);
          const float rd = (float)((rw[k][g >> 2] >> (8 * (g & 3))) & 0xFF);
          const float rh = rsc[k][g] * rd / 255.0f;
          const float v = code < cb ? lt[g * cb + code] : 0.f;
          sum = __builtin_fmaf(rh, v, sum);
        }
        out = sum * a.sm_scale;
      }
      a.logits_out[(int64_t)(hkv * kg + j) * a.max_ctx + n] = out;
    }
  }
}

int launch_lut_logits(const LutLogitsLaunch& L, hipStream_t stream) {
  const int64_t total = (int64_t)L.num_q * L.max_ctx;
  if (total <= 0) return 0;
  const int64_t lds = (int64_t)L.kv_groups * L.num_tiers * L.G_max * L.cb_size_max * 4;
  const int64_t blocks = (int64_t)L.num_kv * ((L.max_ctx + kLutTok - 1) / kLutTok);
  // (code rows and page scales are read in 4- and 16-byte words: their bases must be aligned)
  const bool aligned = ((uintptr_t)L.theta_codes % 4) == 0 && ((uintptr_t)L.radius_codes % 4) == 0 &&
                       ((uintptr_t)L.r_scales % 16) == 0;
  // (the grouped kernel reads row 0 of the tables for absent tokens: both must exist)
  if ((L.G_max == 8 || L.G_max == 4) && aligned && lds <= 48 * 1024 && L.num_q == L.num_kv * L.kv_groups &&
      blocks < (1 << 30) && L.max_blocks >= 1 && L.num_pages >= 1) {
    if (L.G_max == 8)
      hipLaunchKernelGGL(lut_logits_group_kernel<8>, dim3((unsigned)blocks), dim3(256), (size_t)lds, stream, L);
    else
      hipLaunchKernelGGL(lut_logits_group_kernel<4>, dim3((unsigned)blocks), dim3(256), (size_t)lds, stream, L);
  } else {
    const int nblk = (int)((total + 255) / 256 < 8192 ? (total + 255) / 256 : 8192);
    hipLaunchKernelGGL(lut_logits_kernel, dim3(nblk), dim3(256), 0, stream, L);
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace sphkv

namespace sphkv {

// ---------------------------------------------------------------------------
// omega EMA from the decode's per-page statistics (spherical_kv_pipeline.py:
// 952-987): per q head, pages with l > 0 compete in a softmax of their (m, l)
// -- w = exp(max(m - max_p m, -60)) * l, mass = w / max(sum w, 1e-12) -- the
// masses are averaged over each kv head's q heads and blended into omega:
// omega' = omega * beta + mass * (1 - beta).  One workgroup per kv head.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float block_reduce(float v, bool is_max, float* red) {
  for (int o = 32; o >= 1; o >>= 1) {
    const float x = __shfl_xor(v, o, 64);
    v = is_max ? fmaxf(v, x) : v + x;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); ++w) r = is_max ? fmaxf(r, red[w]) : r + red[w];
  return r;
}

__global__ __launch_bounds__(256) void omega_ema_kernel(OmegaLaunch a) {
  __shared__ float red[4];
  __shared__ float mx_s[kOmegaMaxGroups], z_s[kOmegaMaxGroups];
  const int h = blockIdx.x;
  for (int r = 0; r < a.kv_groups; ++r) {
    const int64_t qb = (int64_t)(h * a.kv_groups + r) * a.q_stride;
    float mx = -1e30f;
    for (int p = threadIdx.x; p < a.max_blocks; p += blockDim.x) {
      const float l = a.l[qb + (int64_t)p * a.page_stride];
      if (l > 0.f) mx = fmaxf(mx, a.m[qb + (int64_t)p * a.page_stride]);
    }
    mx = block_reduce(mx, true, red);
    float z = 0.f;
    for (int p = threadIdx.x; p < a.max_blocks; p += blockDim.x) {
      const float l = a.l[qb + (int64_t)p * a.page_stride];
      const float m = l > 0.f ? a.m[qb + (int64_t)p * a.page_stride] : -1e30f;
      z += expf(fmaxf(m - mx, -60.f)) * l;
    }
    z = block_reduce(z, false, red);
    if (threadIdx.x == 0) { mx_s[r] = mx; z_s[r] = fmaxf(z, 1e-12f); }
  }
  __syncthreads();
  for (int p = threadIdx.x; p < a.max_blocks; p += blockDim.x) {
    float s = 0.f;
    for (int r = 0; r < a.kv_groups; ++r) {
      const int64_t qb = (int64_t)(h * a.kv_groups + r) * a.q_stride + (int64_t)p * a.page_stride;
      const float l = a.l[qb];
      const float m = l > 0.f ? a.m[qb] : -1e30f;
      s += expf(fmaxf(m - mx_s[r], -60.f)) * l / z_s[r];
    }
    const float mass = s / (float)a.kv_groups;
    const int64_t o = (int64_t)h * a.max_blocks + p;
    a.omega_out[o] = a.omega_prev[o] * a.beta + mass * (1.f - a.beta);
  }
}

// Single-pass form for kv_groups <= KG (4 or 8) and max_blocks <= 1024 * PPT:
// 1024 threads per kv head, each holding the (m, l) of its PPT pages for every
// q head of the group in registers (read once; one 8-byte load per pair when
// l directly follows m, as in partial_scratch; no load for q heads past
// kv_groups), the group's maxima and sums reduced together.  Same formula as
// omega_ema_kernel.
template <int PPT, int KG>
__global__ __launch_bounds__(1024) void omega_ema_fast_kernel(OmegaLaunch a, int adjacent) {
  __shared__ float red[16][KG];
  const int h = blockIdx.x, kg = a.kv_groups;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float mv[KG][PPT], lv[KG][PPT];
#pragma unroll
  for (int r = 0; r < KG; ++r) {
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int p = threadIdx.x + 1024 * i;
      const bool ok = r < kg && p < a.max_blocks;
      const int64_t o = (int64_t)(h * kg + (r < kg ? r : 0)) * a.q_stride + (int64_t)(ok ? p : 0) * a.page_stride;
      float m = 0.f, l = 0.f;
      if (r >= kg) {                                   // uniform: no q head r in this group
      } else if (adjacent) {
        const float2 v = *reinterpret_cast<const float2*>(a.m + o);
        m = v.x; l = v.y;
      } else {
        m = a.m[o]; l = a.l[o];
      }
      lv[r][i] = ok ? l : 0.f;
      mv[r][i] = (ok && l > 0.f) ? m : -1e30f;          // invalid pages do not win the max
    }
  }
  auto reduce = [&](float (&v)[KG], bool is_max) {     // every q head of the group at once
#pragma unroll
    for (int r = 0; r < KG; ++r)
      for (int d = 32; d >= 1; d >>= 1) {
        const float x = __shfl_xor(v[r], d, 64);
        v[r] = is_max ? fmaxf(v[r], x) : v[r] + x;
      }
    __syncthreads();                                   // red is free
    if (lane == 0)
#pragma unroll
      for (int r = 0; r < KG; ++r) red[wave][r] = v[r];
    __syncthreads();
#pragma unroll
    for (int r = 0; r < KG; ++r) {
      float t = red[0][r];
      for (int w = 1; w < 16; ++w) t = is_max ? fmaxf(t, red[w][r]) : t + red[w][r];
      v[r] = t;
    }
  };
  float mx[KG], z[KG];
#pragma unroll
  for (int r = 0; r < KG; ++r) {
    mx[r] = -1e30f;
#pragma unroll
    for (int i = 0; i < PPT; ++i) mx[r] = fmaxf(mx[r], mv[r][i]);
  }
  reduce(mx, true);
#pragma unroll
  for (int r = 0; r < KG; ++r) {
    z[r] = 0.f;
#pragma unroll
    for (int i = 0; i < PPT; ++i) z[r] += expf(fmaxf(mv[r][i] - mx[r], -60.f)) * lv[r][i];
  }
  reduce(z, false);
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    const int p = threadIdx.x + 1024 * i;
    if (p >= a.max_blocks) continue;
    float s = 0.f;
#pragma unroll
    for (int r = 0; r < KG; ++r)
      if (r < kg) s += expf(fmaxf(mv[r][i] - mx[r], -60.f)) * lv[r][i] / fmaxf(z[r], 1e-12f);
    const float mass = s / (float)kg;
    const int64_t o = (int64_t)h * a.max_blocks + p;
    a.omega_out[o] = a.omega_prev[o] * a.beta + mass * (1.f - a.beta);
  }
}

int launch_omega(const OmegaLaunch& L, hipStream_t stream) {
  if (L.num_kv <= 0 || L.max_blocks <= 0) return 0;
  // (an 8-byte (m, l) load needs l right after m and 8-byte alignment at every page)
  const bool adjacent = L.l == L.m + 1 && ((uintptr_t)L.m % 8) == 0 && L.q_stride % 2 == 0 && L.page_stride % 2 == 0;
  if (L.kv_groups <= 4 && L.max_blocks <= 4096) {
    if (L.max_blocks <= 2048)
      hipLaunchKernelGGL((omega_ema_fast_kernel<2, 4>), dim3(L.num_kv), dim3(1024), 0, stream, L, (int)adjacent);
    else
      hipLaunchKernelGGL((omega_ema_fast_kernel<4, 4>), dim3(L.num_kv), dim3(1024), 0, stream, L, (int)adjacent);
  } else if (L.kv_groups <= 8 && L.max_blocks <= 4096) {
    if (L.max_blocks <= 2048)
      hipLaunchKernelGGL((omega_ema_fast_kernel<2, 8>), dim3(L.num_kv), dim3(1024), 0, stream, L, (int)adjacent);
    else
      hipLaunchKernelGGL((omega_ema_fast_kernel<4, 8>), dim3(L.num_kv), dim3(1024), 0, stream, L, (int)adjacent);
  } else {
    hipLaunchKernelGGL(omega_ema_kernel, dim3(L.num_kv), dim3(256), 0, stream, L);
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace sphkv

namespace sphkv {

// ---------------------------------------------------------------------------
// LayerPool pages from per-(head, tier) token arrays (sphkv_lut.py:44-66):
// page i (pool page pid0 + i) takes npg <= page_size tokens of a tier with
// G_t groups: r_scale[g] = max(max_n r[n, g], 1e-8); radius code =
// clamp(round_half_even(r / r_scale * 255), 0, 255); theta code = low byte of
// theta; V rows copied.  Slots past npg and groups past G_t are left as they
// are (the caller's pools start zeroed).  One workgroup per page.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void layer_pool_build_kernel(PoolBuildLaunch a) {
  __shared__ float rscl[kPoolBuildMaxG];
  const int i = blockIdx.x;
  const int32_t* d = a.page_src + 4 * (int64_t)i;
  const int64_t off = d[0], voff = d[1];
  const int npg = d[2], Gt = d[3];
  if (npg < 0 || npg > a.page_size || Gt < 1 || Gt > a.G_max || off < 0 || voff < 0 ||
      off + (int64_t)npg * Gt > a.n_elems || voff + npg > a.n_vrows)
    return;                                          // malformed descriptor: page left untouched
  const int64_t pid = (int64_t)a.pid0 + i;
  for (int g = threadIdx.x; g < Gt; g += blockDim.x) {
    float m = -INFINITY;
    for (int n = 0; n < npg; ++n) m = fmaxf(m, a.r[off + (int64_t)n * Gt + g]);
    const float s = fmaxf(m, 1e-8f);                 // .amax(dim=0).clamp(min=1e-8)
    rscl[g] = s;
    a.r_scales[pid * a.G_max + g] = s;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < npg * Gt; e += blockDim.x) {
    const int n = e / Gt, g = e - n * Gt;
    const float q = rintf(a.r[off + e] / rscl[g] * 255.0f);
    const int64_t dst = (pid * a.page_size + n) * a.G_max + g;
    a.radius_codes[dst] = (uint8_t)fminf(fmaxf(q, 0.f), 255.f);
    a.theta_codes[dst] = (uint8_t)(a.theta[off + e] & 0xFF);
  }
  const uint32_t* vs = reinterpret_cast<const uint32_t*>(a.v + voff * a.dh);
  uint32_t* vd = reinterpret_cast<uint32_t*>(a.v_pool + pid * a.page_size * a.dh);
  for (int e = threadIdx.x; e < npg * a.dh / 2; e += blockDim.x) vd[e] = vs[e];
}

int launch_pool_build(const PoolBuildLaunch& L, hipStream_t stream) {
  if (L.n_pages > 0)
    hipLaunchKernelGGL(layer_pool_build_kernel, dim3(L.n_pages), dim3(256), 0, stream, L);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace sphkv
