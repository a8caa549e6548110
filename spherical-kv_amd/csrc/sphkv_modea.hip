// Mode-A (LayerPool) kernels: the unpacked-pool decode path of the reference's
// fused_decode.py / sphkv_lut.py / new_fused_decode.py, built for gfx950.
//
// Pools (sphkv_lut.py:71-80): theta_codes / radius_codes uint8
// [n_pages, page_size, G_max], r_scales fp32 [n_pages, G_max], v_pool fp16
// [n_pages, page_size, dh] (token-major); per kv head a block table (logical
// page -> pool page, -1 = none) and a bits table (logical page -> tier index);
// cb_flat fp32 [num_kv, num_tiers, G_max, cb_max, g_max] (zero padded).
// Radii are uint8 with r_hat = r_scale * code / 255 (decode_kernel.cu:171).
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
//   modea_split_kernel Mode-A decode (decode_kernel.cu:108-220): one
//                      workgroup per (kv head, range of logical pages); the
//                      kv head's q heads share every page read; per page and q
//                      head it writes the reference's (m, l) into
//                      partial_scratch[..., 0:2] (read by the omega-EMA update,
//                      spherical_kv_pipeline.py:1690-1701); per range one
//                      online-softmax partial (m, l, acc[dh]).
//   modea_merge_kernel log-sum-exp merge of the ranges (decode_kernel.cu:223-246):
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
  __shared__ float s_k[kAppendMaxDh];
  __shared__ float s_norm[kAppendMaxDh], s_inv[kAppendMaxDh];
  __shared__ float s_sim[kAppendMaxSims];
  const int64_t pid = a.pids[h];
  if (pid < 0 || pid >= a.num_pages) return;        // no such pool page: nothing is written
  const int64_t row = pid * a.page_size + a.slot;   // (page, slot)
  if (tid < a.dh) {
    s_k[tid] = a.k_post[(int64_t)h * a.dh + tid];
    a.v_pool[row * a.dh + tid] = (_Float16)a.v_new[(int64_t)h * a.dh + tid];   // round to nearest even
  }
  __syncthreads();
  // decode_kernel.cu:46-50: norm = sqrt(sum k^2 + 1e-16), inv = 1 / (norm + 1e-8)
  if (tid < a.G) {
    const float* kg = s_k + tid * a.g;
    float nsq = 0.f;
    for (int d = 0; d < a.g; ++d) nsq = __builtin_fmaf(kg[d], kg[d], nsq);
    const float nrm = __builtin_sqrtf(nsq + 1e-16f);
    s_norm[tid] = nrm;
    s_inv[tid] = 1.0f / (nrm + 1e-8f);
  }
  __syncthreads();
  // decode_kernel.cu:52-58: sim_c = sum_d (k_d * inv) * cb[c][d], in d order
  const int nsim = a.G * a.C;
  for (int i = tid; i < nsim; i += kAppendThreads) {
    const int grp = i / a.C, c = i - grp * a.C;
    const float* kg = s_k + grp * a.g;
    const float inv = s_inv[grp];
    const float* cb = a.decode_cb + (((int64_t)h * a.G + grp) * a.C + c) * a.g;
    float sim = 0.f;
    for (int d = 0; d < a.g; ++d) sim = __builtin_fmaf(kg[d] * inv, cb[d], sim);
    s_sim[i] = sim;
  }
  __syncthreads();
  if (tid < a.G) {
    const int grp = tid;
    float best = -1e30f;
    int code = 0;
    for (int c = 0; c < a.C; ++c) {
      const float v = s_sim[grp * a.C + c];
      if (v > best) { best = v; code = c; }
    }
    a.theta_codes[row * a.G_max + grp] = (uint8_t)code;
    // decode_kernel.cu:64-82: per-page running-max radius scale
    const float nrm = s_norm[grp];
    float* rs = a.r_scales + pid * a.G_max + grp;
    float r_scale;
    if (a.is_new_page) {
      *rs = nrm;
      r_scale = nrm;
    } else {
      const float prev = *rs;
      if (nrm > prev) {
        const float ratio = prev / (nrm + 1e-8f);
        for (int t = 0; t < a.slot; ++t) {
          uint8_t* rc = a.radius_codes + (pid * a.page_size + t) * a.G_max + grp;
          float x = (float)(*rc) * ratio;
          x = fminf(fmaxf(roundf(x), 0.f), 255.f);
          *rc = (uint8_t)x;
        }
        *rs = nrm;
        r_scale = nrm;
      } else {
        r_scale = prev;
      }
    }
    float rq = roundf(nrm / (r_scale + 1e-8f) * 255.0f);
    rq = fminf(fmaxf(rq, 0.f), 255.f);
    a.radius_codes[row * a.G_max + grp] = (uint8_t)rq;
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
  for (int d = 0; d < gt; ++d) dot = __builtin_fmaf(qg[d], cb[d], dot);   // decode_kernel.cu:175-177 order
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

template <int DH, int NHP>
__global__ __launch_bounds__(256) void modea_split_kernel(ModeALaunch a) {
  constexpr int NH = 4 * NHP;              // q-head rows (padded)
  constexpr int DPL = DH / 16;             // dims per lane in P V (16 lanes cover a token row)
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int wave = uniform(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int hkv = blockIdx.x / a.nsplit, s = blockIdx.x % a.nsplit;
  const int pb = s * a.ppw, pe = (s == a.nsplit - 1) ? a.max_blocks : pb + a.ppw;
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
          const float rh = rsc[g] * (float)rd[g] / 255.0f;          // decode_kernel.cu:171
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

// One workgroup per q head: log-sum-exp over the ranges' partials.
__global__ __launch_bounds__(128) void modea_merge_kernel(ModeALaunch a) {
  const int hq = blockIdx.x;
  const int d = threadIdx.x;
  if (d >= a.dh) return;
  float Mx = -INFINITY;
  for (int s = 0; s < a.nsplit; ++s)
    Mx = fmaxf(Mx, a.partial[((int64_t)hq * a.max_blocks + s * a.ppw + 1) * (a.dh + 2) + 2]);
  float Ls = 0.f, A = 0.f;
  if (Mx != -INFINITY)
    for (int s = 0; s < a.nsplit; ++s) {
      const float* e0 = a.partial + ((int64_t)hq * a.max_blocks + s * a.ppw) * (a.dh + 2);
      const float* e1 = e0 + (a.dh + 2);
      if (e1[2] == -INFINITY) continue;
      const float f = fast_exp(e1[2] - Mx);
      Ls += f * e1[3];
      A += f * e0[2 + d];
    }
  a.out[(int64_t)hq * a.dh + d] = A / (Ls + 1e-8f);
}

int64_t modea_split_lds_bytes(int dh, int nhp, int num_tiers, int G_max, int cb_max, int page_size) {
  const int NH = 4 * nhp;
  return 4LL * ((int64_t)NH * num_tiers * G_max * cb_max + 4LL * page_size * NH + 4LL * NH * (dh + 2));
}

template <int DH, int NHP>
static int launch_modea_t(const ModeALaunch& L, hipStream_t stream) {
  const int64_t lds = modea_split_lds_bytes(DH, NHP, L.num_tiers, L.G_max, L.cb_max, L.page_size);
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(&modea_split_kernel<DH, NHP>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
    return -1;
  hipLaunchKernelGGL((modea_split_kernel<DH, NHP>), dim3(L.num_kv * L.nsplit), dim3(256), (size_t)lds, stream, L);
  if (L.nsplit > 1) hipLaunchKernelGGL(modea_merge_kernel, dim3(L.num_q), dim3(128), 0, stream, L);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_modea(const ModeALaunch& L, hipStream_t stream) {
  if (L.num_kv <= 0 || L.max_blocks <= 0) return 0;
  const int nhp = L.kv_groups <= 4 ? 1 : 2;
  if (L.dh == 128 && nhp == 1) return launch_modea_t<128, 1>(L, stream);
  if (L.dh == 128 && nhp == 2) return launch_modea_t<128, 2>(L, stream);
  if (L.dh == 64 && nhp == 1) return launch_modea_t<64, 1>(L, stream);
  if (L.dh == 64 && nhp == 2) return launch_modea_t<64, 2>(L, stream);
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

int launch_lut_logits(const LutLogitsLaunch& L, hipStream_t stream) {
  const int64_t total = (int64_t)L.num_q * L.max_ctx;
  if (total > 0) {
    const int blocks = (int)((total + 255) / 256 < 8192 ? (total + 255) / 256 : 8192);
    hipLaunchKernelGGL(lut_logits_kernel, dim3(blocks), dim3(256), 0, stream, L);
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace sphkv
