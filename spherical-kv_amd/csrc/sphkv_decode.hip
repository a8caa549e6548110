// Angle-domain paged attention decode (gfx950).
//
// Work decomposition: one workgroup (kWaves waves) per work item = the
// pointer-table rows first, first + stride, ... (< end) of one (sequence, kv
// head); the host interleaves a head's rows over its items (stride = the
// head's item count), so every item holds the same mix of tiers.  The
// workgroup stages that head's tier codebooks and the RoPE tables in LDS once;
// each wave walks every kWaves-th page of the range with its own online-softmax
// state; the states are merged in LDS and written as one (m, l, acc) partial.
// A second, widely parallel kernel merges the partials of each (sequence, kv
// head) (log-sum-exp) and writes the fp16 output.  (Merging in the workgroup
// that completes a head needs device-scope stores, loads and counters, whose
// cost on MI355X exceeds the kernel boundary.)
//
// Page loop, software pipelined per wave: while page k is computed, the
// 512-byte staging window and positions of the wave's next page and its V and
// (dense pages) its K rows are in flight.  The pointer-table rows, V slots
// and header dwords of 64 pages at a time are loaded one page per lane and
// checked lane-parallel (the page table); a page step reads its page's
// descriptor and load bases with readlane, and its remaining scalar work
// (page centre, issue priority) is integer arithmetic on scalar registers.
// Every lane's load offsets are fixed for the whole item.
//
// Per page (16 tokens, positions pos_t), lane l = (token t = l % 16, quarter
// u = l / 16), page centre t_mid = (min pos + max pos) / 2:
//   1. the query rows are rotated once per page by -t_mid (fp32, lanes = RoPE
//      frequencies j) and kept in LDS in the QK MFMA's operand order;
//   2. k_hat of token t on this lane's 32 dimensions (chunk_dim):
//      compressed  k_hat_d = r_hat_g * centroid_g[code][d mod g],
//                  r_hat_g = int8 / 127 * scale_g         (pagebuilder.py:17-21)
//                  (the 1/127 goes into the page's logit scale)
//      dense       k_hat_d = K[t][d] (fp16);
//   3. k_rot = R(pos_t - t_mid) k_hat in fp32 with phasors from an LDS table
//      of e^{i 2 pi f_j d}, |d| < kDelta (a page with a token beyond forms all
//      its phasors directly).  Since <R(-pos) q, k_hat> = <R(-t_mid) q,
//      R(pos - t_mid) k_hat>, this is the reference's back-rotated query
//      (spherical_kv_pipeline.py:2143-2176; its clip of the cosine to [-1, 1]
//      only acts on rounding error).  Phases are formed in fp64 turns and
//      reduced to [0, 1) before the fp32 hardware sine / cosine;
//   4. S[t][h] = k_rot . q_rot_h on the fp32 MFMA (4x4x1, 16 blocks = 4 lane
//      quarters x 4 token groups, one dimension per instruction; GQA 8 runs
//      two head sets), then the quarters' partial sums are added with row
//      swaps: fp32 products and sums, no operand splitting;
//   5. online softmax in the log2 domain.  The running reference max of a head
//      only moves when a page's max exceeds it by more than 2^8, so the
//      accumulator rescale is rare; p = 2^(s - m) <= 256 is rounded to fp16 and
//      the same rounded p is summed into l, so the output stays an exact
//      convex combination of V rows;
//   6. O[h][d] += P[h][t] V[t][d] on MFMA (4x4x4 f16, 16 blocks of 4 dims),
//      V read in the pool's MFMA operand order.
#include <hip/hip_ext.h>

#include "sphkv_common.h"
#include "sphkv_internal.h"

namespace sphkv {

// Events the next decode_kernel launch on this thread records its own start
// and stop in (hipExtLaunchKernel), then forgets (sphkv_time_next_decode_kernel).
thread_local hipEvent_t g_time_start = nullptr, g_time_stop = nullptr;

void set_decode_timing(hipEvent_t start, hipEvent_t stop) {
  g_time_start = start;
  g_time_stop = stop;
}

// decode_kernel launch, with the kernel-only timestamps when they were asked for
template <typename K, typename... A>
static void launch_timed(K kernel, dim3 grid, dim3 block, hipStream_t stream, A... args) {
  if (g_time_start && g_time_stop) {
    hipExtLaunchKernelGGL(kernel, grid, block, 0, stream, g_time_start, g_time_stop, 0, args...);
    g_time_start = g_time_stop = nullptr;
  } else {
    hipLaunchKernelGGL(kernel, grid, block, 0, stream, args...);
  }
}

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
  uint32_t* status;      // [0]: malformed rows / pages seen (accumulates until a merge)
  int32_t num_kv;
  int32_t num_rows;
  int32_t num_sh;        // num_seqs * num_kv
  int32_t pages32;       // pages_bytes (< 2^31)
  int32_t pages_m8;      // pages_bytes - 8: last offset a page header fits at
  int32_t nvp32;         // num_vpages clamped to 2^31 - 1
  float scale_log2;      // sm_scale * log2(e): logit scale of dense pages
  float scale_log2_c;    // scale_log2 / 127: compressed pages' radii carry the int8 code
  double log2_theta;
};

constexpr float kRescaleLog2 = 8.0f;   // reference-max hysteresis (log2 units)

// Buffer resources of the kernel-wide arrays, built once per wave (scalar
// registers).  A load of absent data adds kOOB to its offset, which puts it
// beyond every resource (the host keeps the byte pool and the position table
// below kOOB bytes), so it returns zeros without touching memory.
struct Res {
  rsrc_t pages, ptab, vslot, pos;
};

__device__ __forceinline__ Res make_res(const DecodeArgs& a) {
  Res r;
  r.pages = make_rsrc(a.pages, a.pages_bytes);
  r.ptab = make_rsrc(a.ptable, (int64_t)a.num_rows * 12);
  r.vslot = make_rsrc(a.vslot, (int64_t)a.num_rows * 4);
  r.pos = make_rsrc(a.positions, (int64_t)a.num_rows * 4 * kTile);
  return r;
}

// Dimension of element s of chunk c for lane quarter u.  A lane's chunks
// cover two runs of DH/8 dimensions: [(DH/8)u, (DH/8)(u+1)) of the first RoPE
// half (chunks c < NP) and the same run of the second half (chunks c >= NP),
// so every RoPE pair (j, j + DH/2) lies in one lane and a lane touches exactly
// two codebook groups.  The QK MFMA's reduction index follows this order on
// both operands.
template <int DH>
__host__ __device__ constexpr int chunk_dim(int c, int u) {
  return (c >= DH / 64 ? DH / 2 : 0) + (DH / 8) * u + 8 * (c % (DH / 64));
}

// Per-lane byte offsets of the page loads, fixed for a whole work item (lane
// l = token t = l % 16, quarter u = l / 16).  Lanes that load nothing carry
// kOOB; the page-dependent part is a wave-uniform base added to them.
struct LaneOff {
  uint32_t stg, pos, kd, v;
};

template <int DH>
__device__ __forceinline__ LaneOff lane_offsets(int lane) {
  const int t = lane & 15, u = lane >> 4;
  LaneOff o;
  o.stg = 8u * lane;                                        // 512-byte staging window
  o.pos = 4u * t;                                           // position of token t
  o.kd = (uint32_t)(t * DH + chunk_dim<DH>(0, u)) * 2u;     // dense K: chunk 0 of (t, u)
  o.v = (uint32_t)lane * kTile * 2u;                        // V: dim `lane`, 16 tokens
  return o;
}

__device__ __forceinline__ uint32_t oob_or(int ok, uint32_t base) { return ok ? base : (uint32_t)kOOB; }

// Page table of up to 64 pages of a wave, one page per lane (lane i: the
// wave's page kb + i).  Lanes load the pages' pointer-table rows, V slots
// and header dwords and check them once, lane-parallel, so a page step only
// reads its page's entries with readlane.  A malformed row or page
// contributes no token and is counted: a row that does not address the pools
// (page_off < 0, not 4-byte aligned, header past the pool, V slot past the
// pool), an unknown tier id, a count above 16, a dense page whose K rows are
// not 16-byte aligned inside its section and the pool, a compressed page
// whose sections leave its 512-byte staging window or the pool.
//   sbase  staging-window offset (page_off), kOOB for a bad row
//   vsl    V slot, -1 for a bad row
//   dbase  dense K rows (th_off) of a row that can be a dense page's (th_off
//          16-byte aligned, th_off + 2*DH <= rad_off: a compressed page's
//          theta section is < 2*DH bytes), kOOB otherwise -- a prefetch hint;
//          the header decides how the page is processed
//   desc   tier (1..3, 0: none) | dense << 2 | n << 3 | thr << 8 | rdr << 18 |
//          bad << 28: the page's tokens to use and its compressed sections'
//          offsets from the page start
struct PageRows { int page_off, th_off, rad_off, vs; };
struct PageTab { int sbase, vsl, dbase, desc; };

__device__ __forceinline__ PageRows rows_issue(const Res& rs, int p0, int wstride, int kb, int nwp, int lane) {
  const int k = kb + lane;
  const uint32_t p = (uint32_t)(k < nwp ? p0 + k * wstride : 0);
  const auto w = __builtin_amdgcn_raw_buffer_load_b96(rs.ptab, (int)(k < nwp ? 12u * p : (uint32_t)kOOB), 0, 0);
  PageRows r;
  r.page_off = (int)w[0];
  r.th_off = (int)w[1];
  r.rad_off = (int)w[2];
  r.vs = __builtin_amdgcn_raw_buffer_load_b32(rs.vslot, (int)(k < nwp ? 4u * p : (uint32_t)kOOB), 0, 0);
  return r;
}

// Row checks (lane-parallel): the staging / V / dense-K load bases.
template <int DH>
__device__ __forceinline__ PageTab page_bases(const DecodeArgs& a, const PageRows& r, int kb, int nwp, int lane) {
  const bool present = kb + lane < nwp;
  const bool ok = present && (r.page_off & 0x80000003) == 0 && r.page_off <= a.pages_m8 &&
                  (uint32_t)r.vs < (uint32_t)a.nvp32;
  const bool dense_like = ok && (r.th_off & 0x8000000F) == 0 && r.rad_off >= 0 &&
                          (uint32_t)r.th_off + 2 * DH <= (uint32_t)r.rad_off;
  PageTab t;
  t.sbase = ok ? r.page_off : kOOB;
  t.vsl = ok ? r.vs : -1;
  t.dbase = dense_like ? r.th_off : kOOB;
  t.desc = 0;
  return t;
}

// Header dword of each lane's page (zero for a bad row: its load is out of
// range).
__device__ __forceinline__ int header_issue(const Res& rs, const PageTab& t) {
  return __builtin_amdgcn_raw_buffer_load_b32(rs.pages, t.sbase, 0, 0);
}

// Header checks (lane-parallel) -> desc; returns the bad pages' count.
template <int DH>
__device__ __forceinline__ int page_check(const DecodeArgs& a, const PageRows& r, PageTab& t, int hw, int kb,
                                          int nwp, int lane) {
  const bool present = kb + lane < nwp;
  const bool ok = t.sbase != kOOB;
  const int tid = ok ? (hw & 0xFF) : 0;
  const int cnt = (hw >> 8) & 0xFF;
  const bool dense = tid == kDenseTier;
  const bool comp = (uint32_t)(tid - 1) < 3u;                  // tiers 1..3
  bool bad = (present && !ok) || (ok && !(dense || comp)) || ((dense || comp) && cnt > kTile);
  int n = (dense || comp) ? min(cnt, kTile) : 0;
  int thr = 0, rdr = 0;
  if (comp) {
    // theta bytes ceil(n*G*b/8) and radius bytes n*G of tiers 1, 2, 3; the
    // theta section ends 4 bytes before the window's end (the code reads
    // take 64 bits)
    const int G = DH / tier_g(tid), tb = (n * G * tier_b(tid) + 7) >> 3, rbytes = n * G;
    const int t0 = (int)((uint32_t)r.th_off - (uint32_t)r.page_off);
    const int r0 = (int)((uint32_t)r.rad_off - (uint32_t)r.page_off);
    const bool sec_ok = r.th_off >= r.page_off && r.rad_off >= r.page_off && t0 <= 508 - tb && r0 <= 512 - rbytes &&
                        r.th_off <= a.pages32 - tb && r.rad_off <= a.pages32 - rbytes;
    bad = bad || !sec_ok;
    n = sec_ok ? n : 0;
    thr = sec_ok ? t0 : 0;
    rdr = sec_ok ? r0 : 0;
  } else if (dense) {
    // an empty dense page (count 0, rad_off == th_off) is well formed
    const uint32_t kend = (uint32_t)r.th_off + (uint32_t)(n * DH * 2);
    const bool dense_ok = n == 0 || (t.dbase != kOOB && kend <= (uint32_t)r.rad_off && kend <= (uint32_t)a.pages32);
    bad = bad || !dense_ok;
    n = dense_ok ? n : 0;
  }
  t.desc = (comp ? tid : 0) | (int)dense << 2 | n << 3 | thr << 8 | rdr << 18 | (int)bad << 28;
  return __builtin_popcountll(__ballot(bad));
}

// 512-byte staging window [sbase, +512) of a page (sbase is 4-byte aligned):
// 8 bytes per lane (bytes past the pool read as zero); the page header is
// lane 0's first dword.
__device__ __forceinline__ uint2 load_stage(const Res& rs, const LaneOff& lo, int sbase) {
  const auto w = __builtin_amdgcn_raw_buffer_load_b64(rs.pages, (int)((uint32_t)sbase + lo.stg), 0, 0);
  return uint2{(uint32_t)w[0], (uint32_t)w[1]};
}

// Positions of row p's 16 tokens (lane t: token t's); none for a bad row.
__device__ __forceinline__ int load_pos(const Res& rs, const LaneOff& lo, int sbase, int p) {
  return __builtin_amdgcn_raw_buffer_load_b32(
      rs.pos, (int)(oob_or(sbase != kOOB, (uint32_t)p * (4u * kTile)) + lo.pos), 0, 0);
}

// V page layout, dim-major: element (token k, dim d) at half d * 16 + k.  Lane
// l loads dims l + 64 hf (hf < DH/64), 16 tokens = 32 bytes each: vreg[2hf]
// holds tokens 0..7, vreg[2hf + 1] tokens 8..15 -- the B operands of the
// 4x4x4 PV MFMA.  vsl < 0: nothing (zeros).
template <int DH>
__device__ __forceinline__ void load_v(const DecodeArgs& a, const LaneOff& lo, int vsl, half8 (&vreg)[DH / 32]) {
  // 64-bit element offset: vslot * DH * 16 exceeds 2^31 from vslot 2^20 (DH 128)
  const rsrc_t rs = make_rsrc(a.v_pool + (int64_t)max(vsl, 0) * (DH * kTile), vsl >= 0 ? DH * kTile * 2 : 0);
#pragma unroll
  for (int hf = 0; hf < DH / 64; ++hf)
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const auto w = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(lo.v + (64 * hf * kTile + 8 * k) * 2), 0, 0);
      vreg[2 * hf + k] = __builtin_bit_cast(half8, uint4{(uint32_t)w[0], (uint32_t)w[1], (uint32_t)w[2], (uint32_t)w[3]});
    }
}

// Dense K rows of a page (fp16 [n][DH] at dbase, 16-byte aligned): lane
// (t, u) loads chunks c = 0..NC-1 (dims chunk_dim(c, u) .. +8) of token t.
// Rows of tokens past the page's count read neighbouring bytes of the pool
// (or zeros past its end) and are not used.
template <int DH>
__device__ __forceinline__ void load_dense(const Res& rs, const LaneOff& lo, int dbase, uint4 (&kd)[DH / 32]) {
  constexpr int NC = DH / 32;
  const uint32_t base = (uint32_t)dbase + lo.kd;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const uint32_t d = (uint32_t)(chunk_dim<DH>(c, 0) - chunk_dim<DH>(0, 0)) * 2u;
    const auto w = __builtin_amdgcn_raw_buffer_load_b128(rs.pages, (int)(base + d), 0, 0);
    kd[c] = uint4{(uint32_t)w[0], (uint32_t)w[1], (uint32_t)w[2], (uint32_t)w[3]};
  }
}

// Waves per decode workgroup: 12 (3 per SIMD, up to 168 VGPRs each), enough
// to keep the per-lane offsets and addresses of the page loop in registers;
// 8 (2 per SIMD, 256 VGPRs) for GQA 8, whose two head sets double the QK
// operands and accumulators.
template <int GQA>
__host__ __device__ constexpr int decode_waves() { return GQA <= 4 ? 12 : 8; }
constexpr int kDelta = 96;             // delta-phasor table rows: |pos - page centre| < kDelta

__host__ __device__ constexpr int align16(int x) { return (x + 15) & ~15; }

// LDS of one decode workgroup (byte offsets).
//  * codebooks of the work item's kv head, fp32, [G][C][g + 4] per tier (rows
//    padded by 16 bytes so rows of random codes start in different banks);
//  * delta-phasor table, row d = |pos - page centre|: for each block of 4
//    RoPE frequencies j, 4 x cos(2 pi f_j d) then 4 x sin(2 pi f_j d), fp32,
//    rows padded by 16 bytes;
//  * f_j in turns per token (fp64);
//  * per wave: the staging area of its page (1 KB: the 512-byte window, and
//    room for the reads of tokens past the page's count), the query rows
//    rotated to the page centre (fp32, in the QK MFMA's operand order; slots
//    of heads >= GQA stay zero), and the page's softmax weights P as fp16
//    [max(GQA, 4)][16 tokens] (rows >= GQA stay zero), read back as the PV
//    MFMA's A operand.
template <int DH, int GQA>
struct DecodeLds {
  static constexpr int kWaves = decode_waves<GQA>();
  static constexpr int NJ = DH / 2;
  static constexpr int NPAIR = DH / 8;          // RoPE pairs (j, j + DH/2) per lane
  static constexpr int MQ = NPAIR / 4;          // float4 groups of pairs per lane
  __host__ __device__ static constexpr int cb_pad(int g) { return g + 4; }
  static constexpr int cb_n1 = (DH / 16) * 64 * 20;
  static constexpr int cb_n2 = (DH / 16) * 16 * 20;
  static constexpr int cb_n3 = (DH / 32) * 8 * 36;
  __host__ __device__ static constexpr int cb_off(int tid) {   // floats
    return tid == 3 ? cb_n1 + cb_n2 : (tid == 2 ? cb_n1 : 0);
  }
  static constexpr int drow = NJ * 8 + 16;                       // bytes
  static constexpr int o_cb = 0;
  static constexpr int o_dtab = align16(4 * (cb_n1 + cb_n2 + cb_n3));
  static constexpr int o_ftab = o_dtab + kDelta * drow;
  static constexpr int o_stage = o_ftab + NJ * 8;
  static constexpr int stage_bytes = 1024;
  static constexpr int PR = GQA < 4 ? 4 : GQA;                   // heads padded to 4 (slots)
  static constexpr int NHS = PR / 4;                             // sets of 4 head slots
  // rotated query, fp32, per set of 4 head slots: block (half hf, group m)
  // of 68 floats = [quarter u][slot][4 pairs e] + 4 padding floats, the
  // float4 of (u, slot) holding pairs 4m .. 4m + 3 of quarter u's RoPE
  // frequencies, first (hf = 0) or second (hf = 1) half.  The A-operand
  // reads (16 float4s of one block) and the per-frequency writes (one float
  // per lane, banks (4 m + e + 16 u) mod 64 distinct) are conflict-free.
  static constexpr int kQBlk = 68;
  static constexpr int qset = 2 * MQ * kQBlk;                    // floats per head-slot set
  static constexpr int o_qr = o_stage + kWaves * stage_bytes;
  static constexpr int qr_wave = NHS * qset * 4;                 // bytes per wave
  static constexpr int o_pt = o_qr + kWaves * qr_wave;
  static constexpr int total = o_pt + kWaves * PR * 32;
  // the end-of-item wave merge reuses the space: [kWaves][GQA][DH] acc,
  // [kWaves][GQA][2] (m, l)
  static constexpr int merge_bytes = kWaves * GQA * (DH + 2) * 4;
  static_assert(merge_bytes <= total, "merge buffer exceeds the workgroup's LDS");
  static_assert(total <= 160 * 1024, "LDS budget");
};

// This lane's two codebook groups (one per RoPE half) of token t on a staged
// compressed page (page byte 0 at st[0]; sections at thr / rdr): LDS byte
// offsets of the two centroid runs the lane needs, and the radii rc * scale
// (pagebuilder.py:17-21 without the 1/127 of the int8 code, which the page's
// logit scale carries).  Only tokens t < n use the results; the reads of the
// others stay inside the wave's 1 KB staging area.
template <int DH, int GQA, int TID>
__device__ __forceinline__ void locate_k(const uint8_t* st, int thr, int rdr, int t, int u, int (&cofs)[2],
                                         float (&rh)[2]) {
  constexpr int g = tier_g(TID), b = tier_b(TID), C = tier_C(TID);
  constexpr int G = DH / g;
  using L = DecodeLds<DH, GQA>;
  const int d0 = (DH / 8) * u;
  const int gi = d0 / g, off = d0 % g;                 // first-half group; its RoPE partner is gi + G/2
  // both codes lie in the 64 bits from the dword holding the first one
  // (token bits LSB first, bitpacking.py:5-29)
  const uint32_t bit = (uint32_t)(thr * 8 + t * (G * b) + gi * b);
  const uint32_t* wp = reinterpret_cast<const uint32_t*>(st) + ((bit >> 5) & 127);
  const uint32_t w = __builtin_amdgcn_alignbit(wp[1], wp[0], bit);
  const int c0 = (int)(w & (C - 1));
  const int c1 = (int)((w >> ((G / 2) * b)) & (C - 1));
  const int8_t* rp = reinterpret_cast<const int8_t*>(st + rdr + t * G + gi);
  const float* sp = reinterpret_cast<const float*>(st + kHeaderBytes) + gi;
  rh[0] = (float)rp[0] * sp[0];
  rh[1] = (float)rp[G / 2] * sp[G / 2];
  constexpr int row = L::cb_pad(g) * 4;                // bytes per padded centroid row
  cofs[0] = L::cb_off(TID) * 4 + (gi * C + c0) * row + off * 4;
  cofs[1] = L::cb_off(TID) * 4 + ((gi + G / 2) * C + c1) * row + off * 4;
}

// Partial of one work item: [16 floats: m[GQA], l[GQA], pad] [acc: GQA * DH]
template <int DH, int GQA>
__host__ __device__ constexpr int partial_stride() { return 16 + GQA * DH; }

// Work item of workgroup b.  Workgroups are dispatched to the 8 XCDs round
// robin (b mod 8); consecutive items belong to the same (sequence, kv head),
// so this mapping gives each XCD a contiguous block of items and its L2 the
// codebooks of few heads.
__device__ __forceinline__ int xcd_item(int b, int nb) {
  const int full = nb & ~7;
  if (b >= full) return b;
  return (b & 7) * (full >> 3) + (b >> 3);
}

constexpr double kInvTwoPi = 0.15915494309189535;      // 1 / (2 pi), rounded to fp64

// e^{i 2 pi x} with x a phase in turns (fp32 hardware sine/cosine take turns).
__device__ __forceinline__ float2 turn_phasor(double x) {
  const float ph = (float)__builtin_amdgcn_fract(x);
  return float2{__builtin_amdgcn_cosf(ph), __builtin_amdgcn_sinf(ph)};
}

// Rotation by N lanes within each 16-lane row (DPP row_ror).
template <int N>
__device__ __forceinline__ float row_ror(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x120 + N, 0xF, 0xF, true));
}

// Max / sum over the 16 lanes of each row (every lane gets its row's result).
__device__ __forceinline__ float row_max16(float x) {
  x = fmaxf(x, row_ror<8>(x));
  x = fmaxf(x, row_ror<4>(x));
  x = fmaxf(x, row_ror<2>(x));
  return fmaxf(x, row_ror<1>(x));
}
__device__ __forceinline__ float row_sum16(float x) {
  x += row_ror<8>(x);
  x += row_ror<4>(x);
  x += row_ror<2>(x);
  return x + row_ror<1>(x);
}

// Sums the four lane quarters' partials of a head set: element i of lane l
// holds head slot i of lane l's token summed over the dimensions of quarter
// l >> 4.  Two row-swap rounds pair the quarters and leave lane l with the
// full sum of head slot {0, 2, 1, 3}[l >> 4].
__device__ __forceinline__ float quarter_sum(floatx4 s) {
  float a0 = s[0], a1 = s[1], b0 = s[2], b1 = s[3];
  swap32(a0, a1);
  swap32(b0, b1);
  float a = a0 + a1, b = b0 + b1;
  swap16(a, b);
  return a + b;
}
__host__ __device__ constexpr int row_slot(int row) { return (0xD8 >> (2 * row)) & 3; }   // {0, 2, 1, 3}
__host__ __device__ constexpr int slot_row(int slot) { return (0xD8 >> (2 * slot)) & 3; }  // its inverse

__device__ __forceinline__ void set_prio(int lvl) {
  if (lvl >= 3) __builtin_amdgcn_s_setprio(3);
  else if (lvl == 2) __builtin_amdgcn_s_setprio(2);
  else if (lvl == 1) __builtin_amdgcn_s_setprio(1);
  else __builtin_amdgcn_s_setprio(0);
}

template <bool B> struct Flag { static constexpr bool value = B; };

// The step's new pre-RoPE key through the tier-3 codebook as one token
// (_encode_keys_with_codebooks on kn.unsqueeze(0), spherical_kv_pipeline.py:
// 2311-2313), bit-exact with torch CPU: N*g*C = 256 < 400 takes ATen's naive
// loop (multiply, then add, in order).  One wave; lane (eg = lane >> 3, ec =
// lane & 7) with eg < G3 (enc) holds group eg's 32 key values in x; crow
// points at centroid ec's row (registers or LDS).  The 32 divisions of a group are shared by its 8
// lanes (lane ec forms values 4 ec .. 4 ec + 3; each quotient is the same
// correctly rounded one whichever lane forms it) and exchanged through LDS
// (dirs [G3][32], sims [G3][8]).  Lanes with ec == 0 return the group's
// radius and first-maximum code (torch.argmax: the ascending scan with '>').
__device__ __forceinline__ void encode_new_token(float (&x)[32], const float* crow, int eg, int ec, bool enc,
                                                 bool fp16_in, float (*dirs)[32], float (*sims)[8], float& r_out,
                                                 int& code_out) {
  float r_enc = 0.f;
  if (enc) {
    r_enc = torch_norm(x, 32);
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = x[e];
#pragma unroll
      for (int k = 1; k < 8; ++k) v[e] = ec == k ? x[4 * k + e] : v[e];
    }
    group_directions<4>(v, __fadd_rn(r_enc, 1e-8f), fp16_in, v);
    *reinterpret_cast<float4*>(&dirs[eg][4 * ec]) = float4{v[0], v[1], v[2], v[3]};
  }
  wave_lds_sync();
  if (enc) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float4 d4 = *reinterpret_cast<const float4*>(&dirs[eg][4 * k]);
      x[4 * k] = d4.x; x[4 * k + 1] = d4.y; x[4 * k + 2] = d4.z; x[4 * k + 3] = d4.w;
    }
    float sm = 0.f;
#pragma unroll
    for (int k = 0; k < 32; ++k) sm = __fadd_rn(sm, __fmul_rn(x[k], crow[k]));
    sims[eg][ec] = sm;
  }
  wave_lds_sync();
  int best = 0;
  if (enc && ec == 0) {
    float bs = sims[eg][0];
#pragma unroll
    for (int k = 1; k < 8; ++k)
      if (sims[eg][k] > bs) { bs = sims[eg][k]; best = k; }
  }
  r_out = r_enc;
  code_out = best;
}


template <int DH, int GQA>
__global__ __launch_bounds__(decode_waves<GQA>() * 64)
__attribute__((amdgpu_waves_per_eu(decode_waves<GQA>() / 4, decode_waves<GQA>() / 4))) void decode_kernel(
    const int32_t* __restrict__ work, int32_t num_items, DecodeArgs a) {
  // work and num_items lead the argument list: the build preloads the first
  // kernel-argument dwords into SGPRs, so the work item's load is issued at
  // wave start instead of after two dependent argument loads
  constexpr int kWaves = decode_waves<GQA>();
  constexpr int NC = DH / 32;        // 8-dim chunks of dense K per lane-token
  constexpr int NJ = DH / 2;         // RoPE frequencies
  using L = DecodeLds<DH, GQA>;
  constexpr int NPAIR = L::NPAIR, MQ = L::MQ;
  __shared__ __attribute__((aligned(16))) uint8_t smem[L::total];
  float* cb_s = reinterpret_cast<float*>(smem + L::o_cb);
  const uint8_t* dtab = smem + L::o_dtab;
  double* ftab = reinterpret_cast<double*>(smem + L::o_ftab);

  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int item = xcd_item(blockIdx.x, num_items);
  // the work list comes from the caller: an item naming no (seq, head) is
  // empty, rows are clamped to the table and the stride to [1, num_rows]
  // (so no row index below overflows and the page loop is bounded)
  // One 16-byte scalar load of the item and branch-free clamps: a load or a
  // division under a condition becomes a branch, and every kernel-argument
  // load after it then waits for the item first (serial round trips).
  const int4 wi = *reinterpret_cast<const int4*>(work + 4 * item);
  const bool item_ok = wi.x >= 0 && wi.x < a.num_sh;
  const int sh = item_ok ? wi.x : 0;
  const int rb = max(wi.y, 0);
  const int re = item_ok ? min(wi.z, a.num_rows) : 0;
  const int rstride = min(max(wi.w, 1), max(a.num_rows, 1));   // rows between consecutive pages of the item
  const int wstride = kWaves * rstride;                // rows between consecutive pages of a wave
  // pages of this wave (rows rb + rstride (wave + kWaves k) < re)
  const int npg = (max(re - rb, 0) + rstride - 1) / rstride;
  const int nwp = max(npg - wave + kWaves - 1, 0) / kWaves;
  const int h = sh % a.num_kv;
  const int seq = sh / a.num_kv;
  const int t = lane & 15;
  const int u = lane >> 4;
  uint8_t* st = smem + L::o_stage + wave * L::stage_bytes;
  float* qr = reinterpret_cast<float*>(smem + L::o_qr + wave * L::qr_wave);
  _Float16* pt = reinterpret_cast<_Float16*>(smem + L::o_pt) + wave * L::PR * kTile;
  const LaneOff lo = lane_offsets<DH>(lane);

  const int p0 = rb + wave * rstride;                   // row of the wave's first page
  const Res rs = make_res(a);
  // ---- pointer-table rows of the wave's first 64 pages (one page per
  //      lane), then the shared tables' loads -----------------------------
  const PageRows rows0 = rows_issue(rs, p0, wstride, 0, nwp, lane);
  // codebooks: every load of a thread is issued before its first LDS store
  constexpr int kT = kWaves * 64;
  constexpr int n4_1 = L::cb_n1 / 20 * 4, n4_2 = L::cb_n2 / 20 * 4, n4_3 = L::cb_n3 / 36 * 8;  // float4s
  constexpr int k1 = (n4_1 + kT - 1) / kT, k2 = (n4_2 + kT - 1) / kT, k3 = (n4_3 + kT - 1) / kT;
  floatx4 cbv[k1 + k2 + k3];
  {
    int slot = 0;
#pragma unroll
    for (int tid = 1; tid <= 3; ++tid) {
      const int g = tier_g(tid), rows = (DH / g) * tier_C(tid);
      const int nf4 = rows * g / 4;
      const rsrc_t rs = make_rsrc(a.cb[tid] ? a.cb[tid] + (int64_t)h * rows * g : nullptr, a.cb[tid] ? nf4 * 16 : 0);
      const int kk = tid == 1 ? k1 : (tid == 2 ? k2 : k3);
#pragma unroll
      for (int k = 0; k < kk; ++k) {
        const int i = threadIdx.x + k * kT;
        cbv[slot++] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rs, i < nf4 ? 16 * i : kOOB, 0, 0));
      }
    }
  }
  // this lane's query pair (j, j + NJ) of every head of the item, fp32
  float qf[GQA][2];
  {
    const _Float16* qh = a.q + ((int64_t)seq * a.num_kv * GQA + (int64_t)h * GQA) * DH;
    const int j = lane % NJ;
#pragma unroll
    for (int hh = 0; hh < GQA; ++hh) {
      qf[hh][0] = (float)qh[hh * DH + j];
      qf[hh][1] = (float)qh[hh * DH + j + NJ];
    }
  }
  // This lane's RoPE frequency f_j (j = lane mod NJ) in turns per token.  A
  // workgroup has a multiple of NJ threads, so the delta-table entries
  // (d, j) = i, i = threadIdx.x + k * kT, of a thread all have its own j: the
  // table is built from registers while the first loads are in flight.
  const double f_lane = exp2(-(2.0 * (lane % NJ) / DH) * a.log2_theta) * kInvTwoPi;  // / (2 pi)
  static_assert((kWaves * 64) % NJ == 0, "delta-table rows need whole frequency runs per thread");
  if (wave == 0 && lane < NJ) ftab[lane] = f_lane;       // the far pages' phasors read it
  for (int i = threadIdx.x; i < kDelta * NJ; i += kT) {
    const int d = i / NJ, j = i % NJ;
    const float2 z = turn_phasor((double)d * f_lane);
    float* row = reinterpret_cast<float*>(const_cast<uint8_t*>(dtab) + d * L::drow) + (j >> 2) * 8;
    row[j & 3] = z.x;
    row[4 + (j & 3)] = z.y;
  }
  // row checks; the pages' header loads and the first page's staging window,
  // positions, V and dense K are issued as soon as the rows are in, so the
  // page data streams in while the codebooks are stored
  PageTab T = page_bases<DH>(a, rows0, 0, nwp, lane);
  const int hdr0 = header_issue(rs, T);
  uint2 stg_c, stg_b;
  int pos_c, pos_b;
  half8 vreg[DH / 32];
  uint4 kd[NC];
  {
    const int sb = __builtin_amdgcn_readfirstlane(T.sbase);
    stg_c = load_stage(rs, lo, sb);
    pos_c = load_pos(rs, lo, sb, p0);
    load_v<DH>(a, lo, __builtin_amdgcn_readfirstlane(T.vsl), vreg);
    const int db = __builtin_amdgcn_readfirstlane(T.dbase);
    if (db != kOOB) load_dense<DH>(rs, lo, db, kd);
  }
  if (GQA < 4) {
    // zero P rows GQA..3 and the query slots GQA..3 of this wave (never written)
    if (lane < (4 - GQA) * 2) {
      half8 z;
      for (int e = 0; e < 8; ++e) z[e] = (_Float16)0.f;
      *reinterpret_cast<half8*>(pt + GQA * kTile + 8 * lane) = z;
    }
    for (int i = lane; i < 2 * MQ * 16; i += 64)          // i = (block, u, slot)
      if ((i & 3) >= GQA) *reinterpret_cast<floatx4*>(qr + (i >> 4) * L::kQBlk + 4 * (i & 15)) = (floatx4){0.f, 0.f, 0.f, 0.f};
  }
  {
    int slot = 0;
#pragma unroll
    for (int tid = 1; tid <= 3; ++tid) {
      const int g = tier_g(tid), gp = L::cb_pad(g), rows = (DH / g) * tier_C(tid);
      const int nf4 = rows * g / 4;
      float* dst = cb_s + L::cb_off(tid);
      const int kk = tid == 1 ? k1 : (tid == 2 ? k2 : k3);
#pragma unroll
      for (int k = 0; k < kk; ++k) {
        const int i = threadIdx.x + k * kT;
        if (i < nf4) *reinterpret_cast<floatx4*>(dst + ((4 * i) / g) * gp + (4 * i) % g) = cbv[slot];
        ++slot;
      }
    }
  }
  __syncthreads();
  // the header checks wait for this wave's header loads only (after the
  // barrier, so no wave waits for another's)
  int nbad = page_check<DH>(a, rows0, T, hdr0, 0, nwp, lane);   // malformed rows / pages of this wave

  // Loop-invariant lane data: LDS addresses of this lane's query writes /
  // reads and P write / read.
  float* qw;
  {
    const int j = lane % NJ, s = j % NPAIR;
    qw = qr + (s >> 2) * L::kQBlk + (j / NPAIR) * 16 + (s & 3);
  }
  const float* qb = qr + u * 16 + (lane & 3) * 4;

  // Online-softmax state.  After a page's quarter sums, lane (row r, token t)
  // holds the logit of head 4 hs + row_slot(r) for token t; the running
  // reference max m_run of that head is the same in all 16 lanes of the row,
  // and l_part is this lane's share (token slot t) of the head's sum of
  // weights, reduced over the row once the item is done.
  constexpr int NHS = L::NHS, NHF = DH / 64;
  const int hr = row_slot(u);
  float m_run[NHS], l_part[NHS];
#pragma unroll
  for (int hs = 0; hs < NHS; ++hs) { m_run[hs] = -INFINITY; l_part[hs] = 0.f; }
  // PV accumulators of the 4x4x4 MFMA: acc[hs][hf] lane l, element i =
  // O[head 4 hs + i][dim 64 hf + l]
  floatx4 acc[NHS][NHF];
#pragma unroll
  for (int hs = 0; hs < NHS; ++hs)
#pragma unroll
    for (int hf = 0; hf < NHF; ++hf) acc[hs][hf] = (floatx4){0.f, 0.f, 0.f, 0.f};

  int prio_next = 0;                                    // page index at which the priority changes
  // issue priority of the wave's page d from its share of pages still to do:
  // a SIMD serves its waves oldest first, so without it the youngest wave
  // would finish last, alone on its SIMD
  auto prio_of = [&](int d) {
    const int left = nwp - d;                           // pages left, page d included
    return 4 * left > 3 * nwp ? 3 : (2 * left > nwp ? 2 : (4 * left > nwp ? 1 : 0));
  };
  // Page k of the pipeline.  The staging window and positions of the next
  // page are loaded into the other register set of a pair, so the loop
  // (unrolled by two) never copies a register that a load is still filling:
  // such a copy would wait for that load.
  auto step = [&](const int k, uint2& stg_c, int& pos_c, uint2& stg_n, int& pos_n) __attribute__((always_inline)) {
    // ---- issue priority (changes at most three times per item) ----------
    if (k == prio_next) {
      const int lvl = prio_of(k);
      set_prio(lvl);
      int d = k + 1;
      while (d < nwp && prio_of(d) == lvl) ++d;
      prio_next = d;
    }
    // ---- this page's descriptor; the last page of 64 loads and checks the
    //      next 64 pages' table (a wait for two loads, once per 64 pages) ---
    const int kl = k & 63;
    const int desc = __builtin_amdgcn_readlane(T.desc, kl);
    if (kl == 63 && k + 1 < nwp) {
      const PageRows rw = rows_issue(rs, p0, wstride, k + 1, nwp, lane);
      T = page_bases<DH>(a, rw, k + 1, nwp, lane);
      nbad += page_check<DH>(a, rw, T, header_issue(rs, T), k + 1, nwp, lane);
    }
    const int kn = (k + 1) & 63;
    // ---- issue: stage / positions one page ahead ------------------------
    {
      const int sb = __builtin_amdgcn_readlane(T.sbase, kn);
      stg_n = load_stage(rs, lo, sb);
      pos_n = load_pos(rs, lo, sb, p0 + (k + 1) * wstride);
    }
    const int tid = desc & 3;                   // compressed tier (0: not compressed)
    const int comp = (int)(tid != 0);
    const int dense = (desc >> 2) & 1;
    const int n = (desc >> 3) & 31;             // tokens to use
    const int thr = (desc >> 8) & 1023, rdr = (desc >> 18) & 1023;   // section offsets from the page start
    const bool valid = (t < n) && (pos_c >= 0);

    // ---- page centre t_mid; query rows rotated by -t_mid into LDS ---------
    //      <q, R(pos) k> = <R(-t_mid) q, R(pos - t_mid) k>
    {
      const int t_lo = __builtin_amdgcn_readlane(pos_c, 0);
      const int t_hi = __builtin_amdgcn_readlane(pos_c, n > 0 ? n - 1 : 0);
      const int t_mid = (t_lo >= 0 && t_hi >= 0) ? t_lo + ((t_hi - t_lo) >> 1) : max(t_lo, 0);
      // lane = frequency j (lanes j and j + NJ write the same values when NJ = 32)
      const float2 z = turn_phasor((double)t_mid * f_lane);
#pragma unroll
      for (int hh = 0; hh < GQA; ++hh) {
        const int o = (hh >> 2) * L::qset + (hh & 3) * 4;
        qw[o] = qf[hh][0] * z.x + qf[hh][1] * z.y;
        qw[o + MQ * L::kQBlk] = qf[hh][1] * z.x - qf[hh][0] * z.y;
      }
      // offset of this lane's token from the centre
      pos_c = valid ? pos_c - t_mid : 0;
    }
    const int dl = pos_c;

    // ---- locate this page's keys: centroid offsets + radii (compressed) ---
    int cofs[2] = {0, 0};
    float rh[2] = {1.f, 1.f};                   // dense K enters unscaled
    if (comp) {
      *reinterpret_cast<uint2*>(st + 8 * lane) = stg_c;
      wave_lds_sync();
      if (tid == 1) locate_k<DH, GQA, 1>(st, thr, rdr, t, u, cofs, rh);
      else if (tid == 2) locate_k<DH, GQA, 2>(st, thr, rdr, t, u, cofs, rh);
      else locate_k<DH, GQA, 3>(st, thr, rdr, t, u, cofs, rh);
    }
    wave_lds_sync();

    // ---- QK.  k_hat = (r1 c1, r2 c2) on the lane's pairs (j, j + DH/2) (c1,
    //      c2 the centroid runs of the two codebook groups, or the dense K
    //      halves with r1 = r2 = 1), d = pos - t_mid, cs = cos(2 pi f_j |d|),
    //      sn = sin(2 pi f_j |d|), sg = sign d, q_c = R(-t_mid) q.  With k1 =
    //      r1 c1 and k2 = sg r2 c2 (dense: sg K2),
    //        x0 = k1 cs - k2 sn,  x1' = k2 cs + k1 sn,
    //      R(d) k_hat = (x0, sg x1'), so <q_c, R(d) k_hat> = sum q0 x0 + sg sum q1 x1'.
    //      Both sums run on the fp32 MFMA (4x4x1, 16 blocks = 4 lane quarters
    //      x 4 token groups; A = the rotated query of head slot i (row), B =
    //      x0 or x1' of the lane's own token (column), one pair per
    //      instruction), so every lane's accumulators hold its own token's
    //      sums for head slots 0..3 and sg applies per lane afterwards.
    //      Phasors come from the LDS delta table; a page with a lane at
    //      |d| >= kDelta forms every lane's phasors directly.
    const int ad = dl < 0 ? -dl : dl;
    const bool any_far = __ballot(ad >= kDelta) != 0;
    const float sg = dl < 0 ? -1.f : 1.f;
    const float r1 = rh[0], r2 = sg * rh[1];
    const uint32_t kneg = dl < 0 ? 0x80008000u : 0u;  // dense: sg applied to K2's fp16 sign bits
    const float* drw = reinterpret_cast<const float*>(dtab + (any_far ? 0 : ad) * L::drow) + 2 * NPAIR * u;
    floatx4 qk[NHS][2];
#pragma unroll
    for (int hs = 0; hs < NHS; ++hs) { qk[hs][0] = (floatx4){0.f, 0.f, 0.f, 0.f}; qk[hs][1] = qk[hs][0]; }
    auto kpath = [&](auto far_f, auto dense_f) __attribute__((always_inline)) {
      constexpr bool FAR = decltype(far_f)::value, DENSE = decltype(dense_f)::value;
#pragma unroll
      for (int m = 0; m < MQ; ++m) {
        float k1[4], k2[4];                      // k1 = r1 c1, k2 = sg r2 c2 on pairs 4m .. 4m + 3
        if constexpr (DENSE) {
          const uint4 w0 = kd[m >> 1], w1 = kd[NC / 2 + (m >> 1)];
          const uint32_t a0 = (m & 1) ? w0.z : w0.x, a1 = (m & 1) ? w0.w : w0.y;
          const uint32_t b0 = ((m & 1) ? w1.z : w1.x) ^ kneg, b1 = ((m & 1) ? w1.w : w1.y) ^ kneg;
          const half2v ha0 = __builtin_bit_cast(half2v, a0), ha1 = __builtin_bit_cast(half2v, a1);
          const half2v hb0 = __builtin_bit_cast(half2v, b0), hb1 = __builtin_bit_cast(half2v, b1);
          k1[0] = (float)ha0[0]; k1[1] = (float)ha0[1]; k1[2] = (float)ha1[0]; k1[3] = (float)ha1[1];
          k2[0] = (float)hb0[0]; k2[1] = (float)hb0[1]; k2[2] = (float)hb1[0]; k2[3] = (float)hb1[1];
        } else {
          const float4 c0 = *reinterpret_cast<const float4*>(smem + cofs[0] + 16 * m);
          const float4 c1 = *reinterpret_cast<const float4*>(smem + cofs[1] + 16 * m);
          k1[0] = r1 * c0.x; k1[1] = r1 * c0.y; k1[2] = r1 * c0.z; k1[3] = r1 * c0.w;
          k2[0] = r2 * c1.x; k2[1] = r2 * c1.y; k2[2] = r2 * c1.z; k2[3] = r2 * c1.w;
        }
        float pc[4], ps[4];
        if constexpr (FAR) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float2 z = turn_phasor((double)ad * ftab[NPAIR * u + 4 * m + e]);
            pc[e] = z.x;
            ps[e] = z.y;
          }
        } else {
          const float4 c03 = *reinterpret_cast<const float4*>(drw + 8 * m);
          const float4 s03 = *reinterpret_cast<const float4*>(drw + 8 * m + 4);
          pc[0] = c03.x; pc[1] = c03.y; pc[2] = c03.z; pc[3] = c03.w;
          ps[0] = s03.x; ps[1] = s03.y; ps[2] = s03.z; ps[3] = s03.w;
        }
        floatx4 q0[NHS], q1[NHS];
#pragma unroll
        for (int hs = 0; hs < NHS; ++hs) {
          q0[hs] = *reinterpret_cast<const floatx4*>(qb + hs * L::qset + m * L::kQBlk);
          q1[hs] = *reinterpret_cast<const floatx4*>(qb + hs * L::qset + (MQ + m) * L::kQBlk);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x0 = k1[e] * pc[e] - k2[e] * ps[e];
          const float x1 = k2[e] * pc[e] + k1[e] * ps[e];
#pragma unroll
          for (int hs = 0; hs < NHS; ++hs) {
            qk[hs][0] = __builtin_amdgcn_mfma_f32_4x4x1f32(q0[hs][e], x0, qk[hs][0], 0, 0, 0);
            qk[hs][1] = __builtin_amdgcn_mfma_f32_4x4x1f32(q1[hs][e], x1, qk[hs][1], 0, 0, 0);
          }
        }
      }
    };
    if (!any_far) {
      if (dense) kpath(Flag<false>(), Flag<true>());
      else kpath(Flag<false>(), Flag<false>());
    } else {
      if (dense) kpath(Flag<true>(), Flag<true>());
      else kpath(Flag<true>(), Flag<false>());
    }

    // ---- logits and online softmax in the log2 domain: lane (row r, token
    //      t) ends with head 4 hs + row_slot(r)'s logit of token t ----------
    const float scale = dense ? a.scale_log2 : a.scale_log2_c;
    float x[NHS];
    bool exceed = false;
#pragma unroll
    for (int hs = 0; hs < NHS; ++hs) {
      floatx4 s;
#pragma unroll
      for (int i = 0; i < 4; ++i) s[i] = sg * qk[hs][1][i] + qk[hs][0][i];
      const float lg = quarter_sum(s);            // the cross-lane sum runs on every lane
      x[hs] = (valid && 4 * hs + hr < GQA) ? lg * scale : -INFINITY;
      exceed |= x[hs] > m_run[hs] + kRescaleLog2;
    }
    // The running reference max of a head moves only when one of its logits
    // exceeds it by more than 2^8, so p = 2^(x - m) <= 256 stays finite in
    // fp16; the max over the row is taken only then.
    if (__ballot(exceed) != 0) {
      float alpha[NHS];
#pragma unroll
      for (int hs = 0; hs < NHS; ++hs) {
        const float mx = row_max16(x[hs]);
        const float m_new = mx > m_run[hs] + kRescaleLog2 ? mx : m_run[hs];
        alpha[hs] = m_new == m_run[hs] ? 1.f : __builtin_amdgcn_exp2f(m_run[hs] - m_new);
        l_part[hs] *= alpha[hs];
        m_run[hs] = m_new;
      }
      // head slot i's factor lives in row slot_row(i); accumulators hold
      // head slot i in element i
#pragma unroll
      for (int hs = 0; hs < NHS; ++hs)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float f = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha[hs]),
                                                                            16 * slot_row(i)));
#pragma unroll
          for (int hf = 0; hf < NHF; ++hf) acc[hs][hf][i] *= f;
        }
    }
    // p rounded to fp16 for the PV MFMA, and the same rounded p summed into
    // l, so the output stays an exact convex combination of V rows
#pragma unroll
    for (int hs = 0; hs < NHS; ++hs) {
      const _Float16 ph = (_Float16)(x[hs] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(x[hs] - m_run[hs]));
      l_part[hs] += (float)ph;
      if (4 * hs + hr < GQA) pt[(4 * hs + hr) * kTile + t] = ph;
    }

    // ---- O += P V on the 4x4x4 MFMA (16 blocks = 16 groups of 4 dims):
    //      A = P[4 heads][4 tokens] (same for every block, from LDS),
    //      B = V[4 tokens][dim 64 hf + l] (lane l's own dim) -----------------
    // slots without a token get V = 0 (their p is already 0; this keeps
    // whatever bytes an unused slot holds out of the sum)
    const uint32_t vmask = (uint32_t)__ballot(valid) & 0xFFFFu;
    if (vmask != 0xFFFFu) {
#pragma unroll
      for (int v = 0; v < DH / 32; ++v)
#pragma unroll
        for (int e = 0; e < 8; ++e)
          vreg[v][e] = ((vmask >> (8 * (v & 1) + e)) & 1u) ? vreg[v][e] : (_Float16)0.f;
    }
    wave_lds_sync();
#pragma unroll
    for (int hs = 0; hs < NHS; ++hs) {
      const half8* prow = reinterpret_cast<const half8*>(pt + (4 * hs + (lane & 3)) * kTile);
      const half8 p0 = prow[0], p1 = prow[1];
#pragma unroll
      for (int tg = 0; tg < 4; ++tg) {
        const half8 pp = tg < 2 ? p0 : p1;
        const half4 pa4 = (tg & 1) ? half4{pp[4], pp[5], pp[6], pp[7]} : half4{pp[0], pp[1], pp[2], pp[3]};
#pragma unroll
        for (int hf = 0; hf < NHF; ++hf) {
          const half8 vv = vreg[2 * hf + (tg >> 1)];
          const half4 vb = (tg & 1) ? half4{vv[4], vv[5], vv[6], vv[7]} : half4{vv[0], vv[1], vv[2], vv[3]};
          acc[hs][hf] = __builtin_amdgcn_mfma_f32_4x4x4f16(pa4, vb, acc[hs][hf], 0, 0, 0);
        }
      }
    }

    // ---- issue V / dense K of the next page into the freed registers ------
    //      (their lane offsets are recomputed: a few VALU ops instead of two
    //      registers held across the page)
    {
      int lane_v = lane;
      asm volatile("" : "+v"(lane_v));
      const LaneOff lv = lane_offsets<DH>(lane_v);
      load_v<DH>(a, lv, __builtin_amdgcn_readlane(T.vsl, kn), vreg);
      const int db = __builtin_amdgcn_readlane(T.dbase, kn);
      if (db != kOOB) load_dense<DH>(rs, lv, db, kd);
    }
    wave_lds_sync();
  };
  for (int k = 0; k < nwp; k += 2) {
    step(k, stg_c, pos_c, stg_b, pos_b);
    if (k + 1 >= nwp) break;
    step(k + 1, stg_b, pos_b, stg_c, pos_c);
  }

  __builtin_amdgcn_s_setprio(0);
  if (nbad != 0 && lane == 0) __hip_atomic_fetch_add(a.status, (uint32_t)nbad, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  float l_run[NHS];
#pragma unroll
  for (int hs = 0; hs < NHS; ++hs) l_run[hs] = row_sum16(l_part[hs]);
  // ---- merge the waves' states in LDS, write this item's partial ----------
  constexpr int PS = partial_stride<DH, GQA>();
  __syncthreads();
  float* mrg = reinterpret_cast<float*>(smem);        // [kWaves][GQA][DH]
  float* mrg_ml = mrg + kWaves * GQA * DH;            // [kWaves][GQA][2]
#pragma unroll
  for (int hs = 0; hs < NHS; ++hs)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (4 * hs + i < GQA)
#pragma unroll
        for (int hf = 0; hf < NHF; ++hf) mrg[(wave * GQA + 4 * hs + i) * DH + 64 * hf + lane] = acc[hs][hf][i];
#pragma unroll
  for (int hs = 0; hs < NHS; ++hs)
    if (t == 0 && 4 * hs + hr < GQA) {
      mrg_ml[(wave * GQA + 4 * hs + hr) * 2] = m_run[hs];
      mrg_ml[(wave * GQA + 4 * hs + hr) * 2 + 1] = l_run[hs];
    }
  __syncthreads();
  // every output thread derives its head's wave weights 2^(m_w - M) itself
  // (the kWaves reads of a head hit one LDS address each: broadcasts), so
  // the merge is one LDS round trip instead of a serial pass per head
  float* part = a.partials + (int64_t)item * PS;
  for (int i = threadIdx.x; i < GQA * DH; i += kWaves * 64) {
    const int hh = i / DH, d = i % DH;
    float mw[kWaves];
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      mw[w] = mrg_ml[(w * GQA + hh) * 2];
      M = fmaxf(M, mw[w]);
    }
    float A = 0.f, Ls = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = (mw[w] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(mw[w] - M);
      A += f * mrg[(w * GQA + hh) * DH + d];
      Ls += f * mrg_ml[(w * GQA + hh) * 2 + 1];
    }
    part[16 + hh * DH + d] = A;
    if (d == 0) {
      part[hh] = M;
      part[GQA + hh] = Ls;
    }
  }
}

// Log-sum-exp merge of the partials of each (sequence, kv head).  One
// workgroup per (sequence, kv head, slice of up to 128 floats of its GQA*DH
// output); thread = (item lane il, float4 column c).  Each thread keeps its
// own running (max, sum, weighted acc) over its items, so all of a thread's
// loads are independent and a merge over <= 32 items costs one memory round
// trip after the work_start read; the 8 item lanes are combined in LDS.
template <int DH, int GQA>
__global__ __launch_bounds__(256) void decode_merge_kernel(const float* __restrict__ partials,
                                                           const int32_t* __restrict__ work_start,
                                                           int32_t num_items, int32_t num_kv,
                                                           _Float16* __restrict__ out, uint32_t* status) {
  constexpr int PS = partial_stride<DH, GQA>();
  constexpr int SL = GQA * DH < 128 ? GQA * DH : 128; // floats per output slice
  constexpr int NSL = (GQA * DH) / SL;                // slices per (seq, kv head)
  constexpr int IL = 8;                               // item lanes: 256 threads = 8 x 32 float4 columns
  constexpr int UN = 4;                               // items per item lane per round trip
  __shared__ float4 red_v[IL][32];
  __shared__ float red_m[IL][32], red_l[IL][32];
  const int sh = blockIdx.x / NSL, slice = blockIdx.x % NSL;
  // the malformed-page count of the decode calls since the last merge becomes
  // this merge's result, and the counter restarts (stream order: every
  // decode workgroup has finished)
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    status[1] = status[0];
    status[0] = 0u;
  }
  // item range of this (seq, head), clamped to the partials that exist
  const int ib = min(max(work_start[sh], 0), num_items);
  const int ni = min(max(work_start[sh + 1], ib), num_items) - ib;
  const int c = threadIdx.x & 31, il = threadIdx.x >> 5;
  const bool col_ok = 4 * c < SL;
  const int f0 = slice * SL + (col_ok ? 4 * c : 0);   // first float of this column in [GQA*DH]
  const int hh = f0 / DH;
  float M = -INFINITY, Ls = 0.f;
  float4 sum = {0.f, 0.f, 0.f, 0.f};
  for (int it0 = il; it0 < ni; it0 += IL * UN) {
    float4 v[UN];
    float mi[UN], li[UN];
#pragma unroll
    for (int k = 0; k < UN; ++k) {
      const int it = it0 + k * IL;
      const float* pp = partials + (int64_t)(ib + (it < ni ? it : 0)) * PS;
      mi[k] = it < ni ? pp[hh] : -INFINITY;
      li[k] = pp[GQA + hh];
      v[k] = *reinterpret_cast<const float4*>(pp + 16 + f0);
    }
    float Mn = M;
#pragma unroll
    for (int k = 0; k < UN; ++k) Mn = fmaxf(Mn, mi[k]);
    if (Mn == -INFINITY) continue;
    const float r = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M - Mn);
    sum.x *= r; sum.y *= r; sum.z *= r; sum.w *= r;
    Ls *= r;
#pragma unroll
    for (int k = 0; k < UN; ++k) {
      const float f = (mi[k] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(mi[k] - Mn);
      Ls += f * li[k];
      sum.x += f * v[k].x; sum.y += f * v[k].y; sum.z += f * v[k].z; sum.w += f * v[k].w;
    }
    M = Mn;
  }
  red_v[il][c] = sum;
  red_m[il][c] = M;
  red_l[il][c] = Ls;
  __syncthreads();
  if (il == 0 && col_ok) {
    float Mx = -INFINITY;
    for (int k = 0; k < IL; ++k) Mx = fmaxf(Mx, red_m[k][c]);
    float4 tot = {0.f, 0.f, 0.f, 0.f};
    float Lt = 0.f;
    if (Mx != -INFINITY)
      for (int k = 0; k < IL; ++k) {
        const float mk = red_m[k][c];
        if (mk == -INFINITY) continue;
        const float f = __builtin_amdgcn_exp2f(mk - Mx);
        const float4 x = red_v[k][c];
        tot.x += f * x.x; tot.y += f * x.y; tot.z += f * x.z; tot.w += f * x.w;
        Lt += f * red_l[k][c];
      }
    const float inv = Lt > 0.f ? 1.f / Lt : 0.f;
    half4 o;
    o[0] = (_Float16)(tot.x * inv); o[1] = (_Float16)(tot.y * inv);
    o[2] = (_Float16)(tot.z * inv); o[3] = (_Float16)(tot.w * inv);
    const int seq = sh / num_kv, h = sh % num_kv;
    *reinterpret_cast<half4*>(out + ((int64_t)seq * num_kv * GQA + (int64_t)h * GQA) * DH + f0) = o;
  }
}

// ---------------------------------------------------------------------------
// Decode-time tail of the Mode-B step (spherical_kv_pipeline.py:2248-2342,
// 2389-2475).  One 256-thread workgroup per (sequence, kv head) sh and slice
// of up to 128 floats of its GQA*DH output (the slice's q heads' tail logits,
// the log-sum-exp of the slice's columns); slice 0 also appends.  The tail
// counts come in two copies: a step reads copy `parity` and an appending
// step writes the other, so the slices of one sh never see each other's
// update.
//
//   * The step's new pre-RoPE key is encoded through the tier-3 codebook as
//     one token (_encode_keys_with_codebooks on kn.unsqueeze(0), :2311-2313):
//     fp32 radius and first-max code per 32-dim group, bit-exact with torch
//     CPU (N*g*C = 256 < 400: ATen's naive loop, a multiply-then-add chain).
//   * Decode (kTailDecode): the staged tokens (their fp32 radii, :2248-2285)
//     and the new token at current_pos (:2315-2342) are scored with
//     logit = sum_g r_g <q, R(pos) c_g> / sqrt(dh) (= the back-rotated query's
//     form with the unit centroids), folded with the work items' partials into
//     one log-sum-exp (the softmax over context + tail, :2347-2348) and
//     attn @ V (:2364-2367, V of the new token = v_new).  Tail weights stay
//     fp32.
//   * Append (kTailAppend, _append_decode_kv :2389-2448): the new token goes
//     to staging slot n (radii, codes, V, position); when that fills the page
//     (n = 15) the 16 tokens become a tier-3 pagebuilder page
//     (_flush_decode_page :2449-2475, build_page_from_codes: max-radius
//     scales, int8 radius codes, LSB-first 3-bit codes) in sh's next decode
//     slot, with its positions row and dim-major V page, the work items of sh
//     take the new row (their end_row grows by one: the decode-time pointer
//     table keeps dec_cap reserved rows right after each (seq, head)'s rows,
//     their pointer-table rows and V slots set up front), and staging
//     restarts empty.
// Slots: waves 0..2 score the staged tokens (slot w < n), wave 3 encodes
// and scores the new token (slot 15).
struct TailArgs {
  const void* k_new;        // [num_sh, DH] pre-RoPE, fp16 or fp32 (k_is_fp32)
  const _Float16* v_new;    // [num_sh, DH]
  const int32_t* cur_pos;   // [num_seqs]
  float* stg_r;             // [num_sh, 16, DH/32]
  int32_t* stg_code;        // [num_sh, 16, DH/32]
  _Float16* stg_v;          // [num_sh, 16, DH]
  int32_t* stg_pos;         // [num_sh, 16]
  int32_t* state;           // [num_sh, 2, 4]: two copies of (staged count, decode pages, dropped tokens, 0)
  uint8_t* pages;
  int32_t* positions;
  _Float16* v_pool;
  int32_t* work;            // [num_items, 4]: end_row of sh's items grows at a flush
  int64_t dec_byte0;
  int32_t dec_cap, dec_vpage0, k_is_fp32, mode, num_items, num_rows, parity;
};

constexpr int kTailThreads = 256;

template <int DH, int GQA>
__global__ __launch_bounds__(kTailThreads) void decode_tail_kernel(DecodeArgs a, TailArgs t) {
  constexpr int G3 = DH / 32, NJ = DH / 2, NS = kTailSlots;
  constexpr int SL = GQA * DH < 128 ? GQA * DH : 128;  // output floats of one workgroup (a slice)
  constexpr int NSL = (GQA * DH) / SL;                 // slices per (seq, head)
  constexpr int HPS = SL / DH;                         // q heads per slice
  constexpr int COLS = SL / 4;                         // float4 columns of a slice
  constexpr int IL = kTailThreads / COLS;              // item lanes
  constexpr int UN = 4;                                // items per item lane per round trip
  constexpr int PS = partial_stride<DH, GQA>();
  constexpr int NCB = G3 * 8 * 32;                     // tier-3 codebook floats of one kv head
  constexpr int FPL = NJ / 16;                         // RoPE frequencies per lane in the logits
  static_assert(kTailThreads == 256 && HPS >= 1 && NCB <= 4 * kTailThreads && (FPL == 4 || FPL == 2),
                "thread maps");
  __shared__ float cbs[NCB];               // the head's tier-3 codebook
  __shared__ __attribute__((aligned(16))) _Float16 vs[NS][DH];   // V of the tail slots (slot NS-1: new token)
  __shared__ double ftab[NJ];              // RoPE frequencies, turns per token
  __shared__ float lg[NS][HPS];            // tail logits of the slice's heads, log2 units (-inf: none)
  __shared__ float tr[NS][G3];             // tail radii
  __shared__ int tc[NS][G3];               // tail codes
  __shared__ int tp[NS];                   // tail positions
  __shared__ float sims[G3][8];
  __shared__ __attribute__((aligned(16))) float dirs[G3][32];   // the new token's directions
  __shared__ float4 red_v[IL][COLS];
  __shared__ float red_m[IL][COLS], red_l[IL][COLS];
  __shared__ float scl[G3];
  __shared__ __attribute__((aligned(16))) uint8_t pg[128];   // the flushed page

  const int sh = blockIdx.x / NSL, slice = blockIdx.x % NSL;
  const int seq = sh / a.num_kv, h = sh % a.num_kv;
  const int h0 = slice * HPS;                          // first q head (of the kv head's GQA) in the slice
  const int i = threadIdx.x, lane = i & 63, wave = i >> 6;
  const bool dec = (t.mode & kTailDecode) != 0;
  const float* cb3 = a.cb[3] + (int64_t)h * NCB;

  // ---- loads: the tail's first (they depend on nothing), then the counts,
  //      the item range and the items' partials --------------------------------
  float4 cbv[NCB / 4 / kTailThreads > 0 ? NCB / 4 / kTailThreads : 1];
#pragma unroll
  for (int k = 0; k < NCB / 4 / kTailThreads; ++k)
    cbv[k] = reinterpret_cast<const float4*>(cb3)[i + k * kTailThreads];
  const bool cb_part = NCB / 4 < kTailThreads && i < NCB / 4;          // dh 64: 128 float4s
  if (cb_part) cbv[0] = reinterpret_cast<const float4*>(cb3)[i];
  half8 vrow;
  if (i < NS * DH / 8) {
    const int w = i / (DH / 8), c8 = i % (DH / 8);
    const _Float16* src = w == NS - 1 ? t.v_new + (int64_t)sh * DH : t.stg_v + ((int64_t)sh * NS + w) * DH;
    vrow = *reinterpret_cast<const half8*>(src + 8 * c8);
  }
  float sr = 0.f;
  int sc = 0, sp = 0;
  if (i < (NS - 1) * G3) {
    sr = t.stg_r[(int64_t)sh * NS * G3 + i];
    sc = t.stg_code[(int64_t)sh * NS * G3 + i];
  }
  if (i < NS - 1) sp = t.stg_pos[(int64_t)sh * NS + i];
  // the new token's encode (wave 3, lane = (group eg, centroid ec)): its
  // group's 32 key values and its centroid row
  const int eg = lane >> 3, ec = lane & 7;
  const bool enc_lane = wave == 3 && eg < G3;
  float x[32], crow[32];
  if (enc_lane) {
    if (t.k_is_fp32) {
      const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(t.k_new) + (int64_t)sh * DH + 32 * eg);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float4 w = src[k];
        x[4 * k] = w.x; x[4 * k + 1] = w.y; x[4 * k + 2] = w.z; x[4 * k + 3] = w.w;
      }
    } else {
      const half8* src = reinterpret_cast<const half8*>(static_cast<const _Float16*>(t.k_new) + (int64_t)sh * DH + 32 * eg);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const half8 hv = src[k];
#pragma unroll
        for (int e = 0; e < 8; ++e) x[8 * k + e] = (float)hv[e];
      }
    }
    const float4* cr = reinterpret_cast<const float4*>(cb3 + (eg * 8 + ec) * 32);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float4 w = cr[k];
      crow[4 * k] = w.x; crow[4 * k + 1] = w.y; crow[4 * k + 2] = w.z; crow[4 * k + 3] = w.w;
    }
  }
  // the logits' lane map: slot 4 * wave + (lane >> 4), frequencies
  // FPL * (lane & 15) .. + FPL - 1; this lane's query values on them
  const int jc = lane & 15, j0 = FPL * jc;
  float qa[HPS][FPL], qb[HPS][FPL];
  if (dec) {
    const _Float16* qh = a.q + ((int64_t)seq * a.num_kv * GQA + (int64_t)h * GQA + h0) * DH;
#pragma unroll
    for (int hh = 0; hh < HPS; ++hh)
#pragma unroll
      for (int f = 0; f < FPL; ++f) {
        qa[hh][f] = (float)qh[hh * DH + j0 + f];
        qb[hh][f] = (float)qh[hh * DH + j0 + f + NJ];
      }
  }
  // the counts, the new token's position and the item range through vector
  // loads (vmcnt): scalar loads share their counter with LDS, and the LDS
  // waits below would then wait for them too
  const int32_t* stp = t.state + (int64_t)sh * 2 * kTailStateInts + t.parity * kTailStateInts;
  const auto st4 = __builtin_amdgcn_raw_buffer_load_b128(make_rsrc(stp, 16), 0, 0, 0);
  const int pos_ld = __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(t.cur_pos + seq, 4), 0, 0, 0);
  const int wsa = __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(a.work_start + sh, 8), 0, 0, 0);
  const int wsb = __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(a.work_start + sh, 8), 4, 0, 0);
  const int c = i % COLS, il = i / COLS;
  const int f0 = slice * SL + 4 * c, hc = f0 / DH;     // first float of this column in [GQA*DH], its head
  // the items' partials: first at the range an even split of the items gives
  // (every (seq, head) with the same item count, the usual list), issued
  // with the item range's own load; reloaded when the range differs
  const int nsh = a.num_sh;
  const int npe = nsh > 0 ? t.num_items / nsh : 0;
  int ib = sh * npe, ni = npe;
  float4 pv[UN];
  float pm[UN], pl[UN];
  auto load_partials = [&](int it0) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < UN; ++k) {
      const int it = it0 + k * IL;
      const float* pp = a.partials + (int64_t)(ib + (it < ni ? it : 0)) * PS;
      pm[k] = it < ni ? pp[hc] : -INFINITY;
      pl[k] = pp[GQA + hc];
      pv[k] = *reinterpret_cast<const float4*>(pp + 16 + f0);
    }
  };
  if (dec && npe * nsh == t.num_items) load_partials(il);

  const int n_st = min(max(__builtin_amdgcn_readfirstlane((int)st4[0]), 0), NS - 1);   // staged tokens
  const int ndec = max(__builtin_amdgcn_readfirstlane((int)st4[1]), 0);                 // decode pages flushed so far
  const int ndrop = max(__builtin_amdgcn_readfirstlane((int)st4[2]), 0);
  const int pos_new = __builtin_amdgcn_readfirstlane(pos_ld);

  // ---- shared tables; the new token's encode -------------------------------
  if (i < NJ) ftab[i] = exp2(-(2.0 * i / DH) * a.log2_theta) * kInvTwoPi;   // inv_freq / 2 pi
#pragma unroll
  for (int k = 0; k < NCB / 4 / kTailThreads; ++k) reinterpret_cast<float4*>(cbs)[i + k * kTailThreads] = cbv[k];
  if (cb_part) reinterpret_cast<float4*>(cbs)[i] = cbv[0];
  if (i < NS * DH / 8) *reinterpret_cast<half8*>(&vs[i / (DH / 8)][8 * (i % (DH / 8))]) = vrow;
  if (i < (NS - 1) * G3) {
    tr[i / G3][i % G3] = sr;
    tc[i / G3][i % G3] = min(max(sc, 0), 7);
  }
  if (i < NS - 1) tp[i] = sp;
  if (i == 0) tp[NS - 1] = pos_new;
  if (wave == 3) {
    // the new token's encode (encode_new_token; its chain of divisions is
    // shared by each group's 8 lanes)
    float r_enc;
    int best;
    encode_new_token(x, crow, eg, ec, enc_lane, !t.k_is_fp32, dirs, sims, r_enc, best);
    if (enc_lane && ec == 0) {
      tr[NS - 1][eg] = r_enc;
      tc[NS - 1][eg] = best;
    }
  }
  __syncthreads();

  if (dec) {
    if (blockIdx.x == 0 && i == 0) {                   // malformed-page count: as the merge kernel
      a.status[1] = a.status[0];
      a.status[0] = 0u;
    }
    // ---- tail logits: 16-lane row = slot, lane = FPL RoPE frequencies --------
    {
      const int w = 4 * wave + (lane >> 4);
      const bool live = w < n_st || w == NS - 1;
      float part[HPS];
#pragma unroll
      for (int hh = 0; hh < HPS; ++hh) part[hh] = 0.f;
      const int g1 = j0 / 32, g2 = (j0 + NJ) / 32;       // the lane's frequencies stay in one group each
      const float* c1p = cbs + (g1 * 8 + tc[w][g1]) * 32 + (j0 & 31);
      const float* c2p = cbs + (g2 * 8 + tc[w][g2]) * 32 + ((j0 + NJ) & 31);
      const float r1 = tr[w][g1], r2 = tr[w][g2];
      const double pw = (double)tp[w];
#pragma unroll
      for (int f = 0; f < FPL; ++f) {
        const float k1 = r1 * c1p[f], k2 = r2 * c2p[f];
        const float2 z = turn_phasor(pw * ftab[j0 + f]);
        // R(pos) k_hat on the pair (j, j + NJ): <q, R(pos) k_hat> = <R(-pos) q, k_hat>
        const float x0 = k1 * z.x - k2 * z.y, x1 = k2 * z.x + k1 * z.y;
#pragma unroll
        for (int hh = 0; hh < HPS; ++hh) part[hh] += qa[hh][f] * x0 + qb[hh][f] * x1;
      }
#pragma unroll
      for (int hh = 0; hh < HPS; ++hh) part[hh] = row_sum16(part[hh]);
      if (jc == 0)
#pragma unroll
        for (int hh = 0; hh < HPS; ++hh) lg[w][hh] = live ? part[hh] * a.scale_log2 : -INFINITY;
    }
    // ---- the work items' log-sum-exp (partials already in registers unless
    //      the item range differs from the even split) -------------------------
    {
      const int ib_w = min(max(__builtin_amdgcn_readfirstlane(wsa), 0), t.num_items);
      const int ie_w = min(max(__builtin_amdgcn_readfirstlane(wsb), ib_w), t.num_items);
      if (ib_w != ib || ie_w - ib_w != ni || npe * nsh != t.num_items) {
        ib = ib_w;
        ni = ie_w - ib_w;
        load_partials(il);
      }
    }
    // the tail slots' logits are all in LDS past this barrier; item lane il
    // starts its state from tail slots il, il + IL, ... (their fp32 weights
    // and V on this column's 4 floats)
    __syncthreads();
    float M = -INFINITY, Ls = 0.f;
    float4 sum = {0.f, 0.f, 0.f, 0.f};
    {
      const int hl = hc - h0, d0 = f0 % DH;
      constexpr int TPL = (NS + IL - 1) / IL;          // tail slots per item lane
      float lw[TPL];
#pragma unroll
      for (int k = 0; k < TPL; ++k) {
        const int w = il + k * IL;
        lw[k] = w < NS ? lg[w][hl] : -INFINITY;
        M = fmaxf(M, lw[k]);
      }
      if (M != -INFINITY) {
#pragma unroll
        for (int k = 0; k < TPL; ++k) {
          const int w = il + k * IL;
          const float p = lw[k] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(lw[k] - M);
          const half4 vv = *reinterpret_cast<const half4*>(&vs[w < NS ? w : 0][d0]);
          Ls += p;
          sum.x += p * (float)vv[0]; sum.y += p * (float)vv[1]; sum.z += p * (float)vv[2]; sum.w += p * (float)vv[3];
        }
      }
    }
    for (int it0 = il, r0 = 0; it0 < ni; it0 += IL * UN, ++r0) {
      if (r0 > 0) load_partials(it0);                  // more than IL * UN items: next round trip
      float Mn = M;
#pragma unroll
      for (int k = 0; k < UN; ++k) Mn = fmaxf(Mn, pm[k]);
      if (Mn == -INFINITY) continue;
      const float r = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M - Mn);
      sum.x *= r; sum.y *= r; sum.z *= r; sum.w *= r;
      Ls *= r;
#pragma unroll
      for (int k = 0; k < UN; ++k) {
        const float f = (pm[k] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(pm[k] - Mn);
        Ls += f * pl[k];
        sum.x += f * pv[k].x; sum.y += f * pv[k].y; sum.z += f * pv[k].z; sum.w += f * pv[k].w;
      }
      M = Mn;
    }
    red_v[il][c] = sum;
    red_m[il][c] = M;
    red_l[il][c] = Ls;
    __syncthreads();
    if (il == 0) {
      // the log-sum-exp of the item lanes' states (the tail already in them)
      float mk[IL];
      float Mx = -INFINITY;
#pragma unroll
      for (int k = 0; k < IL; ++k) {
        mk[k] = red_m[k][c];
        Mx = fmaxf(Mx, mk[k]);
      }
      float4 tot = {0.f, 0.f, 0.f, 0.f};
      float Lt = 0.f;
      if (Mx != -INFINITY) {
#pragma unroll
        for (int k = 0; k < IL; ++k) {
          const float f = mk[k] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mk[k] - Mx);
          const float4 xk = red_v[k][c];
          tot.x += f * xk.x; tot.y += f * xk.y; tot.z += f * xk.z; tot.w += f * xk.w;
          Lt += f * red_l[k][c];
        }
      }
      const float inv = Lt > 0.f ? 1.f / Lt : 0.f;
      half4 o;
      o[0] = (_Float16)(tot.x * inv); o[1] = (_Float16)(tot.y * inv);
      o[2] = (_Float16)(tot.z * inv); o[3] = (_Float16)(tot.w * inv);
      *reinterpret_cast<half4*>(a.out + ((int64_t)seq * a.num_kv * GQA + (int64_t)h * GQA) * DH + f0) = o;
    }
  }
  if (!(t.mode & kTailAppend) || slice != 0) return;
  ib = min(max(__builtin_amdgcn_readfirstlane(wsa), 0), t.num_items);
  const int ie = min(max(__builtin_amdgcn_readfirstlane(wsb), ib), t.num_items);

  // ---- append the new token (_append_decode_kv), by slice 0 -----------------
  // (every staged value and the new token's encode are in LDS since the
  // first barrier)
  int32_t* nst = t.state + (int64_t)sh * 2 * kTailStateInts + (1 - t.parity) * kTailStateInts;   // next counts
  if (n_st < NS - 1) {
    const int sl = n_st;
    if (i < DH / 8)
      *reinterpret_cast<half8*>(t.stg_v + ((int64_t)sh * NS + sl) * DH + 8 * i) =
          *reinterpret_cast<const half8*>(&vs[NS - 1][8 * i]);
    if (i < G3) {
      t.stg_r[((int64_t)sh * NS + sl) * G3 + i] = tr[NS - 1][i];
      t.stg_code[((int64_t)sh * NS + sl) * G3 + i] = tc[NS - 1][i];
    }
    if (i == 0) {
      t.stg_pos[(int64_t)sh * NS + sl] = pos_new;
      nst[0] = sl + 1; nst[1] = ndec; nst[2] = ndrop; nst[3] = 0;
    }
    return;
  }
  // ---- the staged 15 tokens and the new one fill a page: flush it
  //      (_flush_decode_page, build_page_from_codes, pagebuilder.py:8-42) -----
  constexpr int TB = (NS * G3 * 3) / 8;                // theta bytes: 16 tokens x G3 codes x 3 bits
  constexpr int PB = 8 + 4 * G3 + TB + NS * G3;        // page bytes
  constexpr int SLOT = (PB + 15) & ~15;
  const int k = sh * t.dec_cap + ndec;
  const int row = ie > ib ? t.work[4 * (int64_t)ib + 2] : -1;   // sh's next reserved row
  if (ndec >= t.dec_cap || row < 0 || row >= t.num_rows) {
    // no decode slot left (or no item / a corrupted list): the token is dropped
    if (i == 0) { nst[0] = n_st; nst[1] = ndec; nst[2] = ndrop + 1; nst[3] = 0; }
    return;
  }
  if (i < G3) {                                        // r_scale[g] = max_n r[n, g]
    float m = fabsf(tr[0][i]);
    for (int n = 1; n < NS; ++n) {
      const float xn = fabsf(tr[n][i]);
      if (xn > m) m = xn;
    }
    scl[i] = m;
  }
  __syncthreads();
  if (i < SLOT) {
    uint8_t byte = 0;
    if (i == 0) byte = 3;                              // tier id
    else if (i == 1) byte = NS;                        // count
    else if (i >= 8 && i < 8 + 4 * G3) {
      const uint32_t w = __builtin_bit_cast(uint32_t, scl[(i - 8) >> 2]);
      byte = (uint8_t)(w >> (8 * ((i - 8) & 3)));
    } else if (i >= 8 + 4 * G3 && i < 8 + 4 * G3 + TB) {
      // LSB-first stream: bit j of item n*G3 + g at bit (n*G3 + g)*3 + j
      const int b0 = 8 * (i - 8 - 4 * G3);
#pragma unroll
      for (int bb = 0; bb < 8; ++bb) {
        const int gb = b0 + bb, item = gb / 3, jb = gb % 3;
        byte |= (uint8_t)(((tc[item / G3][item % G3] >> jb) & 1) << bb);
      }
    } else if (i >= 8 + 4 * G3 + TB && i < PB) {
      const int item = i - (8 + 4 * G3 + TB), n = item / G3, g = item % G3;
      const float safe = scl[g] < 1e-8f ? 1e-8f : scl[g];
      float qv = __builtin_rintf(__fmul_rn(__fdiv_rn(tr[n][g], safe), 127.0f));
      qv = fminf(fmaxf(qv, -127.f), 127.f);
      byte = (uint8_t)(int8_t)(int)qv;
    }
    pg[i] = byte;
  }
  __syncthreads();
  if (i < SLOT / 4)
    reinterpret_cast<uint32_t*>(t.pages + t.dec_byte0 + (int64_t)k * SLOT)[i] = reinterpret_cast<const uint32_t*>(pg)[i];
  if (i < NS) t.positions[(int64_t)row * NS + i] = tp[i];
  if (i < DH) {                                        // dim-major V page: element (token n, dim d) at d*16 + n
    half8 lo, hi;
#pragma unroll
    for (int n = 0; n < NS; ++n) {
      if (n < 8) lo[n] = vs[n][i]; else hi[n - 8] = vs[n][i];
    }
    half8* dst = reinterpret_cast<half8*>(t.v_pool + ((int64_t)t.dec_vpage0 + k) * (DH * NS) + (int64_t)i * NS);
    dst[0] = lo;
    dst[1] = hi;
  }
  for (int it = ib + i; it < ie; it += kTailThreads) t.work[4 * (int64_t)it + 2] = row + 1;   // sh's items take the row
  if (i == 0) { nst[0] = 0; nst[1] = ndec + 1; nst[2] = ndrop; nst[3] = 0; }
}

// Decode-time pointer table (the layout sphkv_decode_step reads): the
// prefill rows of (seq, head) sh, [row_start[sh], row_start[sh + 1]), move to
// row p + sh * dec_cap, and dec_cap reserved rows follow them: reserved row k
// of sh gets the pointer-table row of a full tier-3 page at bytes dec_byte0 +
// (sh * dec_cap + k) * slot, V page dec_vpage0 + sh * dec_cap + k and
// positions -1.  One thread per prefill row (its sh by binary search of
// row_start) or per reserved row.
__global__ __launch_bounds__(256) void tail_relayout_kernel(const int32_t* __restrict__ row_start, int32_t num_sh,
                                                            int32_t num_rows, const int32_t* __restrict__ ptable,
                                                            const int32_t* __restrict__ vslot,
                                                            const int32_t* __restrict__ positions, int32_t dec_cap,
                                                            int64_t dec_byte0, int32_t dec_vpage0, int32_t slot,
                                                            int32_t G3, int32_t* __restrict__ ptable_d,
                                                            int32_t* __restrict__ vslot_d,
                                                            int32_t* __restrict__ positions_d) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t nres = (int64_t)num_sh * dec_cap;
  if (t < num_rows) {
    const int p = (int)t;
    int lo = 0, hi = num_sh;                           // last sh with row_start[sh] <= p
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (row_start[mid] <= p) lo = mid; else hi = mid;
    }
    const int64_t r = (int64_t)p + (int64_t)lo * dec_cap;   // < num_rows + nres: lo < num_sh
    ptable_d[3 * r] = ptable[3 * (int64_t)p];
    ptable_d[3 * r + 1] = ptable[3 * (int64_t)p + 1];
    ptable_d[3 * r + 2] = ptable[3 * (int64_t)p + 2];
    vslot_d[r] = vslot[p];
    for (int i = 0; i < kTile; ++i) positions_d[r * kTile + i] = positions[(int64_t)p * kTile + i];
  } else if (t < num_rows + nres) {
    const int64_t q = t - num_rows;
    const int sh = (int)(q / dec_cap), k = (int)(q % dec_cap);
    const int64_t r = (int64_t)row_start[sh + 1] + (int64_t)sh * dec_cap + k;
    if (r < 0 || r >= num_rows + nres) return;         // row_start not a table of num_rows rows
    const int64_t off = dec_byte0 + q * slot;
    ptable_d[3 * r] = (int32_t)off;
    ptable_d[3 * r + 1] = (int32_t)(off + 8 + 4 * G3);
    ptable_d[3 * r + 2] = (int32_t)(off + 8 + 4 * G3 + 6 * G3);
    vslot_d[r] = (int32_t)(dec_vpage0 + q);
    for (int i = 0; i < kTile; ++i) positions_d[r * kTile + i] = -1;
  }
}

int launch_tail_relayout(const int32_t* row_start, int32_t num_sh, int32_t num_rows, const int32_t* ptable,
                         const int32_t* vslot, const int32_t* positions, int32_t dec_cap, int64_t dec_byte0,
                         int32_t dec_vpage0, int32_t dh, int32_t* ptable_d, int32_t* vslot_d,
                         int32_t* positions_d, hipStream_t stream) {
  const int64_t n = (int64_t)num_rows + (int64_t)num_sh * dec_cap;
  if (n > 0)
    hipLaunchKernelGGL(tail_relayout_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, row_start,
                       num_sh, num_rows, ptable, vslot, positions, dec_cap, dec_byte0, dec_vpage0,
                       tail_slot_bytes(dh), dh / 32, ptable_d, vslot_d, positions_d);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <int DH, int GQA>
static DecodeArgs decode_args(const DecodeLaunch& L) {
  DecodeArgs a;
  a.pages = L.pages; a.pages_bytes = L.pages_bytes; a.ptable = L.ptable; a.vslot = L.vslot;
  a.positions = L.positions; a.v_pool = reinterpret_cast<const _Float16*>(L.v_pool);
  a.num_vpages = L.num_vpages; a.cb[0] = nullptr; a.cb[1] = L.cb1; a.cb[2] = L.cb2; a.cb[3] = L.cb3;
  a.work = L.work; a.work_start = L.work_start; a.q = reinterpret_cast<const _Float16*>(L.q);
  a.out = reinterpret_cast<_Float16*>(L.out); a.partials = L.partials;
  a.status = L.partials ? reinterpret_cast<uint32_t*>(L.partials + (int64_t)L.num_items * partial_stride<DH, GQA>())
                         : nullptr;
  a.num_kv = L.num_kv; a.num_rows = L.num_rows; a.num_sh = L.num_seqs * L.num_kv;
  a.pages32 = (int32_t)L.pages_bytes;
  a.pages_m8 = (int32_t)L.pages_bytes - 8;
  a.nvp32 = L.num_vpages > 0x7FFFFFFF ? 0x7FFFFFFF : (int32_t)L.num_vpages;
  a.scale_log2 = L.sm_scale * 1.4426950408889634f;
  a.scale_log2_c = a.scale_log2 * (1.0f / 127.0f);
  a.log2_theta = __builtin_log2(L.rope_theta);
  return a;
}

template <int DH, int GQA>
static int launch_decode_t(const DecodeLaunch& L, int phases, hipStream_t stream) {
  const DecodeArgs a = decode_args<DH, GQA>(L);
  if (L.num_items > 0) {
    if (phases & kPhasePartials)
      launch_timed(decode_kernel<DH, GQA>, dim3(L.num_items), dim3(decode_waves<GQA>() * 64), stream, L.work,
                   L.num_items, a);
    const int nsh = L.num_seqs * L.num_kv;
    if ((phases & kPhaseMerge) && nsh > 0)
      hipLaunchKernelGGL((decode_merge_kernel<DH, GQA>), dim3(nsh * ((GQA * DH) / (GQA * DH < 128 ? GQA * DH : 128))),
                         dim3(256), 0, stream, L.partials, L.work_start, L.num_items, L.num_kv,
                         reinterpret_cast<_Float16*>(L.out), a.status);
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_decode(const DecodeLaunch& L, int phases, hipStream_t stream) {
#define SPHKV_DISPATCH(D, Q) if (L.dh == D && L.gqa == Q) return launch_decode_t<D, Q>(L, phases, stream);
  SPHKV_DISPATCH(128, 1) SPHKV_DISPATCH(128, 2) SPHKV_DISPATCH(128, 4) SPHKV_DISPATCH(128, 8)
  SPHKV_DISPATCH(64, 1) SPHKV_DISPATCH(64, 2) SPHKV_DISPATCH(64, 4) SPHKV_DISPATCH(64, 8)
#undef SPHKV_DISPATCH
  return -1;
}

template <int DH, int GQA>
static int launch_decode_tail_t(const DecodeLaunch& L, const TailLaunch& T, hipStream_t stream) {
  const DecodeArgs a = decode_args<DH, GQA>(L);
  TailArgs t;
  t.k_new = T.k_new; t.v_new = reinterpret_cast<const _Float16*>(T.v_new); t.cur_pos = T.cur_pos;
  t.stg_r = T.stg_r; t.stg_code = T.stg_code; t.stg_v = reinterpret_cast<_Float16*>(T.stg_v);
  t.stg_pos = T.stg_pos; t.state = T.state; t.pages = T.pages; t.positions = T.positions;
  t.v_pool = reinterpret_cast<_Float16*>(T.v_pool); t.work = T.work; t.dec_byte0 = T.dec_byte0;
  t.dec_cap = T.dec_cap; t.dec_vpage0 = T.dec_vpage0; t.k_is_fp32 = T.k_is_fp32;
  t.mode = T.mode; t.num_items = L.num_items; t.num_rows = L.num_rows; t.parity = T.parity & 1;
  const int nsh = L.num_seqs * L.num_kv;
  if ((T.mode & kTailDecode) && L.num_items > 0)
    launch_timed(decode_kernel<DH, GQA>, dim3(L.num_items), dim3(decode_waves<GQA>() * 64), stream, L.work,
                 L.num_items, a);
  constexpr int NSL = (GQA * DH) / (GQA * DH < 128 ? GQA * DH : 128);
  if (nsh > 0)
    hipLaunchKernelGGL((decode_tail_kernel<DH, GQA>), dim3(nsh * NSL), dim3(kTailThreads), 0, stream, a, t);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_decode_tail(const DecodeLaunch& L, const TailLaunch& T, hipStream_t stream) {
#define SPHKV_DISPATCH(D, Q) if (L.dh == D && L.gqa == Q) return launch_decode_tail_t<D, Q>(L, T, stream);
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
template <int DH>
__global__ __launch_bounds__(256) void ragged_logits_kernel(RaggedLaunch a) {
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int p = blockIdx.x * 4 + wave;
  if (p >= a.num_pages) return;
  const int t16 = lane & 15, u = lane >> 4;
  const int64_t page_off = a.ptable[3 * p];
  const int64_t th_off = a.ptable[3 * p + 1];
  const int64_t rad_off = a.ptable[3 * p + 2];
  const int G = a.groups, g = a.group_size, b = a.b_theta, dh = DH;
  int n = (page_off >= 0 && page_off + 2 <= a.pages_bytes) ? (int)a.pages[page_off + 1] : 0;
  if (n > a.page_size) n = a.page_size;
  if (page_off + kHeaderBytes + 4 * G > a.pages_bytes || th_off < 0 || rad_off < 0 ||
      th_off + ((int64_t)n * G * b + 7) / 8 > a.pages_bytes || rad_off + (int64_t)n * G > a.pages_bytes)
    n = 0;
  const int C = 1 << b;
  const int hk = a.head_ids[p];
  constexpr int dq = DH / 4;           // dims per lane
  constexpr int half_dh = DH / 2;
  const int64_t total_slots = (int64_t)a.num_pages * a.page_size;
  for (int t0 = 0; t0 < a.page_size; t0 += 16) {
    const int t = t0 + t16;
    const bool in_page = t < a.page_size;
    const int pos = in_page ? a.positions[(int64_t)p * a.page_size + t] : -1;
    const bool valid = in_page && t < n && pos >= 0 && pos < a.max_pos && hk >= 0 && hk < a.num_kv;
    // lane covers RoPE pairs j = u*dq/2 .. +dq/2 of the first half and their partners
    float kr[DH / 4];
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

// Fast form of the ragged kernel for page_size % 16 == 0, group size 16 or
// 32 and grp <= 8 (the reference's call shapes).  One wave per 16 slots of a
// page; lane = (slot t, dim quarter u) as in the decode kernel: the lane
// rebuilds its token's key on its quarter's RoPE pairs (j, j + DH/2), j in
// [DH/8 u, DH/8 (u + 1)), from two codes, two int8 radii, two fp32 scales and
// two centroid runs, rotates it with the caller's cos / sin rows at the
// token's position (first-half entries, HF layout), and the q.k sums run on
// the fp32 4x4x1 MFMA (A = q of head slot t mod 4, B = the lane's own rotated
// key; blocks = (quarter, token group)), then over the quarters with the row
// swaps.  The loads form three round trips: the pointer-table row, head id
// and positions; then the page's bytes (read whatever the token count says
// -- the count only masks the output), the cos / sin rows and q; then the
// centroid runs.  Page bytes are read with buffer loads (absent data reads
// zeros; a buffer load returns zero for a dword that reaches past the pool,
// so the pool's partial last dword is read once bytewise and substituted).
// A page's validity rules are those of ragged_logits_kernel.
template <int DH, int GS, int NHS>
__global__ __launch_bounds__(256) void ragged_fast_kernel(RaggedLaunch a) {
  constexpr int NPL = DH / 8;                          // RoPE pairs per lane
  constexpr int G = DH / GS;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int cpp = a.page_size / 16;                    // 16-slot chunks per page
  const int64_t chunk = (int64_t)blockIdx.x * 4 + wave;
  if (chunk >= (int64_t)a.num_pages * cpp) return;
  const int p = uniform((int)(chunk / cpp)), c16 = uniform((int)(chunk % cpp));
  const int t = lane & 15, u = lane >> 4, ts = 16 * c16 + t;
  // round trip 1: the row, the head, the positions
  const int64_t page_off = a.ptable[3 * (int64_t)p], th_off = a.ptable[3 * (int64_t)p + 1],
                rad_off = a.ptable[3 * (int64_t)p + 2];
  const int hk = a.head_ids[p];
  const int pos_raw = a.positions[(int64_t)p * a.page_size + ts];
  const int b = a.b_theta, C = 1 << b;
  const rsrc_t rs = make_rsrc(a.pages, a.pages_bytes);
  const int64_t pb = a.pages_bytes > 0x7FFFFFFF ? 0x7FFFFFFF : a.pages_bytes;
  const int tail4 = (int)(pb & ~(int64_t)3);
  // offsets inside the pool or kOOB (the validity checks come later)
  auto in_pool = [&](int64_t o) { return (o >= 0 && o < pb) ? (int)o : kOOB; };
  // round trip 2: count byte, the pool's partial last dword, codes, radii,
  // scales; cos / sin at the position; q of the lane's head slots
  const bool hdr_ok = page_off >= 0 && page_off + 2 <= a.pages_bytes;
  const int cnt = __builtin_amdgcn_raw_buffer_load_b8(rs, in_pool(page_off + 1), 0, 0);
  uint32_t tailw = 0;
#pragma unroll
  for (int i = 0; i < 3; ++i)
    tailw |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rs, tail4 + i < pb ? tail4 + i : kOOB, 0, 0) << (8 * i);
  auto dword_at = [&](int64_t o4) {                    // o4: a multiple of 4 (or negative)
    const uint32_t w = __builtin_amdgcn_raw_buffer_load_b32(rs, in_pool(o4), 0, 0);
    return w | (o4 == tail4 ? tailw : 0u);             // the partial dword itself reads as zero
  };
  const int d0 = NPL * u, gi = d0 / GS, off = d0 % GS, gj = gi + G / 2;
  const int gg[2] = {gi, gj};
  uint32_t cwin[2][2], swin[2][2];
  int rcode[2];
  int64_t cbit[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    cbit[k] = th_off * 8 + (int64_t)(ts * G + gg[k]) * b;
    const int64_t o4 = (cbit[k] >> 5) * 4;
    cwin[k][0] = dword_at(o4);
    cwin[k][1] = dword_at(o4 + 4);
    rcode[k] = (int)(int8_t)__builtin_amdgcn_raw_buffer_load_b8(rs, in_pool(rad_off + ts * G + gg[k]), 0, 0);
    const int64_t so = page_off + kHeaderBytes + 4 * gg[k];
    const int64_t s4 = so >= 0 ? (so >> 2) * 4 : -4;
    swin[k][0] = dword_at(s4);
    swin[k][1] = dword_at(s4 + 4);
  }
  const bool pos_ok = pos_raw >= 0 && pos_raw < a.max_pos;
  const int pos = pos_ok ? pos_raw : 0;
  const bool head_ok = hk >= 0 && hk < a.num_kv;
  const int hq = head_ok ? hk : 0;
  const float* cs = a.cos_tbl + (int64_t)pos * DH + d0;
  const float* sn = a.sin_tbl + (int64_t)pos * DH + d0;
  float4 cc[NPL / 4], ss[NPL / 4], q0[NHS][NPL / 4], q1[NHS][NPL / 4];
#pragma unroll
  for (int m = 0; m < NPL / 4; ++m) {
    cc[m] = *reinterpret_cast<const float4*>(cs + 4 * m);
    ss[m] = *reinterpret_cast<const float4*>(sn + 4 * m);
#pragma unroll
    for (int hs = 0; hs < NHS; ++hs) {
      const int slot = 4 * hs + (t & 3);
      const bool q_ok = slot < a.grp;
      const float* qr = a.q + ((int64_t)hq * a.grp + (q_ok ? slot : 0)) * DH + d0 + 4 * m;
      q0[hs][m] = q_ok ? *reinterpret_cast<const float4*>(qr) : float4{0.f, 0.f, 0.f, 0.f};
      q1[hs][m] = q_ok ? *reinterpret_cast<const float4*>(qr + DH / 2) : float4{0.f, 0.f, 0.f, 0.f};
    }
  }
  // validity (ragged_logits_kernel's rules)
  int n = hdr_ok ? min(cnt, a.page_size) : 0;
  if (page_off + kHeaderBytes + 4 * G > a.pages_bytes || th_off < 0 || rad_off < 0 ||
      th_off + ((int64_t)n * G * b + 7) / 8 > a.pages_bytes || rad_off + (int64_t)n * G > a.pages_bytes)
    n = 0;
  const bool valid = ts < n && pos_ok && head_ok;
  // round trip 3: the centroid runs of the two codes
  int code[2];
  float rad[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    code[k] = (int)(__builtin_amdgcn_alignbit(cwin[k][1], cwin[k][0], (uint32_t)(cbit[k] & 31)) & (uint32_t)(C - 1));
    const int64_t so = page_off + kHeaderBytes + 4 * gg[k];
    const float sc = __builtin_bit_cast(float, __builtin_amdgcn_alignbyte(swin[k][1], swin[k][0], (uint32_t)(so & 3)));
    rad[k] = (float)rcode[k] * sc * (1.0f / 127.0f);
  }
  const float* c1 = a.codebooks + ((int64_t)(hq * G + gi) * C + code[0]) * GS + off;
  const float* c2 = a.codebooks + ((int64_t)(hq * G + gj) * C + code[1]) * GS + off;
  floatx4 acc[NHS];
#pragma unroll
  for (int hs = 0; hs < NHS; ++hs) acc[hs] = (floatx4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int m = 0; m < NPL / 4; ++m) {
    const float4 cv1 = *reinterpret_cast<const float4*>(c1 + 4 * m);
    const float4 cv2 = *reinterpret_cast<const float4*>(c2 + 4 * m);
    const float k1[4] = {rad[0] * cv1.x, rad[0] * cv1.y, rad[0] * cv1.z, rad[0] * cv1.w};
    const float k2[4] = {rad[1] * cv2.x, rad[1] * cv2.y, rad[1] * cv2.z, rad[1] * cv2.w};
    const float co[4] = {cc[m].x, cc[m].y, cc[m].z, cc[m].w}, si[4] = {ss[m].x, ss[m].y, ss[m].z, ss[m].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float x0 = k1[e] * co[e] - k2[e] * si[e];
      const float x1 = k2[e] * co[e] + k1[e] * si[e];
#pragma unroll
      for (int hs = 0; hs < NHS; ++hs) {
        const float4 qa4 = q0[hs][m], qb4 = q1[hs][m];
        const float qa = e == 0 ? qa4.x : e == 1 ? qa4.y : e == 2 ? qa4.z : qa4.w;
        const float qb = e == 0 ? qb4.x : e == 1 ? qb4.y : e == 2 ? qb4.z : qb4.w;
        acc[hs] = __builtin_amdgcn_mfma_f32_4x4x1f32(qa, x0, acc[hs], 0, 0, 0);
        acc[hs] = __builtin_amdgcn_mfma_f32_4x4x1f32(qb, x1, acc[hs], 0, 0, 0);
      }
    }
  }
  // lane (t, u): acc[hs][i] = head slot 4 hs + i over quarter u's pairs.  Sum
  // over the quarters so that lane u ends with head slot 4 hs + u
  const int64_t total_slots = (int64_t)a.num_pages * a.page_size;
  const float inv = 1.0f / __builtin_sqrtf((float)DH);
#pragma unroll
  for (int hs = 0; hs < NHS; ++hs) {
    float s0 = acc[hs][0], s2 = acc[hs][2], s1 = acc[hs][1], s3 = acc[hs][3];
    swap32(s0, s2);                                    // lower rows: slot 0 pair, upper: slot 2 pair
    swap32(s1, s3);
    float x = s0 + s2, y = s1 + s3;
    swap16(x, y);                                      // even rows: slots 0 / 2, odd: 1 / 3
    const float v = x + y;
    const int i = 4 * hs + u;
    if (i < a.grp)
      a.logits_out[(int64_t)i * total_slots + (int64_t)p * a.page_size + ts] = valid ? v * inv : -INFINITY;
  }
}

// Pipelined form of the ragged kernel (same shapes as ragged_fast_kernel,
// plus C <= 64 and q of every head within 32 KB): a persistent workgroup of
// four waves takes a contiguous run of iterations, each iteration 4
// consecutive 16-slot chunks (one per wave).  q of every head is staged in
// LDS once, and the codebook of the head of each iteration's first chunk is
// staged when that head changes (pages arrive grouped by head).  Per wave,
// the loads of chunk i + 2's pointer-table row, head ids and positions, and
// of chunk i + 1's page bytes and cos / sin rows, are in flight while chunk i
// is computed (vector loads only: scalar loads share a wait counter with the
// LDS reads and return out of order, so a wait for LDS data would wait for
// them too).  The arithmetic per chunk is ragged_fast_kernel's.
//
// RM (a RopeFit model): kRopeNone reads each token's cos / sin rows from the
// caller's tables (16 rows of 2 x DH/2 floats per chunk, the kernel's largest
// read); kRopeExact and kRopeFp32 form the same phasors in the kernel from
// the fitted frequencies (every table entry within kRopeFitTol of them,
// checked once per table by sphkv_rope_table_fit): the lane's pairs j turn by
// 2 pi pos f[j] (exact angle) or by the fp32 angle fl32(pos * inv32[j])
// reduced in fp64, on the hardware sine / cosine (turns).
constexpr int kRagWaves = 4, kRagThreads = 64 * kRagWaves;     // waves of a pipelined-kernel workgroup
constexpr int kStage4 = (2048 + kRagThreads - 1) / kRagThreads;  // float4 per thread of a 32 KB LDS stage
struct RagRow {          // round trip 1 of one chunk
  uint32_t w0, w1, w2;   // pointer-table row (page_off, th_off, rad_off)
  int hk, hb, pos;       // head of the chunk's page, head of the iteration's first chunk, slot position
  int p, c16;            // the chunk's page and 16-slot chunk within it
};
struct RagPage {         // round trip 2 of one chunk, with its row's fields
  uint32_t cnt, cw[2][2], sw[2][2];
  int rc[2];
  int page_off, th_off, rad_off, hk, hb, pos, p, c16;
};
// LDS of the pipelined kernel: the staged head's q rows (padded by 4 floats,
// so that the 4 rows one read touches start in different banks) and its
// codebook, whose float4 slots are XOR-swizzled by the row (a read of 16
// random codes then spreads over 16 bank groups instead of 4).
template <int DH> __host__ __device__ constexpr int rag_q_stride() { return DH + 4; }
template <int GS>
__device__ __forceinline__ int rag_cb_index(int row, int slot4) {   // float index of float4 slot4 of a row
  constexpr int R4 = GS / 4, SH = R4 == 4 ? 2 : 1;                  // 16 bank groups of 64 banks
  return row * GS + 4 * (slot4 ^ ((row >> SH) & (R4 - 1)));
}

// Offsets are 32-bit: the launcher takes this kernel only for byte pools
// below 2 GiB and fewer than 2^31 slots; a pointer-table row with a negative
// offset reads nothing and contributes no token.
template <int DH, int GS, int NHS, int RM>
__global__ __launch_bounds__(kRagThreads) void ragged_pipe_kernel(RaggedLaunch a) {
  constexpr int NPL = DH / 8, NM = NPL / 4;
  constexpr int G = DH / GS;
  constexpr int QS = rag_q_stride<DH>();
  constexpr int SLOTS = 4 * NHS;                       // q rows of a head in LDS (zeros past grp)
  extern __shared__ float rag_smem[];
  const int lane = threadIdx.x & 63, wave = uniform(threadIdx.x >> 6);
  const int t = lane & 15, u = lane >> 4;
  const int cpp = a.page_size / 16;
  const int cpp_sh = (cpp & (cpp - 1)) == 0 ? __builtin_ctz(cpp) : -1;
  const int nch = a.num_pages * cpp;
  // Work split for L2 locality.  Chunks come grouped by head, each head's in
  // ascending position, and every head covers about the same positions, so
  // [0, nch) is cut into S = NX * K equal segments (K per XCD, K ~ heads)
  // and XCD x (workgroups b with b mod NX = x; the dispatcher deals
  // workgroups to the 8 XCDs in turn) takes segments x, x + NX, ...: about
  // the same 1/NX of the positions of every head, so its L2 holds 1/NX of
  // the cos / sin rows (table path) and a workgroup's run mostly stays in
  // one head (one codebook stage).  Its segments, concatenated, are cut into
  // GPX runs, one per workgroup (below).  Any order of pages is still covered
  // exactly once.  Lane k < K holds segment k's list range and chunk offset;
  // a list position maps to a chunk by a ballot over that table.
  const int NX = (gridDim.x % 8 == 0 && gridDim.x >= 64) ? 8 : 1;
  const int K = NX == 8 ? min(max(a.num_kv, 1), 8) : 1;
  const int S = NX * K, xcd = blockIdx.x % NX, GPX = gridDim.x / NX, wj = blockIdx.x / NX;
  int seg_end = 0, seg_base = 0;                       // lane k < K: list end and chunk - list offset of segment k
  {
    // 32-bit products: sg < 64 and nch < 2^25
    const uint32_t sg = xcd + NX * lane;
    const int b0 = lane < K ? (int)(sg * (uint32_t)nch / (uint32_t)S) : 0;
    const int b1 = lane < K ? (int)((sg + 1) * (uint32_t)nch / (uint32_t)S) : 0;
    const int len = b1 - b0;
    int incl = len;
#pragma unroll
    for (int d = 1; d < 8; d <<= 1) {                  // K <= 8 lanes

      const int o = __shfl_up(incl, d, 64);
      if (lane >= d) incl += o;
    }
    seg_end = incl;
    seg_base = b0 - (incl - len);
  }
  const int Lx = __builtin_amdgcn_readlane(seg_end, K - 1);
  // Workgroups start over several microseconds (the dispatcher places them
  // one after another: the 768 workgroups of 4 waves of a config-2 call
  // start over 4.7 us), and a workgroup dispatched late with an equal share
  // finishes late.  So the XCD's iterations (kRagWaves chunks each) are cut
  // at whole iterations with shares that fall linearly in dispatch order:
  // workgroup wj's run ends at F(x) = x + alpha x (1 - x) of them, x =
  // (wj + 1) / GPX; alpha grows with the grid (the spread) and shrinks with
  // the iterations per workgroup (the work that absorbs it): 2.4e-3 per
  // workgroup of the grid over the mean iterations, at most 0.9.
  const int itot = (Lx + kRagWaves - 1) / kRagWaves;
  const float alpha = fminf(0.9f, 2.4e-3f * (float)gridDim.x * (float)GPX / (float)max(itot, GPX));
  auto cut = [&](int w) {                              // list position where workgroup w's run starts
    if (w >= GPX) return Lx;
    const float x = (float)w / (float)GPX;
    const int c = (int)__builtin_rintf((x + alpha * x * (1.f - x)) * (float)itot);   // itot < 2^23
    return min(kRagWaves * min(max(c, 0), itot), Lx);
  };
  const int q0 = cut(wj), q1 = cut(wj + 1);
  const int it1 = (q1 - q0 + kRagWaves - 1) / kRagWaves;
  if (it1 == 0) return;                                // whole workgroup
  auto chunk_of = [&](int q) {                         // list position (< Lx) -> chunk index
    const uint64_t m = __builtin_amdgcn_ballot_w64(lane < K && seg_end > q);
    const int k = m ? (int)__builtin_ctzll(m) : 0;
    return q + __builtin_amdgcn_readlane(seg_base, k);
  };
  const int b = a.b_theta, C = 1 << b;
  float* q_s = rag_smem;                               // [SLOTS][QS] of the staged head
  float* cb_s = rag_smem + SLOTS * QS;                 // [G * C][GS] (swizzled) of the staged head
  const uint32_t pb = (uint32_t)a.pages_bytes;         // < 2^31
  const rsrc_t rs = make_rsrc(a.pages, a.pages_bytes);
  const rsrc_t rt = make_rsrc(a.ptable, (int64_t)a.num_pages * 12);
  const rsrc_t rh = make_rsrc(a.head_ids, (int64_t)a.num_pages * 4);
  const rsrc_t rp = make_rsrc(a.positions, (int64_t)a.num_pages * a.page_size * 4);
  const rsrc_t rcb = make_rsrc(a.codebooks, (int64_t)a.num_kv * G * C * GS * 4);
  const uint32_t tail4 = pb & ~3u;
  uint32_t tailw = 0;
#pragma unroll
  for (int i = 0; i < 3; ++i)
    tailw |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rs, tail4 + i < pb ? (int)(tail4 + i) : kOOB, 0, 0)
             << (8 * i);
  const rsrc_t rq = make_rsrc(a.q, (int64_t)a.num_kv * a.grp * DH * 4);
  const int d0 = NPL * u, gi = d0 / GS, off = d0 % GS, gj = gi + G / 2;
  // the fitted frequencies in LDS (a lane reads its pairs' four at a time:
  // 16 registers fewer than holding them); a fit of another model or shape
  // makes every logit NaN.  The return above is workgroup-uniform, so every
  // thread reaches the barrier.
  __shared__ double fr_s[RM == kRopeExact ? DH / 2 : 1];
  __shared__ float iv_s[RM == kRopeFp32 ? DH / 2 : 1];
  bool fit_ok = true;
  if constexpr (RM != kRopeNone) {
    fit_ok = a.rope->model == RM && a.rope->dh == DH && a.rope->max_pos == a.max_pos;
    if (threadIdx.x < DH / 2) {
      if constexpr (RM == kRopeExact) fr_s[threadIdx.x] = a.rope->f[threadIdx.x];
      else iv_s[threadIdx.x] = a.rope->inv32[threadIdx.x];
    }
    __syncthreads();
  }

  auto row_of = [&](int it) {                          // issue round trip 1 of this wave's chunk of iteration it
    RagRow r;
    const int q = q0 + kRagWaves * it + wave;
    const bool act = it < it1 && q < q1;
    const int ch = act ? chunk_of(q) : 0, ch0 = it < it1 ? chunk_of(q0 + kRagWaves * it) : 0;
    int p, c16, p0;
    if (cpp_sh >= 0) {
      p = ch >> cpp_sh;
      c16 = ch & (cpp - 1);
      p0 = ch0 >> cpp_sh;
    } else {
      p = (int)((uint32_t)ch / (uint32_t)cpp);
      c16 = ch - p * cpp;
      p0 = (int)((uint32_t)ch0 / (uint32_t)cpp);
    }
    r.p = p;
    r.c16 = c16;
    // unconditional loads (absent ones read zeros): a branch around a load
    // would make the compiler's waits for the loads in flight conservative
    const auto w = __builtin_amdgcn_raw_buffer_load_b96(rt, act ? 12 * p : kOOB, 0, 0);
    r.w0 = (uint32_t)w[0]; r.w1 = (uint32_t)w[1]; r.w2 = (uint32_t)w[2];
    r.hk = (int)__builtin_amdgcn_raw_buffer_load_b32(rh, act ? 4 * p : kOOB, 0, 0);
    r.hb = (int)__builtin_amdgcn_raw_buffer_load_b32(rh, it < it1 ? 4 * p0 : kOOB, 0, 0);
    r.pos = (int)__builtin_amdgcn_raw_buffer_load_b32(rp, act ? 4 * (p * a.page_size + 16 * c16 + t) : kOOB, 0, 0);
    return r;
  };
  auto page_of = [&](const RagRow& r, int ts, float4 (&cc)[NM], float4 (&ss)[NM]) {   // issue round trip 2
    RagPage g;
    g.page_off = (int32_t)__builtin_amdgcn_readfirstlane(r.w0);
    g.th_off = (int32_t)__builtin_amdgcn_readfirstlane(r.w1);
    g.rad_off = (int32_t)__builtin_amdgcn_readfirstlane(r.w2);
    g.hk = __builtin_amdgcn_readfirstlane(r.hk);
    g.hb = __builtin_amdgcn_readfirstlane(r.hb);
    g.pos = r.pos;
    g.p = r.p;
    g.c16 = r.c16;
    const bool row_ok = (g.page_off | g.th_off | g.rad_off) >= 0;
    const uint32_t po = g.page_off, tho = g.th_off, ro = g.rad_off;
    // the page's reads go through a resource of the pool's size (of none for
    // a bad row), so an offset past the pool reads zero by the buffer range
    // check alone, with no per-load select (the offsets, below 2^31 plus a
    // few KB, do not wrap)
    const rsrc_t rsp = make_rsrc(a.pages, row_ok ? (int64_t)pb : 0);
    auto dword_at = [&](uint32_t o4) {
      const uint32_t w = __builtin_amdgcn_raw_buffer_load_b32(rsp, (int)o4, 0, 0);
      return w | (row_ok && o4 == tail4 ? tailw : 0u);  // the partial dword itself reads as zero
    };
    g.cnt = __builtin_amdgcn_raw_buffer_load_b8(rsp, (int)(po + 1), 0, 0);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int gg = k ? gj : gi;
      const uint32_t x = 8u * (tho & 3u) + (uint32_t)((ts * G + gg) * b);   // bit offset from tho & ~3
      const uint32_t o4 = (tho & ~3u) + 4u * (x >> 5);
      g.cw[k][0] = dword_at(o4);
      g.cw[k][1] = dword_at(o4 + 4);
      g.rc[k] = (int)(int8_t)__builtin_amdgcn_raw_buffer_load_b8(rsp, (int)(ro + (uint32_t)(ts * G + gg)), 0, 0);
      const uint32_t s4 = (po + kHeaderBytes + 4 * gg) & ~3u;
      g.sw[k][0] = dword_at(s4);
      g.sw[k][1] = dword_at(s4 + 4);
    }
    if constexpr (RM == kRopeNone) {
      const int pos = (r.pos >= 0 && r.pos < a.max_pos) ? r.pos : 0;
      const float* cs = a.cos_tbl + (int64_t)pos * DH + d0;
      const float* sn = a.sin_tbl + (int64_t)pos * DH + d0;
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        cc[m] = *reinterpret_cast<const float4*>(cs + 4 * m);
        ss[m] = *reinterpret_cast<const float4*>(sn + 4 * m);
      }
    }
    return g;
  };
  const int64_t total_slots = (int64_t)a.num_pages * a.page_size;
  const float inv = 1.0f / __builtin_sqrtf((float)DH);
  int staged = -1;
  auto compute = [&](auto cb_lds_f, const RagPage& g, const float4 (&cc)[NM], const float4 (&ss)[NM])
                     __attribute__((always_inline)) {
    constexpr bool CB_LDS = decltype(cb_lds_f)::value;
    const int p = g.p, ts = 16 * g.c16 + t;
    const bool row_ok = (g.page_off | g.th_off | g.rad_off) >= 0;
    const uint32_t po = g.page_off, tho = g.th_off, ro = g.rad_off;
    const int hk = g.hk;
    int n = row_ok && po + 2 <= pb ? min((int)g.cnt, a.page_size) : 0;
    if (po + kHeaderBytes + 4 * G > pb || tho + (uint32_t)((n * G * b + 7) >> 3) > pb || ro + (uint32_t)(n * G) > pb)
      n = 0;
    const bool head_ok = hk >= 0 && hk < a.num_kv;
    const bool valid = ts < n && g.pos >= 0 && g.pos < a.max_pos && head_ok;
    const int hq = head_ok ? hk : 0;
    const int ppos = (g.pos >= 0 && g.pos < a.max_pos) ? g.pos : 0;
    int code[2];
    float rad[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int gg = k ? gj : gi;
      const uint32_t x = 8u * (tho & 3u) + (uint32_t)((ts * G + gg) * b);
      code[k] = (int)(__builtin_amdgcn_alignbit(g.cw[k][1], g.cw[k][0], x & 31u) & (uint32_t)(C - 1));
      const uint32_t so = po + kHeaderBytes + 4 * gg;
      const float sc = __builtin_bit_cast(float, __builtin_amdgcn_alignbyte(g.sw[k][1], g.sw[k][0], so & 3u));
      rad[k] = (float)g.rc[k] * sc * (1.0f / 127.0f);
    }
    // codebook rows of the two codes: swizzled rows in LDS, or the global table
    const int r1 = gi * C + code[0], r2 = gj * C + code[1];
    const int hbase = hq * G * C * GS;                   // floats; the codebook stays below 2^29 floats
    floatx4 acc[NHS];
#pragma unroll
    for (int hs = 0; hs < NHS; ++hs) acc[hs] = (floatx4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      float4 cv1, cv2;
      if constexpr (CB_LDS) {
        cv1 = *reinterpret_cast<const float4*>(cb_s + rag_cb_index<GS>(r1, off / 4 + m));
        cv2 = *reinterpret_cast<const float4*>(cb_s + rag_cb_index<GS>(r2, off / 4 + m));
      } else {
        cv1 = __builtin_bit_cast(float4,
                                 __builtin_amdgcn_raw_buffer_load_b128(rcb, 4 * (hbase + r1 * GS + off + 4 * m), 0, 0));
        cv2 = __builtin_bit_cast(float4,
                                 __builtin_amdgcn_raw_buffer_load_b128(rcb, 4 * (hbase + r2 * GS + off + 4 * m), 0, 0));
      }
      const float k1[4] = {rad[0] * cv1.x, rad[0] * cv1.y, rad[0] * cv1.z, rad[0] * cv1.w};
      const float k2[4] = {rad[1] * cv2.x, rad[1] * cv2.y, rad[1] * cv2.z, rad[1] * cv2.w};
      float co[4], si[4];
      if constexpr (RM == kRopeNone) {
        co[0] = cc[m].x; co[1] = cc[m].y; co[2] = cc[m].z; co[3] = cc[m].w;
        si[0] = ss[m].x; si[1] = ss[m].y; si[2] = ss[m].z; si[3] = ss[m].w;
      } else {
        float ivm[4];
        double frm[4];
        if constexpr (RM == kRopeFp32) {
          const float4 w = *reinterpret_cast<const float4*>(iv_s + d0 + 4 * m);
          ivm[0] = w.x; ivm[1] = w.y; ivm[2] = w.z; ivm[3] = w.w;
        } else {
          const double2 w0 = *reinterpret_cast<const double2*>(fr_s + d0 + 4 * m);
          const double2 w1 = *reinterpret_cast<const double2*>(fr_s + d0 + 4 * m + 2);
          frm[0] = w0.x; frm[1] = w0.y; frm[2] = w1.x; frm[3] = w1.y;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const double x = RM == kRopeExact ? (double)ppos * frm[e] : (double)((float)ppos * ivm[e]) * kInvTwoPi;
          const float2 z = turn_phasor(x);
          co[e] = z.x;
          si[e] = z.y;
        }
      }
      // q of the lane's head slot: the staged head's rows in LDS, another
      // head's from the global q (slots past grp read zeros)
      float4 q0v[NHS], q1v[NHS];
#pragma unroll
      for (int hs = 0; hs < NHS; ++hs) {
        const int slot = 4 * hs + (t & 3);
        if constexpr (CB_LDS) {
          const int qo = slot * QS + d0 + 4 * m;
          q0v[hs] = *reinterpret_cast<const float4*>(q_s + qo);
          q1v[hs] = *reinterpret_cast<const float4*>(q_s + qo + DH / 2);
        } else {
          const int qo = slot < a.grp ? 4 * ((hq * a.grp + slot) * DH + d0 + 4 * m) : kOOB;
          q0v[hs] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rq, qo, 0, 0));
          q1v[hs] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rq, qo == kOOB ? kOOB : qo + 2 * DH, 0, 0));
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x0 = k1[e] * co[e] - k2[e] * si[e];
        const float x1 = k2[e] * co[e] + k1[e] * si[e];
#pragma unroll
        for (int hs = 0; hs < NHS; ++hs) {
          const float qa = e == 0 ? q0v[hs].x : e == 1 ? q0v[hs].y : e == 2 ? q0v[hs].z : q0v[hs].w;
          const float qb = e == 0 ? q1v[hs].x : e == 1 ? q1v[hs].y : e == 2 ? q1v[hs].z : q1v[hs].w;
          acc[hs] = __builtin_amdgcn_mfma_f32_4x4x1f32(qa, x0, acc[hs], 0, 0, 0);
          acc[hs] = __builtin_amdgcn_mfma_f32_4x4x1f32(qb, x1, acc[hs], 0, 0, 0);
        }
      }
    }
#pragma unroll
    for (int hs = 0; hs < NHS; ++hs) {
      float s0 = acc[hs][0], s2 = acc[hs][2], s1 = acc[hs][1], s3 = acc[hs][3];
      swap32(s0, s2);
      swap32(s1, s3);
      float x = s0 + s2, y = s1 + s3;
      swap16(x, y);
      const float v = x + y;
      const int i = 4 * hs + u;
      if (i < a.grp)
        a.logits_out[(int64_t)i * total_slots + p * a.page_size + ts] =
            !fit_ok ? __builtin_nanf("") : valid ? v * inv : -INFINITY;
    }
  };
  // the codebook of head hb into LDS when it is not the staged one (a
  // workgroup-uniform decision: hb is the head of the iteration's first chunk)
  // the codebook (at most 32 KB) and the q rows (SLOTS x DH, at most 4 KB)
  // of head hb: every load issued before the barrier and the writes
  constexpr int CR4 = GS / 4, QR4 = DH / 4;
  const int cn4 = G * C * CR4;
  constexpr int QK = (SLOTS * QR4 + kRagThreads - 1) / kRagThreads;
  struct StageRegs { float4 cb[kStage4], q[QK]; };
  // The stage's addresses and predicates are formed at each stage (an opaque
  // copy of the thread index keeps the compiler from computing them once in
  // the prologue and holding them, with their predicates, in registers for
  // the whole kernel: a stage is rare, the registers are not).
  auto stage_load = [&](int hb, StageRegs& v) {
    int tx = threadIdx.x;
    asm volatile("" : "+v"(tx));
#pragma unroll
    for (int k = 0; k < kStage4; ++k) {
      const int i = tx + kRagThreads * k;
      v.cb[k] = __builtin_bit_cast(float4,
                                   __builtin_amdgcn_raw_buffer_load_b128(rcb, i < cn4 ? 16 * (hb * cn4 + i) : kOOB, 0, 0));
    }
#pragma unroll
    for (int k = 0; k < QK; ++k) {
      const int i = tx + kRagThreads * k, sl = i / QR4;
      const int src = (i < SLOTS * QR4 && sl < a.grp) ? 16 * ((hb * a.grp + sl) * QR4 + i % QR4) : kOOB;
      v.q[k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rq, src, 0, 0));
    }
  };
  auto stage_store = [&](const StageRegs& v) {
    int tx = threadIdx.x;
    asm volatile("" : "+v"(tx));
#pragma unroll
    for (int k = 0; k < kStage4; ++k) {
      const int i = tx + kRagThreads * k;
      if (i < cn4) *reinterpret_cast<float4*>(cb_s + rag_cb_index<GS>(i / CR4, i % CR4)) = v.cb[k];
    }
#pragma unroll
    for (int k = 0; k < QK; ++k) {
      const int i = tx + kRagThreads * k;
      if (i < SLOTS * QR4) *reinterpret_cast<float4*>(q_s + (i / QR4) * QS + 4 * (i % QR4)) = v.q[k];
    }
  };
  auto stageable = [&](int hb) { return hb != staged && hb >= 0 && hb < a.num_kv && C <= 64; };
  auto stage = [&](int hb) {
    if (!stageable(hb)) return;
    StageRegs v;
    stage_load(hb, v);
    __syncthreads();                                   // every wave is done with the previous head
    stage_store(v);
    __syncthreads();
    staged = hb;
  };

  // pipeline: rows two iterations ahead, page bytes (and, on the table
  // path, table rows) one ahead, in two register sets used alternately (the
  // loop is unrolled by two, so no register a load is still filling is
  // copied)
  RagRow ra = row_of(0), rb = row_of(1);
  float4 cca[NM], ssa[NM], ccb[NM], ssb[NM];
  RagPage ga = page_of(ra, 16 * ra.c16 + t, cca, ssa), gb;
  for (int it = 0; it < it1; it += 2) {
    gb = page_of(rb, 16 * rb.c16 + t, ccb, ssb);       // waits for rows it + 1 (and so for pages it)
    ra = row_of(it + 2);
    stage(ga.hb);
    if (q0 + kRagWaves * it + wave < q1) {
      if (ga.hk == staged) compute(Flag<true>(), ga, cca, ssa);
      else compute(Flag<false>(), ga, cca, ssa);
    }
    if (it + 1 >= it1) break;
    ga = page_of(ra, 16 * ra.c16 + t, cca, ssa);
    rb = row_of(it + 3);
    stage(gb.hb);
    if (q0 + kRagWaves * (it + 1) + wave < q1) {
      if (gb.hk == staged) compute(Flag<true>(), gb, ccb, ssb);
      else compute(Flag<false>(), gb, ccb, ssb);
    }
  }
}

// LDS bytes of ragged_pipe_kernel: the padded q rows (4 or 8 slots) and the
// codebook of one head.
inline int64_t ragged_pipe_lds(const RaggedLaunch& L) {
  const int64_t slots = L.grp > 4 ? 8 : 4;
  return 4 * (slots * (L.dh + 4) + (int64_t)L.dh * (1 << L.b_theta));
}

int launch_ragged(const RaggedLaunch& L, hipStream_t stream) {
  if (L.num_pages <= 0) return 0;
  // the fast forms take 32-bit offsets: byte pools below 2 GiB, slots below 2^29
  const bool fast = L.page_size % 16 == 0 && (L.group_size == 16 || L.group_size == 32) && L.grp <= 8 &&
                    L.groups * L.group_size == L.dh && L.pages_bytes <= 0x7FFFFFFFLL &&
                    (int64_t)L.num_pages * L.page_size * 4 <= 0x7FFFFF00LL;
  const int64_t cb_bytes = (int64_t)L.dh * (1 << L.b_theta) * 4;
  if (fast && L.b_theta <= 6 && cb_bytes <= 32768 && (int64_t)L.num_kv * L.grp * L.dh * 4 <= 0x7FFFFFFFLL) {
    const int64_t chunks = (int64_t)L.num_pages * (L.page_size / 16);
    const int64_t iters = (chunks + kRagWaves - 1) / kRagWaves;
    const size_t lds = (size_t)ragged_pipe_lds(L);
    const int rm = L.rope ? L.rope_model : kRopeNone;
    // one resident round of workgroups: as many per CU as registers and LDS
    // allow, 256 CUs
    auto launch = [&](const void* fn, void (*k)(RaggedLaunch)) {
      struct Occ { const void* fn; size_t lds; int per_cu; };
      thread_local Occ cache[8] = {};
      thread_local int next = 0;
      int per_cu = 0;
      for (const Occ& o : cache)
        if (o.fn == fn && o.lds == lds) per_cu = o.per_cu;
      if (per_cu == 0) {
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kRagThreads, lds) != hipSuccess) per_cu = 1;
        per_cu = per_cu < 1 ? 1 : per_cu > 4 ? 4 : per_cu;
        cache[next] = Occ{fn, lds, per_cu};
        next = (next + 1) % 8;
      }
      const int64_t cap = 256LL * per_cu;
      hipLaunchKernelGGL(k, dim3((unsigned)(iters < cap ? iters : cap)), dim3(kRagThreads), lds, stream, L);
    };
#define SPHKV_RAGGED_RM(D, S, N, R) \
    if (L.dh == D && L.group_size == S && (L.grp > 4) == (N == 2) && rm == R) \
      launch(reinterpret_cast<const void*>(&ragged_pipe_kernel<D, S, N, R>), &ragged_pipe_kernel<D, S, N, R>);
#define SPHKV_RAGGED(D, S, N) \
    SPHKV_RAGGED_RM(D, S, N, kRopeNone) SPHKV_RAGGED_RM(D, S, N, kRopeExact) SPHKV_RAGGED_RM(D, S, N, kRopeFp32)
    SPHKV_RAGGED(128, 16, 1) SPHKV_RAGGED(128, 16, 2) SPHKV_RAGGED(128, 32, 1) SPHKV_RAGGED(128, 32, 2)
    SPHKV_RAGGED(64, 16, 1) SPHKV_RAGGED(64, 16, 2) SPHKV_RAGGED(64, 32, 1) SPHKV_RAGGED(64, 32, 2)
#undef SPHKV_RAGGED
#undef SPHKV_RAGGED_RM
  } else if (fast) {
    const int64_t chunks = (int64_t)L.num_pages * (L.page_size / 16);
    const dim3 grid((unsigned)((chunks + 3) / 4));
#define SPHKV_RAGGED(D, S, N) \
    if (L.dh == D && L.group_size == S && (L.grp > 4) == (N == 2)) \
      hipLaunchKernelGGL((ragged_fast_kernel<D, S, N>), grid, dim3(256), 0, stream, L);
    SPHKV_RAGGED(128, 16, 1) SPHKV_RAGGED(128, 16, 2) SPHKV_RAGGED(128, 32, 1) SPHKV_RAGGED(128, 32, 2)
    SPHKV_RAGGED(64, 16, 1) SPHKV_RAGGED(64, 16, 2) SPHKV_RAGGED(64, 32, 1) SPHKV_RAGGED(64, 32, 2)
#undef SPHKV_RAGGED
  } else {
    if (L.dh == 128)
      hipLaunchKernelGGL(ragged_logits_kernel<128>, dim3((L.num_pages + 3) / 4), dim3(256), 0, stream, L);
    else
      hipLaunchKernelGGL(ragged_logits_kernel<64>, dim3((L.num_pages + 3) / 4), dim3(256), 0, stream, L);
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Every entry of HF-layout cos / sin tables [max_pos, dh] against both
// models of fit (its f and inv32 set): the largest deviation of each model
// over the first-half entries (evaluated with fp64 sine / cosine), and the
// entries whose second half is not a copy of the first.  Results are added
// to fit's counters with vector atomics, one per wave.
__global__ __launch_bounds__(256) void rope_check_kernel(const float* cos_tbl, const float* sin_tbl, int max_pos,
                                                         int dh, RopeFit* fit) {
  const int half = dh / 2;
  const int64_t total = (int64_t)max_pos * half;
  double da = 0.0, db = 0.0;
  int mism = 0;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int p = (int)(i / half), j = (int)(i % half);
    const float* cr = cos_tbl + (int64_t)p * dh;
    const float* sr = sin_tbl + (int64_t)p * dh;
    const float c0 = cr[j], c1 = cr[j + half], s0 = sr[j], s1 = sr[j + half];
    mism += (__float_as_uint(c0) != __float_as_uint(c1)) || (__float_as_uint(s0) != __float_as_uint(s1));
    double t = (double)p * fit->f[j];
    t -= floor(t);
    double sa, ca, sb, cb;
    sincospi(2.0 * t, &sa, &ca);
    const float a32 = (float)p * fit->inv32[j];
    sincos((double)a32, &sb, &cb);
    const double ea = fmax(fabs((double)c0 - ca), fabs((double)s0 - sa));
    const double eb = fmax(fabs((double)c0 - cb), fabs((double)s0 - sb));
    da = ea <= da ? da : ea;        // NaN entries make the deviation NaN (kept: not <=)
    db = eb <= db ? db : eb;
  }
  float fa = da <= 1e30 ? (float)da : INFINITY, fb = db <= 1e30 ? (float)db : INFINITY;
  for (int m = 32; m >= 1; m >>= 1) {
    fa = fmaxf(fa, shfl_xor(fa, m));
    fb = fmaxf(fb, shfl_xor(fb, m));
    mism += __shfl_xor(mism, m, 64);
  }
  if ((threadIdx.x & 63) == 0) {
    atomicMax(&fit->dev_bits[0], __float_as_uint(fa));
    atomicMax(&fit->dev_bits[1], __float_as_uint(fb));
    if (mism) atomicAdd(&fit->half_mismatch, mism);
  }
}

int launch_rope_check(const float* cos_tbl, const float* sin_tbl, int32_t max_pos, int32_t dh, RopeFit* fit,
                      hipStream_t stream) {
  const int64_t total = (int64_t)max_pos * (dh / 2);
  const int64_t blocks = (total + 255) / 256;
  if (blocks > 0)
    hipLaunchKernelGGL(rope_check_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, stream,
                       cos_tbl, sin_tbl, max_pos, dh, fit);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace sphkv
