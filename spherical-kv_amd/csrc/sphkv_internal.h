// Launch descriptors shared by the C-ABI layer (sphkv_capi.hip) and the
// kernel translation units.  Plain pointers and sizes only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sphkv {

struct EncodeLaunch {
  const void* k; int32_t k_is_fp32; const uint16_t* v; int64_t num_src_rows;
  const int64_t* src_rows; const int32_t* tier; const int32_t* count;
  const int32_t* ptable; const int32_t* vslot; const int32_t* seq_head;
  int32_t num_pages; int32_t num_kv;
  const float* cb1; const float* cb2; const float* cb3;
  uint8_t* pages; int64_t pages_bytes; uint16_t* v_pool; int64_t num_vpages;
  float* r_out; int32_t* code_out; int32_t dh;
  const int32_t* order_n;   // per page: N of the torch call whose summation order applies (NULL: count)
  int32_t codes_only;       // 1: write r_out / code_out only (no pages, no V)
};

struct DecodeLaunch {
  const uint8_t* pages; int64_t pages_bytes; const int32_t* ptable;
  const int32_t* vslot; const int32_t* positions; int32_t num_rows;
  const uint16_t* v_pool; int64_t num_vpages;
  const float* cb1; const float* cb2; const float* cb3;
  const int32_t* work; int32_t num_items; const int32_t* work_start;
  int32_t num_seqs; int32_t num_kv; int32_t gqa;
  const uint16_t* q; uint16_t* out; float* partials;
  int32_t dh; float sm_scale; double rope_theta;
};

// Decode-time tail of the Mode-B path (spherical_kv_pipeline.py:2248-2342,
// 2389-2475): per (sequence, kv head) up to kTailSlots - 1 staged tokens
// (tier-3 codes, fp32 radii, fp16 V, positions) and the step's new token.
// Decode page k of (seq, head) sh lives at bytes dec_byte0 + (sh * dec_cap +
// k) * tail_slot_bytes(dh) and V page dec_vpage0 + sh * dec_cap + k; its
// pointer-table row is the row after sh's last one (the work items' end_row),
// reserved with those offsets when the decode-time table was laid out.
constexpr int kTailSlots = 16;
constexpr int kTailDecode = 1;      // score the tail in the step's softmax, write out
constexpr int kTailAppend = 2;      // append the new token (flush a full page)
constexpr int kTailStateInts = 4;   // per (seq, head), twice (step parity): staged count, decode pages, dropped, 0
inline int tail_page_bytes(int dh) { return 8 + 26 * (dh / 32); }          // tier 3, 16 tokens
inline int tail_slot_bytes(int dh) { return (tail_page_bytes(dh) + 15) & ~15; }

struct TailLaunch {
  const void* k_new; int32_t k_is_fp32; const uint16_t* v_new; const int32_t* cur_pos;
  float* stg_r; int32_t* stg_code; uint16_t* stg_v; int32_t* stg_pos; int32_t* state;
  uint8_t* pages; int32_t* positions; uint16_t* v_pool; int32_t* work;
  int64_t dec_byte0; int32_t dec_cap, dec_vpage0;
  int32_t mode;
  int32_t parity;            // which copy of the tail counts this step reads
};

// A RoPE fitted to a caller's HF-layout cos / sin tables [max_pos, dh]
// (sphkv_rope_table_fit), in device memory.  Pair j (dims j, j + dh/2) turns
// by either model:
//   kRopeExact  cos / sin of the exact angle 2 pi pos f[j]  (f in turns per token)
//   kRopeFp32   cos / sin of the fp32 angle fl32(pos * inv32[j])  (the HF
//               construction: fp32 inv_freq times the fp32 position)
// model is the one every table entry follows within kRopeFitTol (kRopeNone:
// neither; the tables are read as given).
constexpr int kRopeNone = 0, kRopeExact = 1, kRopeFp32 = 2;
constexpr float kRopeFitTol = 0x1p-20f;
struct RopeFit {
  int32_t model, dh, max_pos, half_mismatch;   // half_mismatch: entries whose second half differs from the first
  uint32_t dev_bits[2];                        // max |table - model| of kRopeExact, kRopeFp32 (fp32 bits)
  int32_t pad[2];
  double f[64];
  float inv32[64];
};
static_assert(sizeof(RopeFit) <= 1024, "SPHKV_ROPE_FIT_BYTES");

struct RaggedLaunch {
  const uint8_t* pages; int64_t pages_bytes; const int32_t* ptable; const int32_t* head_ids;
  const int32_t* positions; int32_t num_pages; const float* cos_tbl; const float* sin_tbl;
  int32_t max_pos; const float* q; int32_t grp; int32_t num_kv; const float* codebooks;
  int32_t dh; int32_t groups; int32_t group_size; int32_t b_theta; int32_t page_size;
  float* logits_out;
  const RopeFit* rope;       // NULL, or the tables' fit (phases formed in the kernel)
  int32_t rope_model;        // kRopeNone when rope is NULL
};

// Mode-A (LayerPool) path
constexpr int kModeAMaxTiers = 8;

struct AppendLaunch {
  const float* k_post; const float* v_new; const float* decode_cb;
  uint8_t* theta_codes; uint8_t* radius_codes; float* r_scales; _Float16* v_pool;
  const int64_t* pids; int64_t num_pages;
  int32_t num_kv, slot, G, g, C, G_max, dh, page_size, is_new_page;
};

struct ModeALaunch {
  const float* q; const float* cb_flat; const int32_t* tier_G; const int32_t* tier_g;
  const uint8_t* theta_codes; const uint8_t* radius_codes; const float* r_scales; const _Float16* v_pool;
  const int32_t* block_table; const int32_t* bits_table;
  float* out; float* partial;
  int32_t num_q, num_kv, kv_groups, num_tiers, max_blocks, page_size, dh, G_max, cb_max, g_max;
  int64_t num_pages; float sm_scale;
  // set by modea_configure: nsplit ranges of logical pages per kv head (range s
  // = [s * max_blocks / nsplit, (s + 1) * max_blocks / nsplit)); fast = 1 selects
  // the vector-load kernel (G_max 4 or 8), 0 the general one
  int32_t nsplit, fast;
};

struct LutLogitsLaunch {
  const float* q_lut; const uint8_t* theta_codes; const uint8_t* radius_codes; const float* r_scales;
  const int32_t* block_table; const int32_t* bits_table; const int32_t* ctx_lens; float* logits_out;
  int32_t num_q, num_kv, kv_groups, num_tiers, max_blocks, page_size, G_max, cb_size_max, max_ctx;
  int64_t num_pages; float sm_scale;
};

constexpr int kOmegaMaxGroups = 64;
struct OmegaLaunch {
  const float* m; const float* l; int64_t q_stride, page_stride;   // element strides of the (m, l) views
  const float* omega_prev; float* omega_out;                        // [num_kv, max_blocks]; may alias
  int32_t num_kv, kv_groups, max_blocks; float beta;
};

constexpr int kPoolBuildMaxG = 256;
struct PoolBuildLaunch {
  const float* r; const int32_t* theta; int64_t n_elems;    // concatenated [rows, G_t] token arrays
  const _Float16* v; int64_t n_vrows;                       // concatenated fp16 V rows [rows, dh]
  const int32_t* page_src; int32_t n_pages, pid0;           // per page (r offset, V row, npg, G_t)
  uint8_t* theta_codes; uint8_t* radius_codes; float* r_scales; _Float16* v_pool;
  int32_t page_size, G_max, dh;
};

// Device page planning (sphkv_plan.hip)
struct PlanLaunch {
  const uint8_t* tier_of; int64_t tier_stride;   // [num_sh, >= L_s] tier id per token
  const int32_t* lens;                           // [num_seqs] tokens per sequence
  int32_t max_len;                               // >= every lens[s]: sizes the token chunks
  int32_t nchunks;                               // set by launch_plan
  const int32_t* pos; int64_t pos_stride;        // [num_seqs, >= L_s] positions, or null (token index)
  const int64_t* row_base;                       // [num_sh] K row of token 0, or null (no src_rows)
  int32_t num_sh, num_kv, dh;
  int32_t* work;                                 // plan_work_ints(num_sh, max_len) int32
  int32_t* totals;                               // [4]: rows, pool bytes (-1: >= 2 GiB), invalid ids, overflow
  int32_t* row_start;                            // [num_sh + 1]
  int32_t max_rows;                              // capacity of the per-row outputs
  // per row (capacity max_rows): written by the fill phase
  int32_t* tier; int32_t* count; int32_t* ptable; int32_t* seq_head; int32_t* vslot;
  int64_t* tokens; int32_t* positions; int64_t* src_rows;   // [rows, 16]; src_rows may be null
};
int launch_plan(const PlanLaunch& L, int phase, hipStream_t stream);
int64_t plan_work_ints(int num_sh, int max_len);

int launch_append(const AppendLaunch& L, hipStream_t stream);
int launch_omega(const OmegaLaunch& L, hipStream_t stream);
int launch_pool_build(const PoolBuildLaunch& L, hipStream_t stream);
int launch_modea(const ModeALaunch& L, hipStream_t stream);
int launch_qlut(const ModeALaunch& L, float* lut, hipStream_t stream);
int launch_lut_logits(const LutLogitsLaunch& L, hipStream_t stream);
// Chooses the kernel and the page split for a launch; returns the dynamic
// LDS bytes the chosen split kernel needs (callers reject > 160 KiB).
int64_t modea_configure(ModeALaunch& L);

int launch_encode(const EncodeLaunch& L, hipStream_t stream);
// Decode phases: the split kernel writing one (m, l, acc) partial per work
// item, and the log-sum-exp merge of each (sequence, kv head)'s partials.
constexpr int kPhasePartials = 1;
constexpr int kPhaseMerge = 2;
int launch_decode(const DecodeLaunch& L, int phases, hipStream_t stream);
// The decode kernel over prefill + decode-page rows (mode & kTailDecode),
// then the tail kernel: merge, tail terms, output, append / flush.
int launch_decode_tail(const DecodeLaunch& L, const TailLaunch& T, hipStream_t stream);
// The next decode_kernel launch on this thread records its start / stop in
// these events (kernel-only timestamps, hipExtLaunchKernel).
void set_decode_timing(hipEvent_t start, hipEvent_t stop);
int launch_tail_relayout(const int32_t* row_start, int32_t num_sh, int32_t num_rows, const int32_t* ptable,
                         const int32_t* vslot, const int32_t* positions, int32_t dec_cap, int64_t dec_byte0,
                         int32_t dec_vpage0, int32_t dh, int32_t* ptable_d, int32_t* vslot_d,
                         int32_t* positions_d, hipStream_t stream);
int launch_ragged(const RaggedLaunch& L, hipStream_t stream);
// check every table entry against both models of *fit (f / inv32 set); adds
// to fit's half_mismatch and dev_bits (which start at zero)
int launch_rope_check(const float* cos_tbl, const float* sin_tbl, int32_t max_pos, int32_t dh, RopeFit* fit,
                      hipStream_t stream);

// fp32 elements of one work item's partial: 16 (m, l, padding) + gqa * dh
inline int64_t partial_floats(int gqa, int dh) { return 16 + (int64_t)gqa * dh; }
// The decode workspace ends with 16 status bytes after the partials: uint32
// [0] malformed rows / pages counted by the decode kernel since the last
// merge, [1] the count the last merge saw.
constexpr int64_t kDecodeStatusBytes = 16;
inline int64_t decode_workspace_bytes(int num_items, int gqa, int dh) {
  return (int64_t)num_items * partial_floats(gqa, dh) * 4 + kDecodeStatusBytes;
}


}  // namespace sphkv
