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

struct RaggedLaunch {
  const uint8_t* pages; int64_t pages_bytes; const int32_t* ptable; const int32_t* head_ids;
  const int32_t* positions; int32_t num_pages; const float* cos_tbl; const float* sin_tbl;
  int32_t max_pos; const float* q; int32_t grp; int32_t num_kv; const float* codebooks;
  int32_t dh; int32_t groups; int32_t group_size; int32_t b_theta; int32_t page_size;
  float* logits_out;
};

int launch_encode(const EncodeLaunch& L, hipStream_t stream);
// Decode phases: the split kernel writing one (m, l, acc) partial per work
// item, and the log-sum-exp merge of each (sequence, kv head)'s partials.
constexpr int kPhasePartials = 1;
constexpr int kPhaseMerge = 2;
int launch_decode(const DecodeLaunch& L, int phases, hipStream_t stream);
int launch_ragged(const RaggedLaunch& L, hipStream_t stream);

// fp32 elements of one work item's partial: 16 (m, l, padding) + gqa * dh
inline int64_t partial_floats(int gqa, int dh) { return 16 + (int64_t)gqa * dh; }


}  // namespace sphkv
