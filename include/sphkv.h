/*
 * sphkv.h -- C ABI of libsphkv.so, the MI355X (gfx950) angle-domain
 * compressed-KV library.
 *
 * Every entry point takes device pointers, plain integer sizes and a HIP
 * stream (hipStream_t passed as void*; NULL = the null stream), launches
 * asynchronously on that stream and returns 0 on success or a negative
 * SPHKV_E* code.  The caller owns every buffer, outputs included, as in the
 * reference (decode_kernel.cu:249-289 writes through the caller's tensors).
 * sphkv_last_error() returns a message for the last failure on the calling
 * thread.
 *
 * Data layout (all little-endian):
 *   pages      uint8 byte pool holding pagebuilder pages (pagebuilder.py:8-33):
 *              u8 tier id | u8 count | 6 zero bytes | G fp32 radius scales |
 *              LSB-first packed theta codes | int8 radius codes.
 *              Dense fp16 K pages use tier id 0xFF, no scales, and hold the
 *              page's pre-RoPE K rows as fp16 [count, dh] in the theta section.
 *   ptable     int32 [P, 3] rows (page_off, theta_off, radius_off)
 *              (pointer_table.py:4-21, spherical_kv_pipeline.py:1202-1213).
 *   positions  int32 [P, page_size] absolute token positions, -1 = pad.
 *   v_pool     fp16 V pages, token-minor: element (d, t) of V page v at
 *              ((v * dh) + d) * page_size + t.  vslot[p] is row p's V page.
 *   codebooks  per tier id 1..3: fp32 [num_kv, G, C, g] (unit rows).
 *   Tier geometry is tiers.py:35-41: tier 1 g=16 b=6 C=64, tier 2 g=16 b=4
 *   C=16, tier 3 g=32 b=3 C=8.
 *
 * RoPE convention of the decode kernels: default RoPE (no scaling), HF
 * rotate_half pairing (j, j + dh/2), inv_freq_j = theta^(-2j/dh); the phase
 * position * inv_freq_j is formed in fp64 and reduced modulo one turn before
 * the fp32 sine / cosine.
 */
#ifndef SPHKV_H
#define SPHKV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SPHKV_OK 0
#define SPHKV_EINVAL (-1)   /* bad argument (shape, size, alignment, null) */
#define SPHKV_ELAUNCH (-2)  /* a kernel launch failed */
#define SPHKV_EDEVICE (-3)  /* no usable device / wrong architecture */

/* Message for the last failure on this thread ("" if none). */
const char* sphkv_last_error(void);

/* Library version, e.g. "sphkv 0.1 gfx950". */
const char* sphkv_version(void);

/*
 * Fused encode + bitpack + page build + V placement.
 * Replaces, for whole pages, the prefill chain
 *   _encode_keys_with_codebooks  spherical_kv_pipeline.py:1130-1144
 *   build_page_from_codes/build_page  pagebuilder.py:8-42
 *   PageHeader.to_tensor  paging.py:20-31,  pack_bits  bitpacking.py:5-29
 * as called per chunk by _build_per_head_pages (spherical_kv_pipeline.py:1187-1213).
 * Codes, radii and page bytes are bit-exact with the torch CPU execution of
 * those lines.
 *
 *   k, v        [num_src_rows, dh] source rows; k is fp16 (k_is_fp32 = 0)
 *               or fp32 (k_is_fp32 = 1), v is fp16.
 *   src_rows    int64 [P, page_size] source row of each page slot (-1 = pad).
 *   tier,count  int32 [P] tier id (1,2,3,0xFF) and tokens in each page.
 *   ptable      int32 [P, 3] where each page goes (written by this call).
 *   vslot       int32 [P] V page of each row.  seq_head int32 [P]: codebook
 *               head of a row is seq_head[p] % num_kv.
 *   r_out       optional fp32 [P, page_size, dh/16] group radii (NULL = skip)
 *   code_out    optional int32 [P, page_size, dh/16] codes (NULL = skip)
 * dh in {64, 128}; page_size == 16.
 */
int sphkv_encode_pages(const void* k, int32_t k_is_fp32, const uint16_t* v, int64_t num_src_rows,
                       const int64_t* src_rows, const int32_t* tier, const int32_t* count,
                       const int32_t* ptable, const int32_t* vslot, const int32_t* seq_head,
                       int32_t num_pages, int32_t num_kv,
                       const float* cb1, const float* cb2, const float* cb3,
                       uint8_t* pages, int64_t pages_bytes, uint16_t* v_pool, int64_t num_vpages,
                       float* r_out, int32_t* code_out, int32_t dh, int32_t page_size, void* stream);

/*
 * Workspace bytes sphkv_decode_paged needs for num_items work items: one
 * (m, l, acc) partial per item.  No initialisation is needed; calls that share
 * a workspace must not run concurrently.
 */
int64_t sphkv_decode_paged_workspace_bytes(int32_t num_items, int32_t gqa, int32_t dh);

/*
 * Angle-domain paged attention decode (the north-star path): per (sequence,
 * kv head), walks its pointer-table rows, streams packed codes, int8 radii,
 * dense fp16 K and fp16 V, rotates the reconstructed key r_hat * centroid by
 * each token's RoPE angle (equivalently back-rotates q, as
 * spherical_kv_pipeline.py:2143-2151 does), forms
 *   logit = sum_g r_hat_g <q_rot_g, c_g> / sqrt(dh)        (:2158-2176)
 * (dense pages: <q_rot, k> / sqrt(dh)), and runs the softmax over all tokens
 * (:2347-2348) and attn @ V (:2364-2367) as one online softmax.  Replaces the
 * per-head torch path _compressed_head_attention_batched (:2057-2369) for its
 * page-resident context and the missing fused_decode_ragged kernel's callers
 * (:1102-1125, :1865-1870).
 *
 *   work       host-computed work list: work int32 [num_items, 3] =
 *              (seq*num_kv + head, row_begin, row_end) with the items of one
 *              (seq, head) contiguous and in order, and at least one item
 *              (possibly empty) per (seq, head); work_start int32
 *              [num_seqs*num_kv + 1] = first item of each (seq, head).
 *   q          fp16 [num_seqs, num_kv*gqa, dh];  out fp16, same shape.
 *   workspace  device scratch of sphkv_decode_paged_workspace_bytes() bytes.
 * gqa in {1, 2, 4, 8}; dh in {64, 128}; page_size == 16.
 */
int sphkv_decode_paged(const uint8_t* pages, int64_t pages_bytes, const int32_t* ptable,
                       const int32_t* vslot, const int32_t* positions, int32_t num_rows,
                       const uint16_t* v_pool, int64_t num_vpages,
                       const float* cb1, const float* cb2, const float* cb3,
                       const int32_t* work, int32_t num_items, const int32_t* work_start,
                       int32_t num_seqs, int32_t num_kv, int32_t gqa,
                       const uint16_t* q, uint16_t* out, void* workspace, int64_t workspace_bytes,
                       int32_t dh, int32_t page_size, float sm_scale, double rope_theta,
                       void* stream);

/*
 * The two phases of sphkv_decode_paged as separate calls, for callers that
 * combine partials themselves (a context split over several devices, each
 * merging the gathered partials) or time the phases apart.  No reference
 * counterpart: the reference's Mode-A split/reduce pair
 * (decode_kernel.cu:108-246) is internal to its single entry point.
 *
 * sphkv_decode_paged_partials: the arguments of sphkv_decode_paged without
 * the output; writes one partial per work item into the workspace:
 *   float [num_items][16 + gqa*dh]: m[gqa], l[gqa], 16 - 2*gqa unused,
 *   acc[gqa][dh];  m = running max of logit * sm_scale * log2(e) (log2
 *   domain, -inf for an empty item), l = sum of 2^(s - m), acc = sum of
 *   2^(s - m) * V (unnormalised).
 * sphkv_decode_merge_partials: out[seq, head*gqa + i, :] = sum_items
 *   2^(m - M) acc / sum_items 2^(m - M) l over the items of work_start's
 *   ranges (zeros where every item is empty).
 */
int sphkv_decode_paged_partials(const uint8_t* pages, int64_t pages_bytes, const int32_t* ptable,
                                const int32_t* vslot, const int32_t* positions, int32_t num_rows,
                                const uint16_t* v_pool, int64_t num_vpages,
                                const float* cb1, const float* cb2, const float* cb3,
                                const int32_t* work, int32_t num_items, const int32_t* work_start,
                                int32_t num_seqs, int32_t num_kv, int32_t gqa,
                                const uint16_t* q, void* workspace, int64_t workspace_bytes,
                                int32_t dh, int32_t page_size, float sm_scale, double rope_theta,
                                void* stream);
int sphkv_decode_merge_partials(const void* workspace, int64_t workspace_bytes, int32_t num_items,
                                const int32_t* work_start, int32_t num_seqs, int32_t num_kv,
                                int32_t gqa, int32_t dh, uint16_t* out, void* stream);

/*
 * Logits-only ragged kernel with the contract of the reference's missing
 * fused_decode_ragged (call sites spherical_kv_pipeline.py:1102-1125,
 * :1865-1870, :1906-1910): pages of one tier, RoPE from the caller's HF-layout
 * cos/sin tables [max_pos, dh] fp32.
 *   logits_out fp32 [grp, num_pages*page_size]; element (i, p*page_size+s) is
 *   q-head head_ids[p]*grp + i against slot s of page p; pad slots
 *   (position < 0 or s >= page count) are -inf.
 *   codebooks fp32 [num_kv*groups, C, group_size]; q fp32 [num_kv*grp, dh].
 * page_size <= 128.
 */
int sphkv_fused_decode_ragged(const uint8_t* pages, int64_t pages_bytes, const int32_t* ptable,
                              const int32_t* head_ids, const int32_t* positions, int32_t num_pages,
                              const float* cos_tbl, const float* sin_tbl, int32_t max_pos,
                              const float* q, int32_t grp, int32_t num_kv, const float* codebooks,
                              int32_t dh, int32_t groups, int32_t group_size, int32_t b_theta,
                              int32_t page_size, float* logits_out, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* SPHKV_H */
