/*
 * sphkv.h -- C ABI of libsphkv.so, the MI355X (gfx950) angle-domain
 * compressed-KV library.
 *
 * Every entry point takes device pointers, plain integer sizes and a HIP
 * stream (hipStream_t passed as void*; NULL = the null stream), launches
 * asynchronously on that stream and returns 0 on success or a negative
 * SPHKV_E* code (the two host-side work-list routines at the end take host
 * pointers and no stream).  The caller owns every buffer, outputs included, as in the
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
#define SPHKV_EPAGE (-4)    /* the decode skipped malformed pointer-table rows or pages */

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
 * Radii and codes only, for every token of every tier: the all-tier
 * re-encode kept for the online refresh (_codes_all,
 * spherical_kv_pipeline.py:1536-1553), which encodes each (layer, head)'s T
 * tokens at each tier in one _encode_keys_with_codebooks call (:1130-1144).
 * The tokens are given as pages of sphkv_encode_pages (src_rows, tier,
 * count, seq_head; no pointer table, byte pool or V), and order_n[p] is the
 * N of the torch call whose summation order the page's codes follow (its
 * head's T; NULL: the page's count).  r_out fp32 / code_out int32
 * [num_pages, page_size, dh/16] get each (token, group) of the compressed
 * pages (groups past the tier's G untouched); codes are bit-exact with torch
 * CPU's call over order_n tokens.
 */
int sphkv_encode_codes(const void* k, int32_t k_is_fp32, int64_t num_src_rows, const int64_t* src_rows,
                       const int32_t* tier, const int32_t* count, const int32_t* order_n, const int32_t* seq_head,
                       int32_t num_pages, int32_t num_kv, const float* cb1, const float* cb2, const float* cb3,
                       float* r_out, int32_t* code_out, int32_t dh, int32_t page_size, void* stream);

/*
 * Workspace bytes sphkv_decode_paged needs for num_items work items: one
 * (m, l, acc) partial per item, then 16 status bytes (uint32 [0]: malformed
 * rows / pages counted since the last merge, [1]: the count of the last
 * merged decode).  Zero the workspace once when it is allocated (the status
 * words must start at zero); calls that share a workspace must not run
 * concurrently.
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
 *   work       host-computed work list: work int32 [num_items, 4] =
 *              (seq*num_kv + head, first_row, end_row, stride): the item
 *              covers rows first_row, first_row + stride, ... < end_row
 *              (stride >= 1; contiguous items use 1).  The items of one
 *              (seq, head) are contiguous in the list, together cover each
 *              of its rows once, and there is at least one item (possibly
 *              empty) per (seq, head); work_start int32
 *              [num_seqs*num_kv + 1] = first item of each (seq, head).
 *   q          fp16 [num_seqs, num_kv*gqa, dh];  out fp16, same shape.
 *   workspace  device scratch of sphkv_decode_paged_workspace_bytes() bytes.
 * gqa in {1, 2, 4, 8}; dh in {64, 128}; page_size == 16; pages_bytes a
 * multiple of 4 (the pool is read in dwords: pad a back-to-back pool).
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
 * sphkv_decode_paged without the workspace arguments, for callers that cannot
 * allocate (code under HIP graph capture, serving loops or harnesses that
 * forbid hipMalloc).  No reference counterpart.  The partials and status words
 * live in a device array of the library (SPHKV_NOALLOC_SCRATCH_BYTES per GPU,
 * held until the process ends); the call allocates nothing and returns
 * SPHKV_EINVAL when sphkv_decode_paged_workspace_bytes(num_items, gqa, dh)
 * exceeds that size (8 MiB: 3,971 work items at gqa 4 / dh 128, 2,016 at
 * gqa 8).  All calls on one GPU share that GPU's array: calls that overlap
 * on one GPU (several streams or threads) race.  Results equal
 * sphkv_decode_paged's on the same inputs.  Malformed pages are skipped as
 * there, without a report (sphkv_decode_paged_checked reports them).
 */
#define SPHKV_NOALLOC_SCRATCH_BYTES (8 << 20)
int sphkv_decode_paged_noalloc(const uint8_t* pages, int64_t pages_bytes, const int32_t* ptable,
                               const int32_t* vslot, const int32_t* positions, int32_t num_rows,
                               const uint16_t* v_pool, int64_t num_vpages,
                               const float* cb1, const float* cb2, const float* cb3,
                               const int32_t* work, int32_t num_items, const int32_t* work_start,
                               int32_t num_seqs, int32_t num_kv, int32_t gqa,
                               const uint16_t* q, uint16_t* out,
                               int32_t dh, int32_t page_size, float sm_scale, double rope_theta,
                               void* stream);

/*
 * Malformed input.  The decode never reads outside the buffers it is given;
 * a pointer-table row that does not address the pools, a page whose tier id
 * is not 1, 2, 3 or 0xFF, a count above page_size, a non-empty dense page
 * whose K rows are not 16-byte aligned inside its theta section, or a compressed page
 * whose sections leave the byte pool (or the 512 bytes from its page's 16-byte
 * line) contributes no token, and is counted in the workspace's status word.
 *
 * sphkv_decode_paged_status: waits for `stream` and returns in *malformed the
 * count of the last merged decode on this workspace (0 for a well-formed pool).
 * sphkv_decode_paged_checked: sphkv_decode_paged followed by that wait;
 * returns SPHKV_EPAGE when the count is non-zero (the output is still written,
 * without the skipped pages).  Neither has a reference counterpart: the
 * reference launches without any check (decode_kernel.cu:262-288).
 */
int sphkv_decode_paged_status(const void* workspace, int64_t workspace_bytes, int32_t num_items, int32_t gqa,
                              int32_t dh, int32_t* malformed, void* stream);
int sphkv_decode_paged_checked(const uint8_t* pages, int64_t pages_bytes, const int32_t* ptable,
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
 * A bound paged decode, no reference counterpart: every argument of
 * sphkv_decode_paged but q, out and the stream, checked once at creation;
 * each sphkv_decode_plan_run then launches the decode (partials and merge)
 * with no further argument checks.  For serving loops whose per-call host
 * cost matters (the reference's decode is one Python call per layer,
 * spherical_kv_pipeline.py:2057).  The plan holds the pointers it was given:
 * the buffers must outlive it and keep their sizes.  A plan may be run from
 * several threads; runs that share its workspace must not overlap on the
 * device (use one stream, or one plan per stream).
 */
typedef struct sphkv_decode_plan sphkv_decode_plan;
int sphkv_decode_plan_create(const uint8_t* pages, int64_t pages_bytes, const int32_t* ptable,
                             const int32_t* vslot, const int32_t* positions, int32_t num_rows,
                             const uint16_t* v_pool, int64_t num_vpages,
                             const float* cb1, const float* cb2, const float* cb3,
                             const int32_t* work, int32_t num_items, const int32_t* work_start,
                             int32_t num_seqs, int32_t num_kv, int32_t gqa, void* workspace,
                             int64_t workspace_bytes, int32_t dh, int32_t page_size, float sm_scale,
                             double rope_theta, sphkv_decode_plan** plan_out);
int sphkv_decode_plan_run(const sphkv_decode_plan* plan, const uint16_t* q, uint16_t* out, void* stream);
void sphkv_decode_plan_destroy(sphkv_decode_plan* plan);

/*
 * Measurement hook, no reference counterpart: the next launch of the paged
 * decode kernel on the calling thread (by sphkv_decode_paged, _checked,
 * _partials, _noalloc or sphkv_decode_step) records its own start and stop
 * time in the two hipEvent_t the caller created (hipExtLaunchKernel), so
 * hipEventElapsedTime gives that kernel's duration without the gaps between
 * launches, the figure rocprofv3's kernel trace reports.  NULL, NULL cancels.
 */
int sphkv_time_next_decode_kernel(void* start_event, void* stop_event);

/*
 * ---- Decode-time tail of the Mode-B path ---------------------------------
 * A full decode step of the reference: _compressed_head_attention_batched
 * (spherical_kv_pipeline.py:2057-2369; multi-head form _decode_layer_all_heads
 * :1755-2055) scores the page-resident context, the tokens staged since the
 * last decode page (:2248-2285, fp32 radii) and the step's own token (:2294-
 * 2342, its pre-RoPE key encoded through the tier-3 codebook at current_pos)
 * in one softmax (:2347-2348) and attn @ V (:2364-2367, the new token's V =
 * v_new); then _append_decode_kv (:2389-2448) stages the new token (tier-3
 * encode, N = 1) and, at page_size staged tokens, _flush_decode_page
 * (:2449-2475) turns them into a tier-3 pagebuilder page
 * (build_page_from_codes, pagebuilder.py:36-42) that later steps read as
 * context.
 *
 * Tail state, per (sequence, kv head) sh = seq * num_kv + head, G3 = dh/32:
 *   stg_r     fp32  [num_sh, 16, G3]   staged radii (unquantised)
 *   stg_code  int32 [num_sh, 16, G3]   staged tier-3 codes
 *   stg_v     fp16  [num_sh, 16, dh]   staged V rows
 *   stg_pos   int32 [num_sh, 16]       staged positions
 *   tail_state int32 [num_sh, 2, 4]    two copies of (staged count 0..15,
 *                                       decode pages flushed, tokens dropped
 *                                       for want of a decode slot, 0); zero
 *                                       it to start.  A step reads copy
 *                                       step_parity, and an appending step
 *                                       writes the other copy (so the
 *                                       workgroups of one launch never see
 *                                       each other's update): pass
 *                                       step_parity = appending steps so far
 *                                       mod 2
 * Decode pages: sh's page k (k < dec_cap) is written at pages + dec_byte0 +
 * (sh * dec_cap + k) * slot (slot = 16-byte aligned size of a 16-token tier-3
 * page: 112 bytes at dh 128, 64 at dh 64), its V at V page dec_vpage0 +
 * sh * dec_cap + k, and its positions into the pointer-table row after sh's
 * last one; the work items of sh then cover that row (their end_row grows by
 * one).  The pointer table, vslot and positions must be the decode-time
 * layout of sphkv_tail_relayout, and the work list (work int32 [n, 4],
 * work_start) must cover each sh's prefill rows in that layout.
 */

/*
 * The decode-time pointer table: the prefill table (row_start int32
 * [num_sh + 1] on the device, ptable, vslot, positions of num_rows rows) with
 * dec_cap reserved rows after each (seq, head)'s rows: prefill row p of sh
 * moves to p + sh * dec_cap, reserved row k of sh is row row_start[sh + 1] +
 * sh * dec_cap + k, pointing at sh's decode page k (offsets as above, tier-3
 * sections of 16 tokens), positions -1.  Outputs: ptable_d int32
 * [num_rows + num_sh*dec_cap, 3], vslot_d, positions_d of as many rows.  No
 * reference counterpart (the reference keeps each flushed page as its own
 * tensor, spherical_kv_pipeline.py:2487-2495).
 */
int sphkv_tail_relayout(const int32_t* row_start, int32_t num_sh, int32_t num_rows, const int32_t* ptable,
                        const int32_t* vslot, const int32_t* positions, int32_t dec_cap, int64_t dec_byte0,
                        int32_t dec_vpage0, int32_t dh, int32_t* ptable_d, int32_t* vslot_d, int32_t* positions_d,
                        void* stream);

/*
 * One decode step: sphkv_decode_paged over the decode-time table (prefill
 * pages and flushed decode pages), with the staged tokens and the new token
 * in the same softmax; then, when append = 1, the new token is staged (and a
 * full page flushed).  k_new [num_sh, dh] pre-RoPE (fp16, or fp32 with
 * k_is_fp32 = 1), v_new fp16 [num_sh, dh], cur_pos int32 [num_seqs] (the new
 * token's position).  pages, positions, v_pool and work are written by a
 * flush.  The new token's codes and radii are bit-exact with
 * _encode_keys_with_codebooks on one token; the output is within the decode's
 * tolerance of the reference formula.  Other arguments as sphkv_decode_paged.
 */
int sphkv_decode_step(uint8_t* pages, int64_t pages_bytes, const int32_t* ptable, const int32_t* vslot,
                      int32_t* positions, int32_t num_rows, uint16_t* v_pool, int64_t num_vpages,
                      const float* cb1, const float* cb2, const float* cb3,
                      int32_t* work, int32_t num_items, const int32_t* work_start,
                      int32_t num_seqs, int32_t num_kv, int32_t gqa,
                      const uint16_t* q, const void* k_new, int32_t k_is_fp32, const uint16_t* v_new,
                      const int32_t* cur_pos, float* stg_r, int32_t* stg_code, uint16_t* stg_v, int32_t* stg_pos,
                      int32_t* tail_state, int64_t dec_byte0, int32_t dec_vpage0, int32_t dec_cap, int32_t append,
                      int32_t step_parity, uint16_t* out, void* workspace, int64_t workspace_bytes,
                      int32_t dh, int32_t page_size, float sm_scale, double rope_theta, void* stream);

/*
 * A bound decode step (no reference counterpart: the reference re-derives
 * its tensors in Python every step).  sphkv_step_plan_create validates every
 * static argument of sphkv_decode_step once (same meaning; staged / flushed
 * give the tail's current counts and step_parity, 0 for a fresh tail) and
 * keeps them with the host's mirror of the tail counts and parity; sphkv_step_plan_run then takes only
 * the per-step inputs: mode 1 = decode (no append), 2 = append only
 * (sphkv_decode_append), 3 = decode and append.  A run that would need a
 * decode page past dec_cap fails (SPHKV_EINVAL) before launching.  Runs of
 * one plan must be issued from one thread at a time.
 */
typedef struct sphkv_step_plan sphkv_step_plan;
int sphkv_step_plan_create(uint8_t* pages, int64_t pages_bytes, const int32_t* ptable, const int32_t* vslot,
                           int32_t* positions, int32_t num_rows, uint16_t* v_pool, int64_t num_vpages,
                           const float* cb1, const float* cb2, const float* cb3,
                           int32_t* work, int32_t num_items, const int32_t* work_start,
                           int32_t num_seqs, int32_t num_kv, int32_t gqa,
                           float* stg_r, int32_t* stg_code, uint16_t* stg_v, int32_t* stg_pos, int32_t* tail_state,
                           int64_t dec_byte0, int32_t dec_vpage0, int32_t dec_cap, int32_t staged, int32_t flushed,
                           int32_t step_parity, void* workspace, int64_t workspace_bytes, int32_t dh,
                           int32_t page_size, float sm_scale, double rope_theta, sphkv_step_plan** plan_out);
int sphkv_step_plan_run(sphkv_step_plan* plan, const uint16_t* q, const void* k_new, int32_t k_is_fp32,
                        const uint16_t* v_new, const int32_t* cur_pos, uint16_t* out, int32_t mode, void* stream);
int sphkv_step_plan_counts(const sphkv_step_plan* plan, int32_t* staged, int32_t* flushed, int32_t* step_parity);
void sphkv_step_plan_destroy(sphkv_step_plan* plan);

/*
 * _append_decode_kv alone (spherical_kv_pipeline.py:2389-2448, flush
 * :2449-2475): stages every (seq, head)'s new token, flushing full pages, with
 * no attention.  Arguments as sphkv_decode_step.
 */
int sphkv_decode_append(uint8_t* pages, int64_t pages_bytes, int32_t* positions, int32_t num_rows,
                        uint16_t* v_pool, int64_t num_vpages, const float* cb3,
                        int32_t* work, int32_t num_items, const int32_t* work_start, int32_t num_seqs,
                        int32_t num_kv, const void* k_new, int32_t k_is_fp32, const uint16_t* v_new,
                        const int32_t* cur_pos, float* stg_r, int32_t* stg_code, uint16_t* stg_v, int32_t* stg_pos,
                        int32_t* tail_state, int64_t dec_byte0, int32_t dec_vpage0, int32_t dec_cap,
                        int32_t step_parity, int32_t dh, int32_t page_size, void* stream);

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

/*
 * RoPE tables checked once, phases formed in the kernel.  No reference
 * counterpart: the reference's callers pass the same cos / sin tables to
 * every call (spherical_kv_pipeline.py:1102-1125, built once by
 * _ensure_rope_tables :1591-1610 from the model's rotary embedding), and
 * reading a row of each per token is the ragged kernel's largest read.
 *
 * sphkv_rope_table_fit: fits the tables [max_pos, dh] (HF layout: the second
 * half of a row repeats the first) to a rotation per pair j and checks every
 * entry on the device; waits for `stream`.  *model:
 *   0  no fit: some entry is off both models by more than 2^-20, or a row's
 *      halves differ (the tables are read as given)
 *   1  cos / sin of exact angles 2 pi pos f_j (f_j fitted, fp64)
 *   2  cos / sin of fp32 angles fl32(pos * inv_j) (inv_j fitted, fp32): the
 *      HF construction, fp32 inv_freq times the fp32 position
 * (model 1 is preferred when both hold).  fit: device memory of
 * SPHKV_ROPE_FIT_BYTES, written with the frequencies; max_dev (host float[2],
 * may be NULL): the largest deviation of models 1 and 2.  The fit describes
 * the tables' contents at the time of the call: fit again after they change.
 *
 * sphkv_fused_decode_ragged_fitted: sphkv_fused_decode_ragged with the tables'
 * fit: rope_model 1 or 2 (the model returned) forms each token's phases from
 * it instead of reading the table rows (results within about 1e-6 of the
 * table path's per logit unit); 0 reads the tables (rope_fit may be NULL).
 * A fit of another model, dh or max_pos makes every logit NaN.
 */
#define SPHKV_ROPE_FIT_BYTES 1024
int sphkv_rope_table_fit(const float* cos_tbl, const float* sin_tbl, int32_t max_pos, int32_t dh, void* fit,
                         int32_t* model, float* max_dev, void* stream);
int sphkv_fused_decode_ragged_fitted(const uint8_t* pages, int64_t pages_bytes, const int32_t* ptable,
                                     const int32_t* head_ids, const int32_t* positions, int32_t num_pages,
                                     const float* cos_tbl, const float* sin_tbl, int32_t max_pos,
                                     const float* q, int32_t grp, int32_t num_kv, const float* codebooks,
                                     int32_t dh, int32_t groups, int32_t group_size, int32_t b_theta,
                                     int32_t page_size, const void* rope_fit, int32_t rope_model,
                                     float* logits_out, void* stream);

/*
 * ---- Mode-A (LayerPool) path -------------------------------------------
 * Unpacked pools as sphkv_lut.py:71-80 builds them:
 *   theta_codes, radius_codes  uint8 [num_pages, page_size, G_max]
 *   r_scales                   fp32  [num_pages, G_max]
 *   v_pool                     fp16  [num_pages, page_size, dh] (token-major)
 *   block_table, bits_table    int32 [num_kv, max_blocks]: pool page (-1 =
 *                              none) and tier index of each logical page
 *   cb_flat                    fp32  [num_kv, num_tiers, G_max, cb_max, g_max]
 *   tier_G, tier_g             int32 [num_tiers]
 * Radius r_hat = r_scale * code / 255.  No RoPE: q and the encoded keys are
 * post-RoPE.
 */

/*
 * Decode-time single-token encode + append (decode_kernel.cu:10-84, called by
 * fused_decode.py:28-35 from sphkv_lut.py:176-183).  For every kv head h:
 * v_pool[pids[h], slot] = fp16(v_new[h]); per group the first-max argmax of
 * <k_g / (|k_g| + 1e-8), centroid> over decode_cb [num_kv, G, C, g], its code
 * into theta_codes, and the radius against the page's running-max scale
 * (is_new_page: scale = |k_g|; else a larger |k_g| rescales the page's
 * earlier radius codes).  Bit-exact with the reference arithmetic (nvcc's
 * contraction of a*b + c to fmaf, IEEE sqrt / divide, roundf).
 * k_post, v_new fp32 [num_kv, dh]; pids int64 [num_kv] (pool pages; a pid
 * outside [0, num_pages) is skipped).  dh <= 256, G * g <= dh, G * C <= 4096.
 */
int sphkv_encode_append(const float* k_post, const float* v_new, const float* decode_cb,
                        uint8_t* theta_codes, uint8_t* radius_codes, float* r_scales, uint16_t* v_pool,
                        const int64_t* pids, int32_t num_kv, int64_t num_pages, int32_t slot, int32_t G,
                        int32_t g, int32_t C, int32_t G_max, int32_t dh, int32_t page_size,
                        int32_t is_new_page, void* stream);

/*
 * Mode-A decode (fused_decode.py:12-26 -> decode_kernel.cu:108-289).
 * q_all fp32 [num_q, dh] (num_q = num_kv * kv_groups); out fp32 [num_q, dh];
 * partial_scratch fp32 [num_q, max_blocks, dh + 2].  Per q head and logical
 * page, partial_scratch[hq, p, 0:2] = the page's (m, l): m = max logit, l =
 * sum exp(logit - m), logit = sm_scale * sum_g r_hat_g <q_g, centroid_g[code]>
 * (-1e9 where that sum is exactly 0, as the reference masks unwritten slots);
 * (-inf, 0) for absent pages.  out = softmax-weighted V over all pages,
 * acc / (l + 1e-8).  The rest of partial_scratch is scratch.  ctx_lens and
 * max_ctx are accepted for the reference signature and unused, as there.
 * dh in {64, 128}; kv_groups 1..8; page_size a multiple of 16 up to 128.
 */
int sphkv_decode_modea(const float* q_all, const float* cb_flat, const int32_t* tier_G, const int32_t* tier_g,
                       const uint8_t* theta_codes, const uint8_t* radius_codes, const float* r_scales,
                       const uint16_t* v_pool, int64_t num_pages, const int32_t* block_table,
                       const int32_t* bits_table, const int32_t* ctx_lens, float* out, float* partial_scratch,
                       int32_t num_q_heads, int32_t num_kv_heads, int32_t kv_groups, int32_t num_tiers,
                       int32_t max_blocks, int32_t page_size, int32_t dh, int32_t G_max, int32_t cb_max,
                       int32_t g_max, float sm_scale, int32_t max_ctx, void* stream);

/*
 * Per-query q.centroid table (the q_lut that new_fused_decode.py:22-43
 * consumes): q_lut fp32 [num_q, num_tiers, G_max, cb_max],
 * q_lut[hq, t, g, c] = sum_{d < tier_g[t]} q[hq, g*tier_g[t] + d] *
 * cb_flat[hq / kv_groups, t, g, c, d] for g < tier_G[t], else 0.
 * No reference counterpart (the reference never builds the table).
 */
int sphkv_q_lut(const float* q_all, const float* cb_flat, const int32_t* tier_G, const int32_t* tier_g,
                int32_t num_q_heads, int32_t num_kv_heads, int32_t kv_groups, int32_t num_tiers, int32_t dh,
                int32_t G_max, int32_t cb_max, int32_t g_max, float* q_lut, void* stream);

/*
 * Logits from a q_lut (new_fused_decode.py:22-43): logits_out fp32
 * [num_q, max_ctx]; token n of kv head hkv = hq / kv_groups is slot
 * n % page_size of logical page n / page_size; logit = sm_scale *
 * sum_{g < G_max} r_hat_g * q_lut[hq, tier, g, code_g]; -inf for
 * n >= ctx_lens[hkv] or an absent page.
 */
int sphkv_logits_lut(const float* q_lut, const uint8_t* theta_codes, const uint8_t* radius_codes,
                     const float* r_scales, int64_t num_pages, const int32_t* block_table,
                     const int32_t* bits_table, const int32_t* ctx_lens, float* logits_out,
                     int32_t num_q_heads, int32_t num_kv_heads, int32_t kv_groups, int32_t num_tiers,
                     int32_t max_blocks, int32_t page_size, int32_t G_max, int32_t cb_size_max,
                     float sm_scale, int32_t max_ctx, void* stream);

/*
 * omega importance EMA from a decode's per-page statistics; replaces
 * _omega_ema_eager / _omega_ema_compiled (spherical_kv_pipeline.py:952-987)
 * as called by _update_omega_gpu (:1669-1701).  m_q, l_q: the (m, l) of
 * (q head hq, logical page p) at m_q[hq * q_stride + p * page_stride] (the
 * [..., 0] and [..., 1] views of partial_scratch: q_stride =
 * max_blocks * (dh + 2), page_stride = dh + 2).  Per q head, pages with
 * l > 0 get w = exp(max(m - max, -60)) * l, mass = w / max(sum w, 1e-12);
 * omega_out[h, p] = omega_prev[h, p] * ema_beta + mean_{hq of h} mass *
 * (1 - ema_beta).  omega_prev / omega_out fp32 [num_kv, max_blocks]; they
 * may be the same buffer.  kv_groups 1..64.
 */
int sphkv_omega_ema(const float* m_q, const float* l_q, int64_t q_stride, int64_t page_stride,
                    const float* omega_prev, float* omega_out, int32_t num_kv, int32_t kv_groups,
                    int32_t max_blocks, float ema_beta, void* stream);

/*
 * LayerPool page build from per-(head, tier) token arrays; replaces the
 * per-page loop of LayerPool.__init__ (sphkv_lut.py:44-66, 83-87).
 * r fp32 / theta int32: concatenated [rows, G_t] arrays (n_elems elements);
 * v fp16 [n_vrows, dh].  page_src int32 [n_pages, 4]: per page (element
 * offset of its first r / theta row, its first V row, npg, G_t).  Page i
 * becomes pool page pid0 + i: r_scales[g] = max(max_n r, 1e-8), radius code
 * clamp(round_half_even(r / r_scale * 255), 0, 255), theta code = low byte,
 * V rows copied; slots >= npg and groups >= G_t are untouched (the pools
 * start zeroed, as the reference allocates them).  A descriptor outside the
 * given arrays leaves its page untouched.  G_max <= 256.
 */
int sphkv_build_layer_pool(const float* r, const int32_t* theta, int64_t n_elems, const uint16_t* v,
                           int64_t n_vrows, const int32_t* page_src, int32_t n_pages, int32_t pid0,
                           uint8_t* theta_codes, uint8_t* radius_codes, float* r_scales, uint16_t* v_pool,
                           int64_t pool_pages, int32_t page_size, int32_t G_max, int32_t dh, void* stream);

/*
 * Device page planning for prefill; replaces the grouping, sort, chunking and
 * offset computation of _build_per_head_pages (spherical_kv_pipeline.py:
 * 1146-1228; offsets :1202-1213).  The result equals
 * sphkv_format.plan_pages with logical placement.
 *
 * tier_of uint8 [num_seqs * num_kv, tier_stride]: tier id of each token for
 * (sequence s, kv head h) in row s * num_kv + h (0 dropped, 1..3, 0xFF
 * dense); only the first lens[s] entries of a row are read.
 *
 * lens[s] <= max_len <= tier_stride for every sequence; tokens are
 * processed in chunks, max_len sizes the grid.  The workspace holds
 * sphkv_plan_pages_work_ints(num_seqs, num_kv, max_len) int32 and carries
 * the counts from phase 1 to phase 2 (same arguments in both).
 *
 * Phase 1, sphkv_plan_pages_count: row_start int32
 * [num_seqs * num_kv + 1]; totals int32 [4] receives (rows, byte-pool size
 * or -1 when >= 2 GiB, invalid tier ids, sequence-length and offset
 * overflows); both are written whole (no initial value needed) when
 * num_seqs > 0.
 *
 * Phase 2, sphkv_plan_pages_fill: per row (capacity max_rows >= totals[0])
 * tier, count, ptable [rows, 3], seq_head, vslot (= row), tokens int64
 * [rows, 16] (token index, -1 pad), positions_out int32 [rows, 16]
 * (positions[s * pos_stride + t], or t when positions is null; -1 pad) and,
 * when row_base is given, src_rows int64 [rows, 16] = row_base[s * num_kv +
 * h] + t (-1 pad).
 */
int64_t sphkv_plan_pages_work_ints(int32_t num_seqs, int32_t num_kv, int32_t max_len);
int sphkv_plan_pages_count(const uint8_t* tier_of, int64_t tier_stride, const int32_t* lens, int32_t num_seqs,
                           int32_t num_kv, int32_t max_len, int32_t dh, int32_t* work, int64_t work_ints,
                           int32_t* row_start, int32_t* totals, void* stream);
int sphkv_plan_pages_fill(const uint8_t* tier_of, int64_t tier_stride, const int32_t* lens, const int32_t* positions,
                          int64_t pos_stride, const int64_t* row_base, int32_t num_seqs, int32_t num_kv,
                          int32_t max_len, int32_t dh, const int32_t* work, int32_t max_rows, int32_t* tier,
                          int32_t* count, int32_t* ptable, int32_t* seq_head, int32_t* vslot, int64_t* tokens,
                          int32_t* positions_out, int64_t* src_rows, void* stream);

/*
 * Host-side work list of sphkv_decode_paged (host pointers, no stream, no GPU
 * call).  No reference counterpart: the reference's decode
 * (decode_kernel.cu:249-289) runs one program per (batch, head) and has no
 * work list; these split each (seq, head) row range [row_start[i],
 * row_start[i + 1]) over work items.  row_start int32 [num_sh + 1],
 * non-decreasing.
 *
 * sphkv_work_rows_per_item: rows per item.  When one item per CU can cover
 * every range, the smallest r >= max(8, ceil(total / (num_cus *
 * slots_per_cu))) whose item total sum_i max(1, ceil(len_i / r)) fits num_cus
 * * slots_per_cu; otherwise max(8, ceil(total / (4 * num_cus *
 * slots_per_cu))).  Returns r >= 8, or a negative SPHKV_E* code.
 *
 * sphkv_work_fill: work int32 [n, 4] = (sh, first_row, end_row, stride) with
 * n = sum_i max(1, ceil(len_i / rows_per_item)) (capacity max_items), and
 * work_start int32 [num_sh + 1] = first item of each range.  interleave != 0:
 * item j of a range of n_i items takes rows b + j, b + j + n_i, ...;
 * otherwise contiguous runs of rows_per_item rows (stride 1).  Returns n, or
 * a negative SPHKV_E* code.
 */
int32_t sphkv_work_rows_per_item(const int32_t* row_start, int32_t num_sh, int32_t num_cus, int32_t slots_per_cu);
int64_t sphkv_work_fill(const int32_t* row_start, int32_t num_sh, int32_t rows_per_item, int32_t interleave,
                        int32_t* work, int64_t max_items, int32_t* work_start);

#ifdef __cplusplus
}
#endif
#endif /* SPHKV_H */
