// extern "C" boundary of libsphkv.so (declarations: include/sphkv.h).
// Host code only: argument validation, error reporting, kernel dispatch.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <new>

#include "../../include/sphkv.h"
#include "sphkv_internal.h"

namespace {

thread_local char g_err[512] = "";

int fail_v(int code, const char* fmt, va_list ap) {
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  return code;
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  fail_v(code, fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return SPHKV_OK;
}

int launch_status(int rc, const char* what) {
  if (rc != 0) {
    hipError_t e = hipGetLastError();
    return fail(SPHKV_ELAUNCH, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  }
  return ok();
}

// a work list's row_start: num_sh + 1 non-decreasing, non-negative row indices
bool row_start_ok(const int32_t* rs, int32_t num_sh) {
  if (num_sh < 0 || (num_sh > 0 && !rs) || (rs && rs[0] < 0)) return false;
  for (int32_t i = 0; i < num_sh; ++i)
    if (rs[i + 1] < rs[i]) return false;
  return true;
}

// items the ranges take at r rows per item: sum of max(1, ceil(len / r))
int64_t work_items(const int32_t* rs, int32_t num_sh, int64_t r) {
  int64_t n = 0;
  for (int32_t i = 0; i < num_sh; ++i) {
    const int64_t len = (int64_t)rs[i + 1] - rs[i];
    n += len > r ? (len + r - 1) / r : 1;
  }
  return n;
}

bool dh_ok(int32_t dh) { return dh == 64 || dh == 128; }
bool gqa_ok(int32_t g) { return g == 1 || g == 2 || g == 4 || g == 8; }

}  // namespace

extern "C" {

const char* sphkv_last_error(void) { return g_err; }

const char* sphkv_version(void) { return "sphkv 0.1 gfx950"; }

int sphkv_encode_pages(const void* k, int32_t k_is_fp32, const uint16_t* v, int64_t num_src_rows,
                       const int64_t* src_rows, const int32_t* tier, const int32_t* count,
                       const int32_t* ptable, const int32_t* vslot, const int32_t* seq_head,
                       int32_t num_pages, int32_t num_kv,
                       const float* cb1, const float* cb2, const float* cb3,
                       uint8_t* pages, int64_t pages_bytes, uint16_t* v_pool, int64_t num_vpages,
                       float* r_out, int32_t* code_out, int32_t dh, int32_t page_size, void* stream) {
  if (!dh_ok(dh)) return fail(SPHKV_EINVAL, "sphkv_encode_pages: dh must be 64 or 128 (got %d)", dh);
  if (page_size != 16) return fail(SPHKV_EINVAL, "sphkv_encode_pages: page_size must be 16 (got %d)", page_size);
  if (num_pages < 0 || num_kv <= 0 || num_src_rows < 0 || pages_bytes < 0 || num_vpages < 0)
    return fail(SPHKV_EINVAL, "sphkv_encode_pages: negative size");
  if (num_pages == 0) return ok();
  if (!k || !v || !src_rows || !tier || !count || !ptable || !vslot || !seq_head || !pages || !v_pool)
    return fail(SPHKV_EINVAL, "sphkv_encode_pages: null pointer argument");
  sphkv::EncodeLaunch L{k, k_is_fp32, v, num_src_rows, src_rows, tier, count, ptable, vslot, seq_head,
                        num_pages, num_kv, cb1, cb2, cb3, pages, pages_bytes, v_pool, num_vpages,
                        r_out, code_out, dh, nullptr, 0};
  return launch_status(sphkv::launch_encode(L, (hipStream_t)stream), "sphkv_encode_pages");
}

int sphkv_encode_codes(const void* k, int32_t k_is_fp32, int64_t num_src_rows, const int64_t* src_rows,
                       const int32_t* tier, const int32_t* count, const int32_t* order_n, const int32_t* seq_head,
                       int32_t num_pages, int32_t num_kv, const float* cb1, const float* cb2, const float* cb3,
                       float* r_out, int32_t* code_out, int32_t dh, int32_t page_size, void* stream) {
  const char* fn = "sphkv_encode_codes";
  if (!dh_ok(dh)) return fail(SPHKV_EINVAL, "%s: dh must be 64 or 128 (got %d)", fn, dh);
  if (page_size != 16) return fail(SPHKV_EINVAL, "%s: page_size must be 16 (got %d)", fn, page_size);
  if (num_pages < 0 || num_kv <= 0 || num_src_rows < 0) return fail(SPHKV_EINVAL, "%s: negative size", fn);
  if (num_pages == 0) return ok();
  if (!k || !src_rows || !tier || !count || !seq_head || !r_out || !code_out)
    return fail(SPHKV_EINVAL, "%s: null pointer argument", fn);
  sphkv::EncodeLaunch L{k, k_is_fp32, nullptr, num_src_rows, src_rows, tier, count, nullptr, nullptr, seq_head,
                        num_pages, num_kv, cb1, cb2, cb3, nullptr, 0, nullptr, 0, r_out, code_out, dh, order_n, 1};
  return launch_status(sphkv::launch_encode(L, (hipStream_t)stream), fn);
}

int64_t sphkv_decode_paged_workspace_bytes(int32_t num_items, int32_t gqa, int32_t dh) {
  if (num_items < 0 || !gqa_ok(gqa) || !dh_ok(dh)) return -1;
  return sphkv::decode_workspace_bytes(num_items, gqa, dh);
}

}  // extern "C"

namespace {

// argument checks of the paged decode (SPHKV_OK: launchable, or nothing to do for num_seqs == 0)
int decode_checks(const char* fn, int phases, const uint8_t* pages, int64_t pages_bytes,
                  const int32_t* ptable, const int32_t* vslot, const int32_t* positions, int32_t num_rows,
                  const uint16_t* v_pool, int64_t num_vpages, const int32_t* work, int32_t num_items,
                  const int32_t* work_start, int32_t num_seqs, int32_t num_kv, int32_t gqa, const uint16_t* q,
                  uint16_t* out, void* workspace, int64_t workspace_bytes, int32_t dh, int32_t page_size,
                  double rope_theta) {
  if (!dh_ok(dh)) return fail(SPHKV_EINVAL, "%s: dh must be 64 or 128 (got %d)", fn, dh);
  if (!gqa_ok(gqa)) return fail(SPHKV_EINVAL, "%s: gqa must be 1, 2, 4 or 8 (got %d)", fn, gqa);
  if (page_size != 16) return fail(SPHKV_EINVAL, "%s: page_size must be 16 (got %d)", fn, page_size);
  if (num_seqs < 0 || num_kv <= 0 || num_items < 0 || num_rows < 0)
    return fail(SPHKV_EINVAL, "%s: negative size", fn);
  if ((phases & sphkv::kPhasePartials) && !(rope_theta > 1.0))
    return fail(SPHKV_EINVAL, "%s: rope_theta must be > 1", fn);
  if ((phases & sphkv::kPhasePartials) &&
      (pages_bytes < 0 || pages_bytes > 0x7FFFFF00LL || (int64_t)num_rows * 64 > 0x7FFFFF00LL))
    return fail(SPHKV_EINVAL, "%s: byte pool and pointer table must stay below 2 GiB", fn);
  // the kernel reads the pool in dwords, and a buffer load returns zero for a
  // dword that reaches past the pool's end
  if ((phases & sphkv::kPhasePartials) && (pages_bytes & 3))
    return fail(SPHKV_EINVAL, "%s: pages_bytes must be a multiple of 4 (pad the byte pool)", fn);
  // V pages are addressed with 64-bit offsets; vslot is int32, so a larger
  // pool could not be indexed in full
  if ((phases & sphkv::kPhasePartials) && (num_vpages < 0 || num_vpages > (int64_t)1 << 31))
    return fail(SPHKV_EINVAL, "%s: num_vpages must be in [0, 2^31] (int32 vslot)", fn);
  if (num_seqs == 0) return ok();
  const int64_t need = sphkv_decode_paged_workspace_bytes(num_items, gqa, dh);
  if (workspace_bytes < need)
    return fail(SPHKV_EINVAL, "%s: workspace too small (%lld < %lld bytes)", fn,
                (long long)workspace_bytes, (long long)need);
  if (num_items < num_seqs * num_kv)
    return fail(SPHKV_EINVAL, "%s: need at least one work item per (seq, head)", fn);
  if (!work_start || !workspace) return fail(SPHKV_EINVAL, "%s: null pointer argument", fn);
  if ((phases & sphkv::kPhaseMerge) && !out) return fail(SPHKV_EINVAL, "%s: null output", fn);
  if ((phases & sphkv::kPhasePartials) &&
      (!q || !work || !pages || !ptable || !vslot || !positions || !v_pool))
    return fail(SPHKV_EINVAL, "%s: null pointer argument", fn);
  return SPHKV_OK;
}

int decode_call(const char* fn, int phases, const uint8_t* pages, int64_t pages_bytes,
                const int32_t* ptable, const int32_t* vslot, const int32_t* positions, int32_t num_rows,
                const uint16_t* v_pool, int64_t num_vpages, const float* cb1, const float* cb2,
                const float* cb3, const int32_t* work, int32_t num_items, const int32_t* work_start,
                int32_t num_seqs, int32_t num_kv, int32_t gqa, const uint16_t* q, uint16_t* out,
                void* workspace, int64_t workspace_bytes, int32_t dh, int32_t page_size,
                float sm_scale, double rope_theta, void* stream) {
  const int rc = decode_checks(fn, phases, pages, pages_bytes, ptable, vslot, positions, num_rows, v_pool,
                               num_vpages, work, num_items, work_start, num_seqs, num_kv, gqa, q, out, workspace,
                               workspace_bytes, dh, page_size, rope_theta);
  if (rc != SPHKV_OK || num_seqs == 0) return rc == SPHKV_OK ? ok() : rc;
  sphkv::DecodeLaunch L{pages, pages_bytes, ptable, vslot, positions, num_rows, v_pool, num_vpages,
                        cb1, cb2, cb3, work, num_items, work_start, num_seqs, num_kv, gqa, q, out,
                        static_cast<float*>(workspace), dh, sm_scale, rope_theta};
  return launch_status(sphkv::launch_decode(L, phases, (hipStream_t)stream), fn);
}

}  // namespace

// Shared with sphkv_noalloc.hip (its entry point validates and launches as
// sphkv_decode_paged does, on its own scratch).
namespace sphkv {
int noalloc_fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  fail_v(code, fmt, ap);
  va_end(ap);
  return code;
}
int noalloc_decode(const char* fn, const uint8_t* pages, int64_t pages_bytes, const int32_t* ptable,
                   const int32_t* vslot, const int32_t* positions, int32_t num_rows, const uint16_t* v_pool,
                   int64_t num_vpages, const float* cb1, const float* cb2, const float* cb3,
                   const int32_t* work, int32_t num_items, const int32_t* work_start, int32_t num_seqs,
                   int32_t num_kv, int32_t gqa, const uint16_t* q, uint16_t* out, void* workspace,
                   int64_t workspace_bytes, int32_t dh, int32_t page_size, float sm_scale, double rope_theta,
                   void* stream) {
  return decode_call(fn, kPhasePartials | kPhaseMerge, pages, pages_bytes, ptable, vslot, positions, num_rows,
                     v_pool, num_vpages, cb1, cb2, cb3, work, num_items, work_start, num_seqs, num_kv, gqa, q,
                     out, workspace, workspace_bytes, dh, page_size, sm_scale, rope_theta, stream);
}
}  // namespace sphkv

extern "C" {

int sphkv_decode_paged(const uint8_t* pages, int64_t pages_bytes, const int32_t* ptable,
                       const int32_t* vslot, const int32_t* positions, int32_t num_rows,
                       const uint16_t* v_pool, int64_t num_vpages,
                       const float* cb1, const float* cb2, const float* cb3,
                       const int32_t* work, int32_t num_items, const int32_t* work_start,
                       int32_t num_seqs, int32_t num_kv, int32_t gqa,
                       const uint16_t* q, uint16_t* out, void* workspace, int64_t workspace_bytes,
                       int32_t dh, int32_t page_size, float sm_scale, double rope_theta,
                       void* stream) {
  return decode_call("sphkv_decode_paged", sphkv::kPhasePartials | sphkv::kPhaseMerge, pages, pages_bytes,
                     ptable, vslot, positions, num_rows, v_pool, num_vpages, cb1, cb2, cb3, work,
                     num_items, work_start, num_seqs, num_kv, gqa, q, out, workspace, workspace_bytes,
                     dh, page_size, sm_scale, rope_theta, stream);
}

int sphkv_decode_paged_status(const void* workspace, int64_t workspace_bytes, int32_t num_items, int32_t gqa,
                              int32_t dh, int32_t* malformed, void* stream) {
  const char* fn = "sphkv_decode_paged_status";
  if (!malformed) return fail(SPHKV_EINVAL, "%s: null output", fn);
  const int64_t need = sphkv_decode_paged_workspace_bytes(num_items, gqa, dh);
  if (need < 0 || workspace_bytes < need || !workspace)
    return fail(SPHKV_EINVAL, "%s: workspace of %lld bytes does not hold %d items", fn,
                (long long)workspace_bytes, num_items);
  uint32_t st = 0;
  const uint8_t* src = static_cast<const uint8_t*>(workspace) + need - sphkv::kDecodeStatusBytes + 4;
  hipError_t e = hipMemcpyAsync(&st, src, 4, hipMemcpyDeviceToHost, (hipStream_t)stream);
  if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)stream);
  if (e != hipSuccess) return fail(SPHKV_ELAUNCH, "%s: %s", fn, hipGetErrorString(e));
  *malformed = (int32_t)(st > 0x7FFFFFFFu ? 0x7FFFFFFFu : st);
  return ok();
}

int sphkv_decode_paged_checked(const uint8_t* pages, int64_t pages_bytes, const int32_t* ptable,
                               const int32_t* vslot, const int32_t* positions, int32_t num_rows,
                               const uint16_t* v_pool, int64_t num_vpages,
                               const float* cb1, const float* cb2, const float* cb3,
                               const int32_t* work, int32_t num_items, const int32_t* work_start,
                               int32_t num_seqs, int32_t num_kv, int32_t gqa,
                               const uint16_t* q, uint16_t* out, void* workspace, int64_t workspace_bytes,
                               int32_t dh, int32_t page_size, float sm_scale, double rope_theta,
                               void* stream) {
  const char* fn = "sphkv_decode_paged_checked";
  int rc = decode_call(fn, sphkv::kPhasePartials | sphkv::kPhaseMerge, pages, pages_bytes, ptable, vslot,
                       positions, num_rows, v_pool, num_vpages, cb1, cb2, cb3, work, num_items, work_start,
                       num_seqs, num_kv, gqa, q, out, workspace, workspace_bytes, dh, page_size, sm_scale,
                       rope_theta, stream);
  if (rc != SPHKV_OK || num_seqs == 0) return rc;
  int32_t bad = 0;
  rc = sphkv_decode_paged_status(workspace, workspace_bytes, num_items, gqa, dh, &bad, stream);
  if (rc != SPHKV_OK) return rc;
  if (bad != 0)
    return fail(SPHKV_EPAGE, "%s: %d malformed pointer-table rows or pages were skipped", fn, bad);
  return ok();
}

int sphkv_decode_paged_partials(const uint8_t* pages, int64_t pages_bytes, const int32_t* ptable,
                                const int32_t* vslot, const int32_t* positions, int32_t num_rows,
                                const uint16_t* v_pool, int64_t num_vpages,
                                const float* cb1, const float* cb2, const float* cb3,
                                const int32_t* work, int32_t num_items, const int32_t* work_start,
                                int32_t num_seqs, int32_t num_kv, int32_t gqa,
                                const uint16_t* q, void* workspace, int64_t workspace_bytes,
                                int32_t dh, int32_t page_size, float sm_scale, double rope_theta,
                                void* stream) {
  return decode_call("sphkv_decode_paged_partials", sphkv::kPhasePartials, pages, pages_bytes, ptable,
                     vslot, positions, num_rows, v_pool, num_vpages, cb1, cb2, cb3, work, num_items,
                     work_start, num_seqs, num_kv, gqa, q, nullptr, workspace, workspace_bytes, dh,
                     page_size, sm_scale, rope_theta, stream);
}

int sphkv_decode_merge_partials(const void* workspace, int64_t workspace_bytes, int32_t num_items,
                                const int32_t* work_start, int32_t num_seqs, int32_t num_kv,
                                int32_t gqa, int32_t dh, uint16_t* out, void* stream) {
  return decode_call("sphkv_decode_merge_partials", sphkv::kPhaseMerge, nullptr, 0, nullptr, nullptr,
                     nullptr, 0, nullptr, 0, nullptr, nullptr, nullptr, nullptr, num_items, work_start,
                     num_seqs, num_kv, gqa, nullptr, out, const_cast<void*>(workspace), workspace_bytes,
                     dh, 16, 1.f, 0.0, stream);
}

}  // extern "C"

namespace {

// Shared checks of the tail entries: the tail state, the decode-page region
// and the step inputs.
int tail_checks(const char* fn, int64_t pages_bytes, int32_t num_rows, int64_t num_vpages, const float* cb3,
                int32_t num_seqs, int32_t num_kv, const void* k_new, const uint16_t* v_new, const int32_t* cur_pos,
                const float* stg_r, const int32_t* stg_code, const uint16_t* stg_v, const int32_t* stg_pos,
                const int32_t* tail_state, int64_t dec_byte0, int32_t dec_vpage0, int32_t dec_cap, int32_t dh) {
  if (!cb3) return fail(SPHKV_EINVAL, "%s: the tier-3 codebook is required (decode tokens are tier 3)", fn);
  if (!k_new || !v_new || !cur_pos || !stg_r || !stg_code || !stg_v || !stg_pos || !tail_state)
    return fail(SPHKV_EINVAL, "%s: null pointer argument", fn);
  if (dec_cap < 0 || dec_byte0 < 0 || dec_vpage0 < 0 || (dec_byte0 & 15))
    return fail(SPHKV_EINVAL, "%s: dec_cap, dec_vpage0 and dec_byte0 must be >= 0, dec_byte0 16-byte aligned", fn);
  const int64_t nres = (int64_t)num_seqs * num_kv * dec_cap;
  if (dec_byte0 + nres * sphkv::tail_slot_bytes(dh) > pages_bytes)
    return fail(SPHKV_EINVAL, "%s: the decode-page region (%lld pages of %d bytes from %lld) leaves the byte pool",
                fn, (long long)nres, sphkv::tail_slot_bytes(dh), (long long)dec_byte0);
  if ((int64_t)dec_vpage0 + nres > num_vpages)
    return fail(SPHKV_EINVAL, "%s: the decode pages' V slots leave the V pool", fn);
  if (num_rows < 0) return fail(SPHKV_EINVAL, "%s: negative size", fn);
  return SPHKV_OK;
}

}  // namespace

extern "C" {

int sphkv_decode_step(uint8_t* pages, int64_t pages_bytes, const int32_t* ptable, const int32_t* vslot,
                      int32_t* positions, int32_t num_rows, uint16_t* v_pool, int64_t num_vpages,
                      const float* cb1, const float* cb2, const float* cb3,
                      int32_t* work, int32_t num_items, const int32_t* work_start,
                      int32_t num_seqs, int32_t num_kv, int32_t gqa,
                      const uint16_t* q, const void* k_new, int32_t k_is_fp32, const uint16_t* v_new,
                      const int32_t* cur_pos, float* stg_r, int32_t* stg_code, uint16_t* stg_v, int32_t* stg_pos,
                      int32_t* tail_state, int64_t dec_byte0, int32_t dec_vpage0, int32_t dec_cap, int32_t append,
                      int32_t step_parity, uint16_t* out, void* workspace, int64_t workspace_bytes,
                      int32_t dh, int32_t page_size, float sm_scale, double rope_theta, void* stream) {
  const char* fn = "sphkv_decode_step";
  // the page-resident part is checked exactly as sphkv_decode_paged's (no launch)
  if (!dh_ok(dh)) return fail(SPHKV_EINVAL, "%s: dh must be 64 or 128 (got %d)", fn, dh);
  if (!gqa_ok(gqa)) return fail(SPHKV_EINVAL, "%s: gqa must be 1, 2, 4 or 8 (got %d)", fn, gqa);
  if (page_size != 16) return fail(SPHKV_EINVAL, "%s: page_size must be 16 (got %d)", fn, page_size);
  if (num_seqs < 0 || num_kv <= 0 || num_items < 0 || num_rows < 0) return fail(SPHKV_EINVAL, "%s: negative size", fn);
  if (!(rope_theta > 1.0)) return fail(SPHKV_EINVAL, "%s: rope_theta must be > 1", fn);
  if (pages_bytes < 0 || pages_bytes > 0x7FFFFF00LL || (int64_t)num_rows * 64 > 0x7FFFFF00LL)
    return fail(SPHKV_EINVAL, "%s: byte pool and pointer table must stay below 2 GiB", fn);
  if (pages_bytes & 3) return fail(SPHKV_EINVAL, "%s: pages_bytes must be a multiple of 4 (pad the byte pool)", fn);
  if (num_vpages < 0 || num_vpages > (int64_t)1 << 31)
    return fail(SPHKV_EINVAL, "%s: num_vpages must be in [0, 2^31] (int32 vslot)", fn);
  if (append != 0 && append != 1) return fail(SPHKV_EINVAL, "%s: append must be 0 or 1", fn);
  if (step_parity != 0 && step_parity != 1) return fail(SPHKV_EINVAL, "%s: step_parity must be 0 or 1", fn);
  if (num_seqs == 0) return ok();
  int rc = tail_checks(fn, pages_bytes, num_rows, num_vpages, cb3, num_seqs, num_kv, k_new, v_new, cur_pos, stg_r,
                       stg_code, stg_v, stg_pos, tail_state, dec_byte0, dec_vpage0, dec_cap, dh);
  if (rc != SPHKV_OK) return rc;
  const int64_t need = sphkv_decode_paged_workspace_bytes(num_items, gqa, dh);
  if (workspace_bytes < need)
    return fail(SPHKV_EINVAL, "%s: workspace too small (%lld < %lld bytes)", fn, (long long)workspace_bytes,
                (long long)need);
  if (num_items < num_seqs * num_kv) return fail(SPHKV_EINVAL, "%s: need at least one work item per (seq, head)", fn);
  if (!work_start || !workspace || !out || !q || !work || !pages || !ptable || !vslot || !positions || !v_pool)
    return fail(SPHKV_EINVAL, "%s: null pointer argument", fn);
  sphkv::DecodeLaunch L{pages, pages_bytes, ptable, vslot, positions, num_rows, v_pool, num_vpages,
                        cb1, cb2, cb3, work, num_items, work_start, num_seqs, num_kv, gqa, q, out,
                        static_cast<float*>(workspace), dh, sm_scale, rope_theta};
  sphkv::TailLaunch T{k_new, k_is_fp32, v_new, cur_pos, stg_r, stg_code, stg_v, stg_pos, tail_state,
                      pages, positions, v_pool, work, dec_byte0, dec_cap, dec_vpage0,
                      sphkv::kTailDecode | (append ? sphkv::kTailAppend : 0), step_parity};
  return launch_status(sphkv::launch_decode_tail(L, T, (hipStream_t)stream), fn);
}

int sphkv_decode_append(uint8_t* pages, int64_t pages_bytes, int32_t* positions, int32_t num_rows,
                        uint16_t* v_pool, int64_t num_vpages, const float* cb3,
                        int32_t* work, int32_t num_items, const int32_t* work_start, int32_t num_seqs,
                        int32_t num_kv, const void* k_new, int32_t k_is_fp32, const uint16_t* v_new,
                        const int32_t* cur_pos, float* stg_r, int32_t* stg_code, uint16_t* stg_v, int32_t* stg_pos,
                        int32_t* tail_state, int64_t dec_byte0, int32_t dec_vpage0, int32_t dec_cap,
                        int32_t step_parity, int32_t dh, int32_t page_size, void* stream) {
  const char* fn = "sphkv_decode_append";
  if (!dh_ok(dh)) return fail(SPHKV_EINVAL, "%s: dh must be 64 or 128 (got %d)", fn, dh);
  if (page_size != 16) return fail(SPHKV_EINVAL, "%s: page_size must be 16 (got %d)", fn, page_size);
  if (num_seqs < 0 || num_kv <= 0 || num_items < 0 || pages_bytes < 0 || num_vpages < 0)
    return fail(SPHKV_EINVAL, "%s: negative size", fn);
  if (step_parity != 0 && step_parity != 1) return fail(SPHKV_EINVAL, "%s: step_parity must be 0 or 1", fn);
  if (num_seqs == 0) return ok();
  int rc = tail_checks(fn, pages_bytes, num_rows, num_vpages, cb3, num_seqs, num_kv, k_new, v_new, cur_pos, stg_r,
                       stg_code, stg_v, stg_pos, tail_state, dec_byte0, dec_vpage0, dec_cap, dh);
  if (rc != SPHKV_OK) return rc;
  if (num_items < num_seqs * num_kv) return fail(SPHKV_EINVAL, "%s: need at least one work item per (seq, head)", fn);
  if (!work || !work_start || !pages || !positions || !v_pool) return fail(SPHKV_EINVAL, "%s: null pointer argument", fn);
  sphkv::DecodeLaunch L{pages, pages_bytes, nullptr, nullptr, positions, num_rows, v_pool, num_vpages,
                        nullptr, nullptr, cb3, work, num_items, work_start, num_seqs, num_kv, 1, nullptr, nullptr,
                        nullptr, dh, 1.f, 2.0};
  sphkv::TailLaunch T{k_new, k_is_fp32, v_new, cur_pos, stg_r, stg_code, stg_v, stg_pos, tail_state,
                      pages, positions, v_pool, work, dec_byte0, dec_cap, dec_vpage0, sphkv::kTailAppend,
                      step_parity};
  return launch_status(sphkv::launch_decode_tail(L, T, (hipStream_t)stream), fn);
}

}  // extern "C"

// A bound decode step: every static argument of sphkv_decode_step, validated
// once, and the host's mirror of the tail counts (every (seq, head) stages
// one token per appending step).
// Plans carry a tag, cleared when they are destroyed: a run on a destroyed
// plan whose memory still holds the cleared tag fails instead of launching.
constexpr uint32_t kStepPlanTag = 0x53504C31u, kDecodePlanTag = 0x44504C31u, kDeadPlanTag = 0u;

struct sphkv_step_plan {
  uint32_t tag;
  sphkv::DecodeLaunch L;
  sphkv::TailLaunch T;
  int64_t workspace_bytes;
  int32_t staged, flushed, parity;
};

extern "C" {

int sphkv_step_plan_create(uint8_t* pages, int64_t pages_bytes, const int32_t* ptable, const int32_t* vslot,
                           int32_t* positions, int32_t num_rows, uint16_t* v_pool, int64_t num_vpages,
                           const float* cb1, const float* cb2, const float* cb3,
                           int32_t* work, int32_t num_items, const int32_t* work_start,
                           int32_t num_seqs, int32_t num_kv, int32_t gqa,
                           float* stg_r, int32_t* stg_code, uint16_t* stg_v, int32_t* stg_pos, int32_t* tail_state,
                           int64_t dec_byte0, int32_t dec_vpage0, int32_t dec_cap, int32_t staged, int32_t flushed,
                           int32_t step_parity, void* workspace, int64_t workspace_bytes, int32_t dh,
                           int32_t page_size, float sm_scale, double rope_theta, sphkv_step_plan** plan_out) {
  const char* fn = "sphkv_step_plan_create";
  if (!plan_out) return fail(SPHKV_EINVAL, "%s: null plan_out", fn);
  *plan_out = nullptr;
  // the step's per-call inputs are checked for presence at run time; here a
  // stand-in address lets the shared checks run
  static const uint16_t probe[1] = {0};
  int rc = sphkv_decode_step(nullptr, pages_bytes, ptable, vslot, positions, num_rows, v_pool, num_vpages, cb1,
                             cb2, cb3, work, num_items, work_start, 0, num_kv, gqa, probe, probe, 0, probe,
                             nullptr, stg_r, stg_code, stg_v, stg_pos, tail_state, dec_byte0, dec_vpage0, dec_cap,
                             1, step_parity, nullptr, workspace, workspace_bytes, dh, page_size, sm_scale, rope_theta,
                             nullptr);
  if (rc != SPHKV_OK) return rc;                    // size / shape checks (num_seqs = 0: no launch)
  if (num_seqs <= 0) return fail(SPHKV_EINVAL, "%s: num_seqs must be > 0", fn);
  rc = tail_checks(fn, pages_bytes, num_rows, num_vpages, cb3, num_seqs, num_kv, probe, probe,
                   reinterpret_cast<const int32_t*>(probe), stg_r, stg_code, stg_v, stg_pos, tail_state, dec_byte0,
                   dec_vpage0, dec_cap, dh);
  if (rc != SPHKV_OK) return rc;
  const int64_t need = sphkv_decode_paged_workspace_bytes(num_items, gqa, dh);
  if (workspace_bytes < need)
    return fail(SPHKV_EINVAL, "%s: workspace too small (%lld < %lld bytes)", fn, (long long)workspace_bytes,
                (long long)need);
  if (num_items < num_seqs * num_kv) return fail(SPHKV_EINVAL, "%s: need at least one work item per (seq, head)", fn);
  if (!work_start || !workspace || !work || !pages || !ptable || !vslot || !positions || !v_pool)
    return fail(SPHKV_EINVAL, "%s: null pointer argument", fn);
  if (staged < 0 || staged >= sphkv::kTailSlots || flushed < 0 || flushed > dec_cap)
    return fail(SPHKV_EINVAL, "%s: staged must be 0..15 and flushed 0..dec_cap", fn);
  auto* p = new (std::nothrow) sphkv_step_plan;
  if (!p) return fail(SPHKV_EINVAL, "%s: out of host memory", fn);
  p->tag = kStepPlanTag;
  p->L = sphkv::DecodeLaunch{pages, pages_bytes, ptable, vslot, positions, num_rows, v_pool, num_vpages,
                             cb1, cb2, cb3, work, num_items, work_start, num_seqs, num_kv, gqa, nullptr, nullptr,
                             static_cast<float*>(workspace), dh, sm_scale, rope_theta};
  p->T = sphkv::TailLaunch{nullptr, 0, nullptr, nullptr, stg_r, stg_code, stg_v, stg_pos, tail_state,
                           pages, positions, v_pool, work, dec_byte0, dec_cap, dec_vpage0, 0, 0};
  p->workspace_bytes = workspace_bytes;
  p->staged = staged;
  p->flushed = flushed;
  p->parity = step_parity;
  *plan_out = p;
  return ok();
}

int sphkv_step_plan_run(sphkv_step_plan* plan, const uint16_t* q, const void* k_new, int32_t k_is_fp32,
                        const uint16_t* v_new, const int32_t* cur_pos, uint16_t* out, int32_t mode, void* stream) {
  const char* fn = "sphkv_step_plan_run";
  if (!plan || plan->tag != kStepPlanTag) return fail(SPHKV_EINVAL, "%s: null or destroyed plan", fn);
  if (mode < 1 || mode > 3) return fail(SPHKV_EINVAL, "%s: mode must be 1 (decode), 2 (append) or 3 (both)", fn);
  const bool dec = mode & sphkv::kTailDecode, app = mode & sphkv::kTailAppend;
  if (!k_new || !v_new || !cur_pos || (dec && (!q || !out))) return fail(SPHKV_EINVAL, "%s: null pointer argument", fn);
  if (app && plan->staged == sphkv::kTailSlots - 1 && plan->flushed >= plan->T.dec_cap)
    return fail(SPHKV_EINVAL, "%s: no decode-page slot left (capacity %d pages per (seq, head))", fn,
                plan->T.dec_cap);
  sphkv::DecodeLaunch L = plan->L;
  L.q = q;
  L.out = out;
  sphkv::TailLaunch T = plan->T;
  T.k_new = k_new;
  T.k_is_fp32 = k_is_fp32 ? 1 : 0;
  T.v_new = v_new;
  T.cur_pos = cur_pos;
  T.mode = mode;
  T.parity = plan->parity;
  const int rc = launch_status(sphkv::launch_decode_tail(L, T, (hipStream_t)stream), fn);
  if (rc == SPHKV_OK && app) {
    plan->parity ^= 1;
    if (++plan->staged == sphkv::kTailSlots) {
      plan->staged = 0;
      ++plan->flushed;
    }
  }
  return rc;
}

int sphkv_step_plan_counts(const sphkv_step_plan* plan, int32_t* staged, int32_t* flushed, int32_t* step_parity) {
  if (!plan || plan->tag != kStepPlanTag || !staged || !flushed || !step_parity)
    return fail(SPHKV_EINVAL, "sphkv_step_plan_counts: null argument or destroyed plan");
  *staged = plan->staged;
  *flushed = plan->flushed;
  *step_parity = plan->parity;
  return ok();
}

void sphkv_step_plan_destroy(sphkv_step_plan* plan) {
  if (!plan) return;
  *reinterpret_cast<volatile uint32_t*>(&plan->tag) = kDeadPlanTag;
  delete plan;
}

}  // extern "C"

struct sphkv_decode_plan {
  uint32_t tag;
  sphkv::DecodeLaunch L;
};

extern "C" {

int sphkv_decode_plan_create(const uint8_t* pages, int64_t pages_bytes, const int32_t* ptable,
                             const int32_t* vslot, const int32_t* positions, int32_t num_rows,
                             const uint16_t* v_pool, int64_t num_vpages,
                             const float* cb1, const float* cb2, const float* cb3,
                             const int32_t* work, int32_t num_items, const int32_t* work_start,
                             int32_t num_seqs, int32_t num_kv, int32_t gqa, void* workspace,
                             int64_t workspace_bytes, int32_t dh, int32_t page_size, float sm_scale,
                             double rope_theta, sphkv_decode_plan** plan_out) {
  const char* fn = "sphkv_decode_plan_create";
  if (!plan_out) return fail(SPHKV_EINVAL, "%s: null plan_out", fn);
  *plan_out = nullptr;
  // q and out come with each run: a stand-in address lets the checks run
  static uint16_t probe[1] = {0};
  int rc = decode_checks(fn, sphkv::kPhasePartials | sphkv::kPhaseMerge, pages, pages_bytes, ptable, vslot,
                         positions, num_rows, v_pool, num_vpages, work, num_items, work_start, num_seqs, num_kv,
                         gqa, probe, probe, workspace, workspace_bytes, dh, page_size, rope_theta);
  if (rc != SPHKV_OK) return rc;
  if (num_seqs <= 0) return fail(SPHKV_EINVAL, "%s: num_seqs must be > 0", fn);
  auto* p = new (std::nothrow) sphkv_decode_plan;
  if (!p) return fail(SPHKV_EINVAL, "%s: out of host memory", fn);
  p->tag = kDecodePlanTag;
  p->L = sphkv::DecodeLaunch{pages, pages_bytes, ptable, vslot, positions, num_rows, v_pool, num_vpages,
                             cb1, cb2, cb3, work, num_items, work_start, num_seqs, num_kv, gqa, nullptr, nullptr,
                             static_cast<float*>(workspace), dh, sm_scale, rope_theta};
  *plan_out = p;
  return ok();
}

int sphkv_decode_plan_run(const sphkv_decode_plan* plan, const uint16_t* q, uint16_t* out, void* stream) {
  if (!plan || plan->tag != kDecodePlanTag || !q || !out)
    return fail(SPHKV_EINVAL, "sphkv_decode_plan_run: null argument or destroyed plan");
  sphkv::DecodeLaunch L = plan->L;
  L.q = q;
  L.out = out;
  return launch_status(sphkv::launch_decode(L, sphkv::kPhasePartials | sphkv::kPhaseMerge, (hipStream_t)stream),
                       "sphkv_decode_plan_run");
}

void sphkv_decode_plan_destroy(sphkv_decode_plan* plan) {
  if (!plan) return;
  *reinterpret_cast<volatile uint32_t*>(&plan->tag) = kDeadPlanTag;
  delete plan;
}

int sphkv_time_next_decode_kernel(void* start_event, void* stop_event) {
  if ((start_event == nullptr) != (stop_event == nullptr))
    return fail(SPHKV_EINVAL, "sphkv_time_next_decode_kernel: give both events or neither");
  sphkv::set_decode_timing(static_cast<hipEvent_t>(start_event), static_cast<hipEvent_t>(stop_event));
  return ok();
}

int sphkv_tail_relayout(const int32_t* row_start, int32_t num_sh, int32_t num_rows, const int32_t* ptable,
                        const int32_t* vslot, const int32_t* positions, int32_t dec_cap, int64_t dec_byte0,
                        int32_t dec_vpage0, int32_t dh, int32_t* ptable_d, int32_t* vslot_d, int32_t* positions_d,
                        void* stream) {
  const char* fn = "sphkv_tail_relayout";
  if (!dh_ok(dh)) return fail(SPHKV_EINVAL, "%s: dh must be 64 or 128 (got %d)", fn, dh);
  if (num_sh < 0 || num_rows < 0 || dec_cap < 0 || dec_byte0 < 0 || dec_vpage0 < 0 || (dec_byte0 & 15))
    return fail(SPHKV_EINVAL, "%s: bad size or a dec_byte0 that is not 16-byte aligned", fn);
  const int64_t nres = (int64_t)num_sh * dec_cap;
  if ((int64_t)num_rows + nres > 0x7FFFFFFFLL / 64 || dec_byte0 + nres * sphkv::tail_slot_bytes(dh) > 0x7FFFFF00LL ||
      (int64_t)dec_vpage0 + nres > 0x7FFFFFFFLL)
    return fail(SPHKV_EINVAL, "%s: the decode-time table, byte pool or V pool outgrows int32 indices", fn);
  if ((int64_t)num_rows + nres == 0) return ok();
  if (!row_start || !ptable_d || !vslot_d || !positions_d || (num_rows > 0 && (!ptable || !vslot || !positions)))
    return fail(SPHKV_EINVAL, "%s: null pointer argument", fn);
  return launch_status(sphkv::launch_tail_relayout(row_start, num_sh, num_rows, ptable, vslot, positions, dec_cap,
                                                   dec_byte0, dec_vpage0, dh, ptable_d, vslot_d, positions_d,
                                                   (hipStream_t)stream), fn);
}

static int ragged_call(const char* fn, const uint8_t* pages, int64_t pages_bytes, const int32_t* ptable,
                       const int32_t* head_ids, const int32_t* positions, int32_t num_pages,
                       const float* cos_tbl, const float* sin_tbl, int32_t max_pos,
                       const float* q, int32_t grp, int32_t num_kv, const float* codebooks,
                       int32_t dh, int32_t groups, int32_t group_size, int32_t b_theta,
                       int32_t page_size, const void* rope_fit, int32_t rope_model, float* logits_out,
                       void* stream) {
  if (!dh_ok(dh)) return fail(SPHKV_EINVAL, "%s: dh must be 64 or 128 (got %d)", fn, dh);
  if (group_size <= 0 || groups * group_size != dh || (group_size % 8) != 0)
    return fail(SPHKV_EINVAL, "%s: groups*group_size must equal dh, group_size %% 8 == 0", fn);
  if (b_theta < 1 || b_theta > 8) return fail(SPHKV_EINVAL, "%s: b_theta must be 1..8", fn);
  if (page_size < 1 || page_size > 128)
    return fail(SPHKV_EINVAL, "%s: page_size must be 1..128 (got %d)", fn, page_size);
  if (num_pages < 0 || grp <= 0 || num_kv <= 0 || max_pos <= 0) return fail(SPHKV_EINVAL, "%s: bad size", fn);
  if (rope_model < sphkv::kRopeNone || rope_model > sphkv::kRopeFp32 || (rope_model != sphkv::kRopeNone && !rope_fit))
    return fail(SPHKV_EINVAL, "%s: rope_model must be 0, 1 or 2 (1 and 2 with a fit)", fn);
  if (num_pages == 0) return ok();
  if (!pages || !ptable || !head_ids || !positions || !cos_tbl || !sin_tbl || !q || !codebooks || !logits_out)
    return fail(SPHKV_EINVAL, "%s: null pointer argument", fn);
  sphkv::RaggedLaunch L{pages, pages_bytes, ptable, head_ids, positions, num_pages, cos_tbl, sin_tbl,
                        max_pos, q, grp, num_kv, codebooks, dh, groups, group_size, b_theta,
                        page_size, logits_out,
                        rope_model != sphkv::kRopeNone ? static_cast<const sphkv::RopeFit*>(rope_fit) : nullptr,
                        rope_model};
  return launch_status(sphkv::launch_ragged(L, (hipStream_t)stream), fn);
}

int sphkv_fused_decode_ragged(const uint8_t* pages, int64_t pages_bytes, const int32_t* ptable,
                              const int32_t* head_ids, const int32_t* positions, int32_t num_pages,
                              const float* cos_tbl, const float* sin_tbl, int32_t max_pos,
                              const float* q, int32_t grp, int32_t num_kv, const float* codebooks,
                              int32_t dh, int32_t groups, int32_t group_size, int32_t b_theta,
                              int32_t page_size, float* logits_out, void* stream) {
  return ragged_call("sphkv_fused_decode_ragged", pages, pages_bytes, ptable, head_ids, positions, num_pages,
                     cos_tbl, sin_tbl, max_pos, q, grp, num_kv, codebooks, dh, groups, group_size, b_theta,
                     page_size, nullptr, sphkv::kRopeNone, logits_out, stream);
}

int sphkv_fused_decode_ragged_fitted(const uint8_t* pages, int64_t pages_bytes, const int32_t* ptable,
                                     const int32_t* head_ids, const int32_t* positions, int32_t num_pages,
                                     const float* cos_tbl, const float* sin_tbl, int32_t max_pos,
                                     const float* q, int32_t grp, int32_t num_kv, const float* codebooks,
                                     int32_t dh, int32_t groups, int32_t group_size, int32_t b_theta,
                                     int32_t page_size, const void* rope_fit, int32_t rope_model,
                                     float* logits_out, void* stream) {
  return ragged_call("sphkv_fused_decode_ragged_fitted", pages, pages_bytes, ptable, head_ids, positions,
                     num_pages, cos_tbl, sin_tbl, max_pos, q, grp, num_kv, codebooks, dh, groups, group_size,
                     b_theta, page_size, rope_fit, rope_model, logits_out, stream);
}

int sphkv_rope_table_fit(const float* cos_tbl, const float* sin_tbl, int32_t max_pos, int32_t dh, void* fit,
                         int32_t* model, float* max_dev, void* stream) {
  const char* fn = "sphkv_rope_table_fit";
  if (!dh_ok(dh)) return fail(SPHKV_EINVAL, "%s: dh must be 64 or 128 (got %d)", fn, dh);
  if (max_pos < 1 || max_pos > (1 << 24))
    return fail(SPHKV_EINVAL, "%s: max_pos must be 1..2^24 (got %d)", fn, max_pos);
  if (!cos_tbl || !sin_tbl || !fit || !model) return fail(SPHKV_EINVAL, "%s: null pointer argument", fn);
  const hipStream_t s = (hipStream_t)stream;
  const int half = dh / 2;
  constexpr double kTwoPi = 6.283185307179586;
  sphkv::RopeFit h;
  memset(&h, 0, sizeof(h));
  h.model = sphkv::kRopeNone;
  h.dh = dh;
  h.max_pos = max_pos;
  // rows 1, 2, 4, ... and the last: each pair's frequency is read from row
  // 1 (atan2, turns) and refined on each later row, whose angle is unwrapped
  // by the previous estimate (an estimate good to e turns per token predicts
  // row 2r to 2 r e turns, far inside the half turn the unwrap needs)
  int rows[40];
  int nr = 0;
  for (int64_t r = 1; r < max_pos; r *= 2) rows[nr++] = (int)r;
  if (nr > 0 && rows[nr - 1] != max_pos - 1) rows[nr++] = max_pos - 1;
  float* hc = nullptr;
  if (nr > 0) {
    hc = new (std::nothrow) float[2 * (size_t)nr * dh];
    if (!hc) return fail(SPHKV_EINVAL, "%s: host allocation failed", fn);
    hipError_t e = hipSuccess;
    for (int i = 0; i < nr && e == hipSuccess; ++i) {
      e = hipMemcpyAsync(hc + (size_t)i * dh, cos_tbl + (int64_t)rows[i] * dh, dh * 4, hipMemcpyDeviceToHost, s);
      if (e == hipSuccess)
        e = hipMemcpyAsync(hc + (size_t)(nr + i) * dh, sin_tbl + (int64_t)rows[i] * dh, dh * 4,
                           hipMemcpyDeviceToHost, s);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
      delete[] hc;
      return fail(SPHKV_ELAUNCH, "%s: reading the tables failed: %s", fn, hipGetErrorString(e));
    }
    for (int j = 0; j < half; ++j) {
      const float* c = hc;
      const float* sn = hc + (size_t)nr * dh;
      double f = atan2((double)sn[j], (double)c[j]) / kTwoPi;
      for (int i = 1; i < nr; ++i) {
        const double t = atan2((double)sn[(size_t)i * dh + j], (double)c[(size_t)i * dh + j]) / kTwoPi;
        f = (t + nearbyint(rows[i] * f - t)) / rows[i];
      }
      h.f[j] = f;
      // the fp32 inverse frequency: of the floats within 4 ulps of 2 pi f,
      // the one whose fp32 angles best reproduce the ladder rows
      float cand = (float)(f * kTwoPi);
      for (int k = 0; k < 4; ++k) cand = nextafterf(cand, -INFINITY);
      float best = cand;
      double best_dev = INFINITY;
      for (int k = 0; k < 9; ++k, cand = nextafterf(cand, INFINITY)) {
        double dev = 0.0;
        for (int i = 0; i < nr; ++i) {
          const float a = (float)rows[i] * cand;
          dev = fmax(dev, fmax(fabs((double)c[(size_t)i * dh + j] - cos((double)a)),
                               fabs((double)sn[(size_t)i * dh + j] - sin((double)a))));
        }
        if (dev < best_dev) {
          best_dev = dev;
          best = cand;
        }
      }
      h.inv32[j] = best;
    }
    delete[] hc;
  }
  // every entry against both models (on the device), then the choice
  sphkv::RopeFit* d = static_cast<sphkv::RopeFit*>(fit);
  sphkv::RopeFit back;
  hipError_t e = hipMemcpyAsync(d, &h, sizeof(h), hipMemcpyHostToDevice, s);
  if (e == hipSuccess && sphkv::launch_rope_check(cos_tbl, sin_tbl, max_pos, dh, d, s) != 0) e = hipGetLastError();
  if (e == hipSuccess) e = hipMemcpyAsync(&back, d, 32, hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return fail(SPHKV_ELAUNCH, "%s: the table check failed: %s", fn, hipGetErrorString(e));
  float dev[2];
  memcpy(&dev[0], &back.dev_bits[0], 4);
  memcpy(&dev[1], &back.dev_bits[1], 4);
  int32_t m = sphkv::kRopeNone;
  if (nr > 0 && back.half_mismatch == 0) {
    if (dev[0] <= sphkv::kRopeFitTol) m = sphkv::kRopeExact;
    else if (dev[1] <= sphkv::kRopeFitTol) m = sphkv::kRopeFp32;
  }
  e = hipMemcpyAsync(&d->model, &m, 4, hipMemcpyHostToDevice, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return fail(SPHKV_ELAUNCH, "%s: writing the fit failed: %s", fn, hipGetErrorString(e));
  *model = m;
  if (max_dev) {
    max_dev[0] = dev[0];
    max_dev[1] = dev[1];
  }
  return ok();
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Mode-A (LayerPool) path
// ---------------------------------------------------------------------------
namespace {

bool modea_geometry(const char* fn, int32_t num_q, int32_t num_kv, int32_t kv_groups, int32_t num_tiers,
                    int32_t dh, int32_t G_max, int32_t cb_max, int32_t g_max, int* rc) {
  if (num_kv < 0 || kv_groups < 1 || kv_groups > 8 || num_q != num_kv * kv_groups) {
    *rc = fail(SPHKV_EINVAL, "%s: need num_q_heads == num_kv_heads * kv_groups, kv_groups 1..8", fn);
    return false;
  }
  if (num_tiers < 1 || num_tiers > sphkv::kModeAMaxTiers) {
    *rc = fail(SPHKV_EINVAL, "%s: num_tiers must be 1..%d", fn, sphkv::kModeAMaxTiers);
    return false;
  }
  if (G_max < 1 || cb_max < 1 || cb_max > 256 || g_max < 1 || G_max * g_max < 1 || dh < 1) {
    *rc = fail(SPHKV_EINVAL, "%s: bad table geometry (G_max %d, cb_max %d, g_max %d)", fn, G_max, cb_max, g_max);
    return false;
  }
  return true;
}

}  // namespace

extern "C" {

int sphkv_encode_append(const float* k_post, const float* v_new, const float* decode_cb,
                        uint8_t* theta_codes, uint8_t* radius_codes, float* r_scales, uint16_t* v_pool,
                        const int64_t* pids, int32_t num_kv, int64_t num_pages, int32_t slot, int32_t G,
                        int32_t g, int32_t C, int32_t G_max, int32_t dh, int32_t page_size,
                        int32_t is_new_page, void* stream) {
  const char* fn = "sphkv_encode_append";
  if (dh < 1 || dh > 256) return fail(SPHKV_EINVAL, "%s: dh must be 1..256 (got %d)", fn, dh);
  if (G < 1 || g < 1 || G * g > dh || G > G_max)
    return fail(SPHKV_EINVAL, "%s: need 1 <= G <= G_max and G * g <= dh", fn);
  if (C < 1 || C > 256 || G * C > 4096) return fail(SPHKV_EINVAL, "%s: need C <= 256 and G * C <= 4096", fn);
  if (page_size < 1 || slot < 0 || slot >= page_size)
    return fail(SPHKV_EINVAL, "%s: slot must be in [0, page_size)", fn);
  if (num_kv < 0 || num_pages < 0) return fail(SPHKV_EINVAL, "%s: negative size", fn);
  if (num_kv == 0) return ok();
  if (!k_post || !v_new || !decode_cb || !theta_codes || !radius_codes || !r_scales || !v_pool || !pids)
    return fail(SPHKV_EINVAL, "%s: null pointer argument", fn);
  sphkv::AppendLaunch L{k_post, v_new, decode_cb, theta_codes, radius_codes, r_scales,
                        reinterpret_cast<_Float16*>(v_pool), pids, num_pages, num_kv, slot, G, g, C,
                        G_max, dh, page_size, is_new_page ? 1 : 0};
  return launch_status(sphkv::launch_append(L, (hipStream_t)stream), fn);
}

int sphkv_decode_modea(const float* q_all, const float* cb_flat, const int32_t* tier_G, const int32_t* tier_g,
                       const uint8_t* theta_codes, const uint8_t* radius_codes, const float* r_scales,
                       const uint16_t* v_pool, int64_t num_pages, const int32_t* block_table,
                       const int32_t* bits_table, const int32_t* ctx_lens, float* out, float* partial_scratch,
                       int32_t num_q_heads, int32_t num_kv_heads, int32_t kv_groups, int32_t num_tiers,
                       int32_t max_blocks, int32_t page_size, int32_t dh, int32_t G_max, int32_t cb_max,
                       int32_t g_max, float sm_scale, int32_t max_ctx, void* stream) {
  const char* fn = "sphkv_decode_modea";
  (void)ctx_lens;
  (void)max_ctx;
  int rc = 0;
  if (!dh_ok(dh)) return fail(SPHKV_EINVAL, "%s: dh must be 64 or 128 (got %d)", fn, dh);
  if (!modea_geometry(fn, num_q_heads, num_kv_heads, kv_groups, num_tiers, dh, G_max, cb_max, g_max, &rc))
    return rc;
  if (page_size < 16 || page_size > 128 || page_size % 16 != 0)
    return fail(SPHKV_EINVAL, "%s: page_size must be a multiple of 16 in 16..128 (got %d)", fn, page_size);
  if (max_blocks < 0 || num_pages < 0) return fail(SPHKV_EINVAL, "%s: negative size", fn);
  sphkv::ModeALaunch L{q_all, cb_flat, tier_G, tier_g, theta_codes, radius_codes, r_scales,
                       reinterpret_cast<const _Float16*>(v_pool), block_table, bits_table, out, partial_scratch,
                       num_q_heads, num_kv_heads, kv_groups, num_tiers, max_blocks, page_size, dh, G_max,
                       cb_max, g_max, num_pages, sm_scale, 1, 0};
  const int64_t lds = sphkv::modea_configure(L);
  if (lds > 160 * 1024)
    return fail(SPHKV_EINVAL, "%s: per-query tables need %lld bytes of LDS (> 160 KiB)", fn, (long long)lds);
  if (num_kv_heads == 0 || max_blocks == 0) return ok();
  if (!q_all || !cb_flat || !tier_G || !tier_g || !theta_codes || !radius_codes || !r_scales || !v_pool ||
      !block_table || !bits_table || !out || !partial_scratch)
    return fail(SPHKV_EINVAL, "%s: null pointer argument", fn);
  return launch_status(sphkv::launch_modea(L, (hipStream_t)stream), fn);
}

int sphkv_q_lut(const float* q_all, const float* cb_flat, const int32_t* tier_G, const int32_t* tier_g,
                int32_t num_q_heads, int32_t num_kv_heads, int32_t kv_groups, int32_t num_tiers, int32_t dh,
                int32_t G_max, int32_t cb_max, int32_t g_max, float* q_lut, void* stream) {
  const char* fn = "sphkv_q_lut";
  int rc = 0;
  if (!modea_geometry(fn, num_q_heads, num_kv_heads, kv_groups, num_tiers, dh, G_max, cb_max, g_max, &rc))
    return rc;
  if (num_q_heads == 0) return ok();
  if (!q_all || !cb_flat || !tier_G || !tier_g || !q_lut) return fail(SPHKV_EINVAL, "%s: null pointer argument", fn);
  sphkv::ModeALaunch L{q_all, cb_flat, tier_G, tier_g, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                       nullptr, nullptr, num_q_heads, num_kv_heads, kv_groups, num_tiers, 0, 16, dh, G_max,
                       cb_max, g_max, 0, 1.f, 1, 0};
  return launch_status(sphkv::launch_qlut(L, q_lut, (hipStream_t)stream), fn);
}

int sphkv_logits_lut(const float* q_lut, const uint8_t* theta_codes, const uint8_t* radius_codes,
                     const float* r_scales, int64_t num_pages, const int32_t* block_table,
                     const int32_t* bits_table, const int32_t* ctx_lens, float* logits_out,
                     int32_t num_q_heads, int32_t num_kv_heads, int32_t kv_groups, int32_t num_tiers,
                     int32_t max_blocks, int32_t page_size, int32_t G_max, int32_t cb_size_max,
                     float sm_scale, int32_t max_ctx, void* stream) {
  const char* fn = "sphkv_logits_lut";
  if (num_kv_heads < 0 || kv_groups < 1 || num_q_heads != num_kv_heads * kv_groups)
    return fail(SPHKV_EINVAL, "%s: need num_q_heads == num_kv_heads * kv_groups", fn);
  if (num_tiers < 1 || G_max < 1 || cb_size_max < 1 || cb_size_max > 256 || page_size < 1)
    return fail(SPHKV_EINVAL, "%s: bad table geometry", fn);
  if (max_blocks < 0 || max_ctx < 0 || num_pages < 0) return fail(SPHKV_EINVAL, "%s: negative size", fn);
  if (num_q_heads == 0 || max_ctx == 0) return ok();
  if (!q_lut || !theta_codes || !radius_codes || !r_scales || !block_table || !bits_table || !ctx_lens ||
      !logits_out)
    return fail(SPHKV_EINVAL, "%s: null pointer argument", fn);
  sphkv::LutLogitsLaunch L{q_lut, theta_codes, radius_codes, r_scales, block_table, bits_table, ctx_lens,
                           logits_out, num_q_heads, num_kv_heads, kv_groups, num_tiers, max_blocks, page_size,
                           G_max, cb_size_max, max_ctx, num_pages, sm_scale};
  return launch_status(sphkv::launch_lut_logits(L, (hipStream_t)stream), fn);
}

int sphkv_omega_ema(const float* m_q, const float* l_q, int64_t q_stride, int64_t page_stride,
                    const float* omega_prev, float* omega_out, int32_t num_kv, int32_t kv_groups,
                    int32_t max_blocks, float ema_beta, void* stream) {
  const char* fn = "sphkv_omega_ema";
  if (num_kv < 0 || max_blocks < 0) return fail(SPHKV_EINVAL, "%s: negative size", fn);
  if (kv_groups < 1 || kv_groups > sphkv::kOmegaMaxGroups)
    return fail(SPHKV_EINVAL, "%s: kv_groups must be 1..%d", fn, sphkv::kOmegaMaxGroups);
  if (q_stride < 0 || page_stride < 0) return fail(SPHKV_EINVAL, "%s: negative stride", fn);
  if (num_kv == 0 || max_blocks == 0) return ok();
  if (!m_q || !l_q || !omega_prev || !omega_out) return fail(SPHKV_EINVAL, "%s: null pointer argument", fn);
  sphkv::OmegaLaunch L{m_q, l_q, q_stride, page_stride, omega_prev, omega_out, num_kv, kv_groups, max_blocks,
                       ema_beta};
  return launch_status(sphkv::launch_omega(L, (hipStream_t)stream), fn);
}

int sphkv_build_layer_pool(const float* r, const int32_t* theta, int64_t n_elems, const uint16_t* v,
                           int64_t n_vrows, const int32_t* page_src, int32_t n_pages, int32_t pid0,
                           uint8_t* theta_codes, uint8_t* radius_codes, float* r_scales, uint16_t* v_pool,
                           int64_t pool_pages, int32_t page_size, int32_t G_max, int32_t dh, void* stream) {
  const char* fn = "sphkv_build_layer_pool";
  if (n_pages < 0 || pid0 < 0 || n_elems < 0 || n_vrows < 0 || pool_pages < 0)
    return fail(SPHKV_EINVAL, "%s: negative size", fn);
  if ((int64_t)pid0 + n_pages > pool_pages)
    return fail(SPHKV_EINVAL, "%s: pages %d..%lld exceed the pool (%lld pages)", fn, pid0,
                (long long)pid0 + n_pages, (long long)pool_pages);
  if (page_size < 1 || G_max < 1 || G_max > sphkv::kPoolBuildMaxG || dh < 2 || (dh & 1))
    return fail(SPHKV_EINVAL, "%s: bad geometry (page_size %d, G_max %d, dh %d)", fn, page_size, G_max, dh);
  if (n_pages == 0) return ok();
  if (!r || !theta || !v || !page_src || !theta_codes || !radius_codes || !r_scales || !v_pool)
    return fail(SPHKV_EINVAL, "%s: null pointer argument", fn);
  sphkv::PoolBuildLaunch L{r, theta, n_elems, reinterpret_cast<const _Float16*>(v), n_vrows, page_src, n_pages, pid0,
                           theta_codes, radius_codes, r_scales, reinterpret_cast<_Float16*>(v_pool), page_size,
                           G_max, dh};
  return launch_status(sphkv::launch_pool_build(L, (hipStream_t)stream), fn);
}

int64_t sphkv_plan_pages_work_ints(int32_t num_seqs, int32_t num_kv, int32_t max_len) {
  if (num_seqs < 0 || num_kv < 1 || max_len < 0) return -1;
  return sphkv::plan_work_ints(num_seqs * num_kv, max_len);
}

int sphkv_plan_pages_count(const uint8_t* tier_of, int64_t tier_stride, const int32_t* lens, int32_t num_seqs,
                           int32_t num_kv, int32_t max_len, int32_t dh, int32_t* work, int64_t work_ints,
                           int32_t* row_start, int32_t* totals, void* stream) {
  const char* fn = "sphkv_plan_pages_count";
  if (!dh_ok(dh)) return fail(SPHKV_EINVAL, "%s: dh must be 64 or 128 (got %d)", fn, dh);
  if (num_seqs < 0 || num_kv < 1 || tier_stride < 0 || max_len < 0 || max_len > tier_stride)
    return fail(SPHKV_EINVAL, "%s: bad sizes (need 0 <= max_len <= tier_stride)", fn);
  if (num_seqs == 0) return ok();
  if (work_ints < sphkv::plan_work_ints(num_seqs * num_kv, max_len))
    return fail(SPHKV_EINVAL, "%s: workspace too small", fn);
  if (!tier_of || !lens || !work || !row_start || !totals) return fail(SPHKV_EINVAL, "%s: null pointer argument", fn);
  sphkv::PlanLaunch L{};
  L.tier_of = tier_of; L.tier_stride = tier_stride; L.lens = lens; L.max_len = max_len; L.num_sh = num_seqs * num_kv;
  L.num_kv = num_kv; L.dh = dh; L.work = work; L.totals = totals; L.row_start = row_start;
  return launch_status(sphkv::launch_plan(L, 0, (hipStream_t)stream), fn);
}

int sphkv_plan_pages_fill(const uint8_t* tier_of, int64_t tier_stride, const int32_t* lens, const int32_t* positions,
                          int64_t pos_stride, const int64_t* row_base, int32_t num_seqs, int32_t num_kv,
                          int32_t max_len, int32_t dh, const int32_t* work, int32_t max_rows, int32_t* tier,
                          int32_t* count, int32_t* ptable, int32_t* seq_head, int32_t* vslot, int64_t* tokens,
                          int32_t* positions_out, int64_t* src_rows, void* stream) {
  const char* fn = "sphkv_plan_pages_fill";
  if (!dh_ok(dh)) return fail(SPHKV_EINVAL, "%s: dh must be 64 or 128 (got %d)", fn, dh);
  if (num_seqs < 0 || num_kv < 1 || tier_stride < 0 || pos_stride < 0 || max_rows < 0 || max_len < 0 ||
      max_len > tier_stride || (positions && max_len > pos_stride && num_seqs > 1))
    return fail(SPHKV_EINVAL, "%s: bad sizes", fn);
  if (num_seqs == 0 || max_rows == 0) return ok();
  if (!tier_of || !lens || !work || !tier || !count || !ptable || !seq_head || !vslot || !tokens || !positions_out)
    return fail(SPHKV_EINVAL, "%s: null pointer argument", fn);
  sphkv::PlanLaunch L{};
  L.tier_of = tier_of; L.tier_stride = tier_stride; L.lens = lens; L.max_len = max_len; L.pos = positions;
  L.pos_stride = pos_stride; L.row_base = row_base; L.num_sh = num_seqs * num_kv; L.num_kv = num_kv; L.dh = dh;
  L.work = const_cast<int32_t*>(work); L.max_rows = max_rows; L.tier = tier; L.count = count; L.ptable = ptable;
  L.seq_head = seq_head; L.vslot = vslot; L.tokens = tokens; L.positions = positions_out; L.src_rows = src_rows;
  return launch_status(sphkv::launch_plan(L, 1, (hipStream_t)stream), fn);
}

int32_t sphkv_work_rows_per_item(const int32_t* row_start, int32_t num_sh, int32_t num_cus, int32_t slots_per_cu) {
  const char* fn = "sphkv_work_rows_per_item";
  if (num_cus < 1 || slots_per_cu < 1) return fail(SPHKV_EINVAL, "%s: num_cus and slots_per_cu must be >= 1", fn);
  if (!row_start_ok(row_start, num_sh))
    return fail(SPHKV_EINVAL, "%s: row_start must hold num_sh + 1 non-decreasing rows >= 0", fn);
  const int64_t total = num_sh > 0 ? (int64_t)row_start[num_sh] - row_start[0] : 0;
  if (total == 0) { ok(); return 8; }
  const int64_t target = (int64_t)num_cus * slots_per_cu;
  int64_t max_len = 0;
  for (int32_t i = 0; i < num_sh; ++i) max_len = std::max<int64_t>(max_len, (int64_t)row_start[i + 1] - row_start[i]);
  int64_t lo = std::max<int64_t>(8, (total + target - 1) / target), hi = std::max(lo, max_len);
  ok();
  // more ranges than one item per CU covers: about four smaller items per CU
  if (work_items(row_start, num_sh, hi) > target) return (int32_t)std::max<int64_t>(8, (total + 4 * target - 1) / (4 * target));
  // the item total does not grow with r: the first r in [lo, hi] that fits
  while (lo < hi) {
    const int64_t mid = lo + (hi - lo) / 2;
    if (work_items(row_start, num_sh, mid) <= target) hi = mid; else lo = mid + 1;
  }
  return (int32_t)lo;
}

int64_t sphkv_work_fill(const int32_t* row_start, int32_t num_sh, int32_t rows_per_item, int32_t interleave,
                        int32_t* work, int64_t max_items, int32_t* work_start) {
  const char* fn = "sphkv_work_fill";
  if (rows_per_item < 1) return fail(SPHKV_EINVAL, "%s: rows_per_item must be >= 1", fn);
  if (!row_start_ok(row_start, num_sh))
    return fail(SPHKV_EINVAL, "%s: row_start must hold num_sh + 1 non-decreasing rows >= 0", fn);
  const int64_t n = work_items(row_start, num_sh, rows_per_item);
  if (n > INT32_MAX) return fail(SPHKV_EINVAL, "%s: more than 2^31 - 1 work items", fn);
  if (n > max_items) return fail(SPHKV_EINVAL, "%s: %lld items exceed the capacity %lld", fn, (long long)n, (long long)max_items);
  if (!work_start || (n > 0 && !work)) return fail(SPHKV_EINVAL, "%s: null pointer argument", fn);
  int32_t k = 0;
  for (int32_t i = 0; i < num_sh; ++i) {
    const int32_t b = row_start[i], e = row_start[i + 1];
    const int64_t len = (int64_t)e - b;
    const int32_t ni = len > rows_per_item ? (int32_t)((len + rows_per_item - 1) / rows_per_item) : 1;
    work_start[i] = k;
    for (int32_t j = 0; j < ni; ++j, ++k) {
      int32_t* w = work + 4 * (int64_t)k;
      w[0] = i;
      if (interleave) {
        w[1] = b + j; w[2] = e; w[3] = ni;
      } else {
        const int64_t r0 = b + (int64_t)j * rows_per_item;
        w[1] = (int32_t)r0; w[2] = (int32_t)std::min<int64_t>(e, r0 + rows_per_item); w[3] = 1;
      }
    }
  }
  work_start[num_sh] = k;
  ok();
  return n;
}

}  // extern "C"
