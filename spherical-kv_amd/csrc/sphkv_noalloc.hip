// sphkv_decode_paged_noalloc: the paged decode with its workspace in a
// file-scope device array instead of caller or library allocations, for
// callers that cannot allocate (code under HIP graph capture, serving loops
// that forbid allocation).  Host code only, besides the array.
//
// The array `scratch` holds the decode's per-item partials followed by its 16
// status bytes, exactly the layout of sphkv_decode_paged's workspace.  Each
// GPU the library runs on holds its own copy until the process ends.  Its
// device address is looked up once per device, on the entry point's first
// call on that device (hipGetSymbolAddress with that device current), and
// only that address is handed to kernels: the array's name is a host-side
// stand-in in host code.
//
// Every call on a GPU shares that GPU's array and leaves the last call's
// partials in it; calls that overlap on one GPU (concurrent streams or
// threads) race.  Nothing needs clearing per call: every work item's partial
// is written in full before the merge reads it, and the status counter is
// zero when the module loads and is reset by every call's merge.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/sphkv.h"
#include "sphkv_internal.h"

static __device__ __align__(256) uint8_t scratch[SPHKV_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
void* g_ptr[kMaxDevices] = {};
std::mutex g_mu;

// Device address of this device's `scratch`, looked up on first use.
hipError_t scratch_ptr(int dev, void** out) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_ptr[dev] = p;
  }
  *out = g_ptr[dev];
  return hipSuccess;
}

}  // namespace

namespace sphkv {
int noalloc_fail(int code, const char* fmt, ...);
int noalloc_decode(const char* fn, const uint8_t* pages, int64_t pages_bytes, const int32_t* ptable,
                   const int32_t* vslot, const int32_t* positions, int32_t num_rows, const uint16_t* v_pool,
                   int64_t num_vpages, const float* cb1, const float* cb2, const float* cb3,
                   const int32_t* work, int32_t num_items, const int32_t* work_start, int32_t num_seqs,
                   int32_t num_kv, int32_t gqa, const uint16_t* q, uint16_t* out, void* workspace,
                   int64_t workspace_bytes, int32_t dh, int32_t page_size, float sm_scale, double rope_theta,
                   void* stream);
}  // namespace sphkv

extern "C" int sphkv_decode_paged_noalloc(const uint8_t* pages, int64_t pages_bytes, const int32_t* ptable,
                                          const int32_t* vslot, const int32_t* positions, int32_t num_rows,
                                          const uint16_t* v_pool, int64_t num_vpages,
                                          const float* cb1, const float* cb2, const float* cb3,
                                          const int32_t* work, int32_t num_items, const int32_t* work_start,
                                          int32_t num_seqs, int32_t num_kv, int32_t gqa,
                                          const uint16_t* q, uint16_t* out,
                                          int32_t dh, int32_t page_size, float sm_scale, double rope_theta,
                                          void* stream) {
  const char* fn = "sphkv_decode_paged_noalloc";
  const int64_t need = sphkv_decode_paged_workspace_bytes(num_items, gqa, dh);
  if (need > (int64_t)SPHKV_NOALLOC_SCRATCH_BYTES)
    return sphkv::noalloc_fail(SPHKV_EINVAL,
                               "%s: %d work items need %lld bytes of scratch, more than its %lld bytes "
                               "(use sphkv_decode_paged with a workspace, or fewer, larger items)",
                               fn, num_items, (long long)need, (long long)SPHKV_NOALLOC_SCRATCH_BYTES);
  if (num_seqs == 0)                        // nothing to decode: validated without any device access
    return sphkv::noalloc_decode(fn, pages, pages_bytes, ptable, vslot, positions, num_rows, v_pool, num_vpages,
                                 cb1, cb2, cb3, work, num_items, work_start, num_seqs, num_kv, gqa, q, out,
                                 nullptr, need, dh, page_size, sm_scale, rope_theta, stream);
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return sphkv::noalloc_fail(SPHKV_EDEVICE, "%s: no current device (%s)", fn, hipGetErrorString(e));
  void* ws = nullptr;
  e = scratch_ptr(dev, &ws);
  if (e != hipSuccess)
    return sphkv::noalloc_fail(SPHKV_EDEVICE, "%s: scratch address of device %d: %s", fn, dev,
                               hipGetErrorString(e));
  return sphkv::noalloc_decode(fn, pages, pages_bytes, ptable, vslot, positions, num_rows, v_pool, num_vpages,
                               cb1, cb2, cb3, work, num_items, work_start, num_seqs, num_kv, gqa, q, out, ws,
                               need, dh, page_size, sm_scale, rope_theta, stream);
}
