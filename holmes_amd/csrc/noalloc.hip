// hck_rotate_noalloc: hck_rotate for callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc).  The key-switch workspace comes
// from a fixed device array of this file instead of a caller's buffer; everything else is
// hck_rotate's code path (same kernels, same results).
//
// The array is a device global: each GPU that loads the library holds its own copy, at its own
// address, until the process ends.  Host code never uses the array's name as an address (on the host
// it names a stand-in, not device memory): the first call on a device resolves that device's
// address with hipGetSymbolAddress, and kernels only ever receive that pointer.  Every call on one
// GPU shares the array, so calls that overlap on one GPU (different streams, different threads)
// race; calls on one stream are ordered.  The key switch writes every workspace word it reads, so
// nothing needs clearing between calls.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/holmes_ckks.h"
#include "internal.hpp"

namespace {

constexpr size_t kScratchBytes = HCK_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) char scratch[kScratchBytes];

std::mutex g_lock;
void* g_scratch_ptr[kMaxDevices];  // per device, resolved once

// The current device's address of `scratch` (0 or a HIP error / HCK code).
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return HCK_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> guard(g_lock);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return HCK_ERR_UNSUPPORTED;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return HCK_OK;
}

}  // namespace

extern "C" size_t hck_rotate_noalloc_limit(const hck_context* ctx, int level_limbs) {
  // largest batch whose launches (<= 64 items each) fit the scratch array at this level
  if (!ctx || level_limbs < 1 || level_limbs > ctx->L) return 0;
  const size_t one = hck::ks_fused_bytes(ctx, level_limbs, 1);
  const size_t fit = one ? kScratchBytes / one : 0;
  return fit >= 64 ? (size_t)1 << 30 : fit;  // 64 items fit: any batch (it runs in 64-item launches)
}

extern "C" int hck_rotate_noalloc(const hck_context* ctx, int level_limbs, int batch, uint32_t galois,
                                  const uint64_t* c0, const uint64_t* c1, int64_t in_stride,
                                  const uint64_t* const* ksk, const uint64_t* acc0, const uint64_t* acc1,
                                  int64_t acc_stride, uint64_t* out0, uint64_t* out1, int64_t out_stride,
                                  void* stream) {
  if (!ctx || batch < 0 || level_limbs < 1 || level_limbs > ctx->L) return HCK_ERR_ARG;
  const int chunk = batch < 64 ? batch : 64;
  const size_t need = hck::ks_fused_bytes(ctx, level_limbs, chunk);
  if (need > kScratchBytes) return HCK_ERR_SCRATCH;
  void* ws = nullptr;
  if (batch > 0) {
    const int rc = scratch_address(&ws);
    if (rc) return rc;
  }
  return hck::rotate_impl(ctx, level_limbs, batch, galois, nullptr, c0, c1, in_stride, ksk, acc0, acc1, acc_stride,
                          out0, out1, out_stride, ws, kScratchBytes, stream, false);
}
