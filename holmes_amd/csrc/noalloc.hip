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

// Items per launch that fit the scratch array at this level (at most 64, the key switch's own launch
// size); 0 when not even one item fits.
int items_per_launch(const hck_context* ctx, int level_limbs) {
  int n = 64;
  while (n > 0 && hck::ks_fused_bytes(ctx, level_limbs, n) > kScratchBytes) --n;
  return n;
}

}  // namespace

extern "C" size_t hck_rotate_noalloc_limit(const hck_context* ctx, int level_limbs) {
  // any batch runs (in launches of as many items as fit) once one item fits the array
  if (!ctx || level_limbs < 1 || level_limbs > ctx->L) return 0;
  return items_per_launch(ctx, level_limbs) > 0 ? (size_t)1 << 30 : 0;
}

extern "C" int hck_rotate_noalloc(const hck_context* ctx, int level_limbs, int batch, uint32_t galois,
                                  const uint64_t* c0, const uint64_t* c1, int64_t in_stride,
                                  const uint64_t* const* ksk, const uint64_t* acc0, const uint64_t* acc1,
                                  int64_t acc_stride, uint64_t* out0, uint64_t* out1, int64_t out_stride,
                                  void* stream) {
  if (!ctx || batch < 0 || level_limbs < 1 || level_limbs > ctx->L) return HCK_ERR_ARG;
  const int per = items_per_launch(ctx, level_limbs);
  if (per < 1) return HCK_ERR_SCRATCH;
  if (batch == 0)
    return hck::rotate_impl(ctx, level_limbs, 0, galois, nullptr, c0, c1, in_stride, ksk, acc0, acc1, acc_stride,
                            out0, out1, out_stride, nullptr, 0, stream, false);
  // every per-item argument is checked before the first launch, so an error launches nothing
  if (!ksk) return HCK_ERR_ARG;
  for (int b = 0; b < batch; ++b)
    if (!ksk[b]) return HCK_ERR_ARG;
  void* ws = nullptr;
  const int rc0 = scratch_address(&ws);
  if (rc0) return rc0;
  // launches of `per` items, in order on one stream, each reusing the whole array
  for (int i0 = 0; i0 < batch; i0 += per) {
    const int nb = batch - i0 < per ? batch - i0 : per;
    const int64_t ii = (int64_t)i0 * in_stride, ai = (int64_t)i0 * acc_stride, oi = (int64_t)i0 * out_stride;
    const int rc = hck::rotate_impl(ctx, level_limbs, nb, galois, nullptr, c0 ? c0 + ii : nullptr,
                                    c1 ? c1 + ii : nullptr, in_stride, ksk + i0, acc0 ? acc0 + ai : nullptr,
                                    acc1 ? acc1 + ai : nullptr, acc_stride, out0 ? out0 + oi : nullptr,
                                    out1 ? out1 + oi : nullptr, out_stride, ws, kScratchBytes, stream, false);
    if (rc) return rc;
  }
  return HCK_OK;
}
