// Key-switch C ABI (the fused kernels live in ksfused.hip), rotation, ModDown and rescale.
#include <hip/hip_runtime.h>

#include "../../include/holmes_ckks.h"
#include "internal.hpp"
#include "wide.hpp"

namespace hck {
namespace {

constexpr int kMaxBatch = 64;

}  // namespace
}  // namespace hck

extern "C" size_t hck_keyswitch_workspace_bytes(const hck_context* ctx, int level_limbs, int batch) {
  if (!ctx || level_limbs < 1 || level_limbs > ctx->L || batch < 0) return 0;
  const int chunk = batch < hck::kMaxBatch ? batch : hck::kMaxBatch;
  return hck::ks_fused_bytes(ctx, level_limbs, chunk);
}

extern "C" int hck_keyswitch(const hck_context* ctx, int level_limbs, int batch, const uint64_t* d,
                             int64_t d_stride, const uint64_t* const* ksk, const uint64_t* add_b,
                             int64_t add_stride, uint64_t* out_b, uint64_t* out_a, int64_t out_stride,
                             void* workspace, size_t workspace_bytes, void* stream) {
  if (!ctx || !d || !ksk || !out_b || !out_a || batch < 0) return HCK_ERR_ARG;
  if (level_limbs < 1 || level_limbs > ctx->L) return HCK_ERR_ARG;
  if (batch == 0) return HCK_OK;
  for (int b = 0; b < batch; ++b) if (!ksk[b]) return HCK_ERR_ARG;
  const int chunk = batch < hck::kMaxBatch ? batch : hck::kMaxBatch;
  if (!workspace || workspace_bytes < hck::ks_fused_bytes(ctx, level_limbs, chunk)) return HCK_ERR_WORKSPACE;
  for (int b0 = 0; b0 < batch; b0 += chunk) {
    const int nb = batch - b0 < chunk ? batch - b0 : chunk;
    int rc = hck::ks_fused(ctx, level_limbs, nb, d + (long long)b0 * d_stride, d_stride, 1u, ksk + b0,
                           add_b ? add_b + (long long)b0 * add_stride : nullptr, add_stride, nullptr, nullptr, 0,
                           out_b + (long long)b0 * out_stride, out_a + (long long)b0 * out_stride, out_stride,
                           (char*)workspace, (hipStream_t)stream);
    if (rc) return rc;
  }
  return HCK_OK;
}

extern "C" size_t hck_rotate_workspace_bytes(const hck_context* ctx, int level_limbs, int batch) {
  return hck_keyswitch_workspace_bytes(ctx, level_limbs, batch);
}

namespace {

bool galois_ok(uint32_t g) { return (g & 1u) != 0 && g < 2u * hck::kN; }

}  // namespace

// Rotation of every item b by galois (or galois_items[b]), plain or ending in the extended basis.
int hck::rotate_impl(const hck_context* ctx, int level_limbs, int batch, uint32_t galois, const uint32_t* galois_items,
                const uint64_t* c0, const uint64_t* c1, int64_t in_stride, const uint64_t* const* ksk,
                const uint64_t* acc0, const uint64_t* acc1, int64_t acc_stride, uint64_t* out0, uint64_t* out1,
                int64_t out_stride, void* workspace, size_t workspace_bytes, void* stream, bool ext) {
  if (!ctx || !c0 || !c1 || !ksk || !out0 || !out1 || batch < 0) return HCK_ERR_ARG;
  if (level_limbs < 1 || level_limbs > ctx->L) return HCK_ERR_ARG;
  if ((acc0 == nullptr) != (acc1 == nullptr)) return HCK_ERR_ARG;
  // the inputs are gathered through sigma while the outputs are written: no aliasing
  if (out0 == c0 || out0 == c1 || out1 == c0 || out1 == c1) return HCK_ERR_ARG;
  if (ext) {
    // item strides only matter between items: a single item may carry any stride (numpy views of
    // size-1 axes have stride 0)
    const int64_t ext_limb_words = (int64_t)(level_limbs + ctx->K) * hck::kN;
    if (acc0 && batch > 1 && acc_stride < ext_limb_words) return HCK_ERR_ARG;
    if (out0 == out1) return HCK_ERR_ARG;
    if (batch > 1 && out_stride < ext_limb_words) return HCK_ERR_ARG;
  }
  if (galois_items) {
    for (int b = 0; b < batch; ++b)
      if (!galois_ok(galois_items[b])) return HCK_ERR_ARG;
  } else if (!galois_ok(galois)) {
    return HCK_ERR_ARG;
  }
  if (batch == 0) return HCK_OK;
  for (int b = 0; b < batch; ++b) if (!ksk[b]) return HCK_ERR_ARG;
  const int chunk = batch < hck::kMaxBatch ? batch : hck::kMaxBatch;
  if (!workspace || workspace_bytes < hck::ks_fused_bytes(ctx, level_limbs, chunk)) return HCK_ERR_WORKSPACE;
  for (int b0 = 0; b0 < batch; b0 += chunk) {
    const int nb = batch - b0 < chunk ? batch - b0 : chunk;
    const long long oi = (long long)b0 * out_stride, ai = (long long)b0 * acc_stride;
    const uint32_t* gi = galois_items ? galois_items + b0 : nullptr;
    int rc;
    if (ext) {
      rc = hck::ks_fused(ctx, level_limbs, nb, c1 + (long long)b0 * in_stride, in_stride, galois, ksk + b0,
                         c0 + (long long)b0 * in_stride, in_stride, acc0 ? acc0 + ai : nullptr,
                         acc1 ? acc1 + ai : nullptr, acc_stride, nullptr, nullptr, 0, (char*)workspace,
                         (hipStream_t)stream, out0 + oi, out1 + oi, out_stride, gi);
    } else {
      rc = hck::ks_fused(ctx, level_limbs, nb, c1 + (long long)b0 * in_stride, in_stride, galois, ksk + b0,
                         c0 + (long long)b0 * in_stride, in_stride, acc0 ? acc0 + ai : nullptr,
                         acc1 ? acc1 + ai : nullptr, acc_stride, out0 + oi, out1 + oi, out_stride,
                         (char*)workspace, (hipStream_t)stream, nullptr, nullptr, 0, gi);
    }
    if (rc) return rc;
  }
  return HCK_OK;
}

using hck::rotate_impl;

extern "C" int hck_rotate(const hck_context* ctx, int level_limbs, int batch, uint32_t galois,
                          const uint64_t* c0, const uint64_t* c1, int64_t in_stride,
                          const uint64_t* const* ksk, const uint64_t* acc0, const uint64_t* acc1,
                          int64_t acc_stride, uint64_t* out0, uint64_t* out1, int64_t out_stride,
                          void* workspace, size_t workspace_bytes, void* stream) {
  return rotate_impl(ctx, level_limbs, batch, galois, nullptr, c0, c1, in_stride, ksk, acc0, acc1, acc_stride,
                     out0, out1, out_stride, workspace, workspace_bytes, stream, false);
}

// Rotation followed by the rescale: on the matrix-core conversion engine one pass (ks_rescaled, the
// rotation's ModDown and the rescale share the conversion), otherwise the rotation into the
// workspace and then the rescale.  Both give the same residues.
static bool rotate_rescale_fused(const hck_context* ctx, int ell) {
  return ell >= 2 && (ctx->wide ? hck::wide_fused_ok(ctx) : ctx->conv_engine == 1);
}

static size_t rotate_rescale_ks_bytes(const hck_context* ctx, int ell, int chunk) {
  if (rotate_rescale_fused(ctx, ell)) return hck::ks_rs_bytes(ctx, ell, chunk);
  const size_t ks = hck::ks_fused_bytes(ctx, ell, chunk), rs = hck::rescale_bytes(ctx, ell, chunk);
  return ks > rs ? ks : rs;
}

extern "C" size_t hck_rotate_rescale_workspace_bytes(const hck_context* ctx, int level_limbs, int batch) {
  if (!ctx || level_limbs < 2 || level_limbs > ctx->L || batch < 0) return 0;
  const int chunk = batch < hck::kMaxBatch ? batch : hck::kMaxBatch;
  const size_t mid = rotate_rescale_fused(ctx, level_limbs) ? 0 : (size_t)2 * chunk * level_limbs * hck::kN * 8;
  return rotate_rescale_ks_bytes(ctx, level_limbs, chunk) + mid;
}

extern "C" int hck_rotate_rescale(const hck_context* ctx, int level_limbs, int batch, uint32_t galois,
                                  const uint64_t* c0, const uint64_t* c1, int64_t in_stride,
                                  const uint64_t* const* ksk, uint64_t* out0, uint64_t* out1, int64_t out_stride,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  if (!ctx || !c0 || !c1 || !ksk || !out0 || !out1 || batch < 0) return HCK_ERR_ARG;
  if (level_limbs < 2 || level_limbs > ctx->L || !galois_ok(galois)) return HCK_ERR_ARG;
  if (out0 == c0 || out0 == c1 || out1 == c0 || out1 == c1 || out0 == out1) return HCK_ERR_ARG;
  {
    // no partial overlaps either: the fused pass reads c0 through the automorphism (any position of
    // a limb) while tiles of other limbs and items store the outputs
    const int64_t in_len = (int64_t)level_limbs * hck::kN, out_len = (int64_t)(level_limbs - 1) * hck::kN;
    for (const uint64_t* o : {out0, out1})
      for (const uint64_t* c : {c0, c1})
        if (hck::batches_overlap(o, out_stride, out_len, c, in_stride, in_len, batch)) return HCK_ERR_ARG;
    if (hck::batches_overlap(out0, out_stride, out_len, out1, out_stride, out_len, batch)) return HCK_ERR_ARG;
  }
  if (batch == 0) return HCK_OK;
  for (int b = 0; b < batch; ++b) if (!ksk[b]) return HCK_ERR_ARG;
  if (!workspace || workspace_bytes < hck_rotate_rescale_workspace_bytes(ctx, level_limbs, batch))
    return HCK_ERR_WORKSPACE;
  const int ell = level_limbs;
  const int chunk = batch < hck::kMaxBatch ? batch : hck::kMaxBatch;
  const bool fused = rotate_rescale_fused(ctx, ell);
  char* ks_ws = (char*)workspace;
  uint64_t* mid = (uint64_t*)(ks_ws + rotate_rescale_ks_bytes(ctx, ell, chunk));  // [2][chunk][ell][N] (unfused)
  const long long poly = (long long)ell * hck::kN;
  hipStream_t s = (hipStream_t)stream;
  for (int b0 = 0; b0 < batch; b0 += chunk) {
    const int nb = batch - b0 < chunk ? batch - b0 : chunk;
    const long long ii = (long long)b0 * in_stride, oi = (long long)b0 * out_stride;
    int rc;
    if (fused) {
      rc = hck::ks_rescaled(ctx, ell, nb, c1 + ii, in_stride, galois, ksk + b0, c0 + ii, in_stride, nullptr, nullptr,
                            0, out0 + oi, out1 + oi, out_stride, ks_ws, s);
      if (rc) return rc;
      continue;
    }
    rc = hck::ks_fused(ctx, ell, nb, c1 + ii, in_stride, galois, ksk + b0, c0 + ii, in_stride, nullptr, nullptr, 0,
                       mid, mid + (long long)nb * poly, poly, ks_ws, s);
    if (rc) return rc;
    rc = hck::rescale_fused(ctx, ell, nb, mid, poly, out0 + oi, out_stride, ks_ws, s);
    if (rc) return rc;
    rc = hck::rescale_fused(ctx, ell, nb, mid + (long long)nb * poly, poly, out1 + oi, out_stride, ks_ws, s);
    if (rc) return rc;
  }
  return HCK_OK;
}

extern "C" int hck_rotate_many(const hck_context* ctx, int level_limbs, int batch, const uint32_t* galois,
                               const uint64_t* c0, const uint64_t* c1, int64_t in_stride,
                               const uint64_t* const* ksk, const uint64_t* acc0, const uint64_t* acc1,
                               int64_t acc_stride, uint64_t* out0, uint64_t* out1, int64_t out_stride,
                               void* workspace, size_t workspace_bytes, void* stream) {
  if (!galois) return HCK_ERR_ARG;
  return rotate_impl(ctx, level_limbs, batch, 1u, galois, c0, c1, in_stride, ksk, acc0, acc1, acc_stride,
                     out0, out1, out_stride, workspace, workspace_bytes, stream, false);
}

extern "C" int hck_rotate_ext(const hck_context* ctx, int level_limbs, int batch, uint32_t galois,
                              const uint64_t* c0, const uint64_t* c1, int64_t in_stride,
                              const uint64_t* const* ksk, const uint64_t* acc0, const uint64_t* acc1,
                              int64_t acc_stride, uint64_t* out0, uint64_t* out1, int64_t out_stride,
                              void* workspace, size_t workspace_bytes, void* stream) {
  return rotate_impl(ctx, level_limbs, batch, galois, nullptr, c0, c1, in_stride, ksk, acc0, acc1, acc_stride,
                     out0, out1, out_stride, workspace, workspace_bytes, stream, true);
}

extern "C" int hck_rotate_ext_many(const hck_context* ctx, int level_limbs, int batch, const uint32_t* galois,
                                   const uint64_t* c0, const uint64_t* c1, int64_t in_stride,
                                   const uint64_t* const* ksk, const uint64_t* acc0, const uint64_t* acc1,
                                   int64_t acc_stride, uint64_t* out0, uint64_t* out1, int64_t out_stride,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  if (!galois) return HCK_ERR_ARG;
  return rotate_impl(ctx, level_limbs, batch, 1u, galois, c0, c1, in_stride, ksk, acc0, acc1, acc_stride,
                     out0, out1, out_stride, workspace, workspace_bytes, stream, true);
}

extern "C" int hck_rotate_ext_sum(const hck_context* ctx, int level_limbs, int outputs, int group,
                                  const uint32_t* galois, const uint64_t* c0, const uint64_t* c1, int64_t in_stride,
                                  const uint64_t* const* ksk, const uint64_t* acc0, const uint64_t* acc1,
                                  int64_t acc_stride, uint64_t* out0, uint64_t* out1, int64_t out_stride,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  if (!ctx || !galois || !c0 || !c1 || !ksk || !out0 || !out1) return HCK_ERR_ARG;
  if (level_limbs < 1 || level_limbs > ctx->L || outputs < 0 || group < 1) return HCK_ERR_ARG;
  if ((long long)outputs * group > hck::kMaxBatch) return HCK_ERR_ARG;
  if ((acc0 == nullptr) != (acc1 == nullptr) || out0 == out1) return HCK_ERR_ARG;
  if (out0 == c0 || out0 == c1 || out1 == c0 || out1 == c1) return HCK_ERR_ARG;
  const int64_t ext_limb_words = (int64_t)(level_limbs + ctx->K) * hck::kN;
  if (outputs > 1 && (out_stride < ext_limb_words || (acc0 && acc_stride < ext_limb_words))) return HCK_ERR_ARG;
  for (int m = 0; m < group; ++m)
    if (!galois_ok(galois[m]) || !ksk[m]) return HCK_ERR_ARG;
  if (outputs == 0) return HCK_OK;
  const int batch = outputs * group;
  if (!workspace || workspace_bytes < hck::ks_fused_bytes(ctx, level_limbs, batch)) return HCK_ERR_WORKSPACE;
  uint32_t gi[hck::kMaxBatch];
  const uint64_t* keys[hck::kMaxBatch];
  for (int m = 0; m < group; ++m)
    for (int o = 0; o < outputs; ++o) {
      gi[m * outputs + o] = galois[m];
      keys[m * outputs + o] = ksk[m];
    }
  return hck::ks_fused_sum(ctx, level_limbs, outputs, group, c1, in_stride, gi, keys, c0, in_stride, acc0, acc1,
                           acc_stride, out0, out1, out_stride, (char*)workspace, (hipStream_t)stream);
}

extern "C" size_t hck_rotate_hoist_digits_bytes(const hck_context* ctx, int level_limbs, int inputs) {
  if (!ctx || level_limbs < 1 || level_limbs > ctx->L || inputs < 0) return 0;
  const size_t beta = (size_t)(level_limbs + ctx->alpha - 1) / ctx->alpha;
  return (size_t)inputs * beta * (size_t)(level_limbs + ctx->K) * hck::kN * 8;
}

extern "C" size_t hck_rotate_hoist_workspace_bytes(const hck_context* ctx, int level_limbs, int inputs, int items) {
  if (!ctx || level_limbs < 1 || level_limbs > ctx->L || inputs < 0 || items < 0) return 0;
  const size_t a = hck::ks_hoist_bytes(ctx, level_limbs, inputs), b = hck::ks_hoisted_bytes(ctx, level_limbs, items);
  return a > b ? a : b;
}

extern "C" int hck_rotate_hoist_prepare(const hck_context* ctx, int level_limbs, int inputs, const uint64_t* c1,
                                        int64_t in_stride, uint64_t* digits, void* workspace, size_t workspace_bytes,
                                        void* stream) {
  if (!ctx || !c1 || !digits || level_limbs < 1 || level_limbs > ctx->L || inputs < 0) return HCK_ERR_ARG;
  if (inputs > 1 && in_stride < (int64_t)level_limbs * hck::kN) return HCK_ERR_ARG;
  if (inputs == 0) return HCK_OK;
  if (!workspace || workspace_bytes < hck::ks_hoist_bytes(ctx, level_limbs, inputs)) return HCK_ERR_WORKSPACE;
  return hck::ks_hoist(ctx, level_limbs, inputs, c1, in_stride, digits, (char*)workspace, (hipStream_t)stream);
}

extern "C" int hck_rotate_hoisted(const hck_context* ctx, int level_limbs, int inputs, int items,
                                  const uint32_t* galois, const uint64_t* c0, const uint64_t* c1, int64_t in_stride,
                                  const uint64_t* digits, const uint64_t* const* ksk, uint64_t* out0, uint64_t* out1,
                                  int64_t out_stride, void* workspace, size_t workspace_bytes, void* stream) {
  if (!ctx || !galois || !c0 || !c1 || !digits || !ksk || !out0 || !out1) return HCK_ERR_ARG;
  if (level_limbs < 1 || level_limbs > ctx->L || inputs < 1 || items < 0) return HCK_ERR_ARG;
  const int64_t limb_words = (int64_t)level_limbs * hck::kN;
  if (inputs > 1 && in_stride < limb_words) return HCK_ERR_ARG;
  if (items > 1 && out_stride < limb_words) return HCK_ERR_ARG;
  if (out0 == out1 || out0 == c0 || out0 == c1 || out1 == c0 || out1 == c1) return HCK_ERR_ARG;
  for (int i = 0; i < items; ++i)
    if (!galois_ok(galois[i]) || !ksk[i]) return HCK_ERR_ARG;
  if (items == 0) return HCK_OK;
  if (!workspace || workspace_bytes < hck::ks_hoisted_bytes(ctx, level_limbs, items)) return HCK_ERR_WORKSPACE;
  return hck::ks_hoisted(ctx, level_limbs, inputs, items, galois, ksk, c0, c1, in_stride, digits, out0, out1,
                         out_stride, (char*)workspace, (hipStream_t)stream);
}

extern "C" size_t hck_moddown_workspace_bytes(const hck_context* ctx, int level_limbs, int polys) {
  if (!ctx || level_limbs < 1 || level_limbs > ctx->L || polys < 0) return 0;
  const int chunk = polys < 65535 ? polys : 65535;
  return hck::moddown_bytes(ctx, level_limbs, chunk);
}

extern "C" int hck_moddown(const hck_context* ctx, int level_limbs, int polys, const uint64_t* in,
                           int64_t in_stride, uint64_t* out, int64_t out_stride, void* workspace,
                           size_t workspace_bytes, void* stream) {
  if (!ctx || !in || !out || polys < 0 || polys > 65535) return HCK_ERR_ARG;
  if (level_limbs < 1 || level_limbs > ctx->L) return HCK_ERR_ARG;
  if (polys > 1 && (in_stride < (int64_t)(level_limbs + ctx->K) * hck::kN ||
                    out_stride < (int64_t)level_limbs * hck::kN))
    return HCK_ERR_ARG;
  if (polys == 0) return HCK_OK;
  if (!workspace || workspace_bytes < hck::moddown_bytes(ctx, level_limbs, polys)) return HCK_ERR_WORKSPACE;
  return hck::moddown_ext(ctx, level_limbs, polys, in, in_stride, out, out_stride, (char*)workspace,
                          (hipStream_t)stream);
}

extern "C" size_t hck_rescale_workspace_bytes(const hck_context* ctx, int level_limbs, int polys) {
  if (!ctx || level_limbs < 2 || level_limbs > ctx->L || polys < 0) return 0;
  return hck::rescale_bytes(ctx, level_limbs, polys);
}

extern "C" int hck_rescale(const hck_context* ctx, int level_limbs, int polys, const uint64_t* in,
                           int64_t in_stride, uint64_t* out, int64_t out_stride, void* workspace,
                           size_t workspace_bytes, void* stream) {
  if (!ctx || !in || !out || polys < 0 || polys > 65535) return HCK_ERR_ARG;
  if (level_limbs < 2 || level_limbs > ctx->L) return HCK_ERR_ARG;
  if (polys == 0) return HCK_OK;
  const int64_t n = hck::kN;
  if (polys > 1 && (in_stride < level_limbs * n || out_stride < (level_limbs - 1) * n)) return HCK_ERR_ARG;
  // The finish kernel reads in[p][i] and writes out[p][i] in the same thread: in place is safe with
  // equal strides; any other overlap lets one poly's output overwrite input another block still reads.
  {
    const uint64_t* in_end = in + (int64_t)(polys - 1) * in_stride + level_limbs * n;
    const uint64_t* out_end = out + (int64_t)(polys - 1) * out_stride + (level_limbs - 1) * n;
    const bool overlap = in < out_end && out < in_end;
    if (overlap && !(in == out && in_stride == out_stride)) return HCK_ERR_ARG;
  }
  if (!workspace || workspace_bytes < hck::rescale_bytes(ctx, level_limbs, polys)) return HCK_ERR_WORKSPACE;
  return hck::rescale_fused(ctx, level_limbs, polys, in, in_stride, out, out_stride, (char*)workspace,
                            (hipStream_t)stream);
}

extern "C" size_t hck_modraise_workspace_bytes(const hck_context* ctx, int to_limbs, int polys) {
  if (!ctx || to_limbs < 2 || to_limbs > ctx->L || polys < 0) return 0;
  return hck::modraise_bytes(ctx, to_limbs, polys);
}

extern "C" int hck_modraise(const hck_context* ctx, int to_limbs, int polys, const uint64_t* in, int64_t in_stride,
                            uint64_t* out, int64_t out_stride, void* workspace, size_t workspace_bytes, void* stream) {
  if (!ctx || !in || !out || polys < 0 || polys > 65535) return HCK_ERR_ARG;
  if (to_limbs < 2 || to_limbs > ctx->L) return HCK_ERR_ARG;
  if (polys > 1 && (in_stride < hck::kN || out_stride < (int64_t)to_limbs * hck::kN)) return HCK_ERR_ARG;
  if (in == out) return HCK_ERR_ARG;
  if (polys == 0) return HCK_OK;
  if (!workspace || workspace_bytes < hck::modraise_bytes(ctx, to_limbs, polys)) return HCK_ERR_WORKSPACE;
  return hck::modraise_fused(ctx, to_limbs, polys, in, in_stride, out, out_stride, (char*)workspace,
                             (hipStream_t)stream);
}
