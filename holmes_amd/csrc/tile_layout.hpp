// Tile layout of the fused key-switch kernels (FP64 words in ksfused.hip, 64-bit words in
// wide_fused.hip): index maps, LDS exchanges and the XCD-aware tile decode, shared by both widths.
//
// A limb (N = 2^16 words) is a 256 x 256 matrix, n = 256 r + c.  A rows-kernel block owns row group
// g: the 16 rows g + 16 m.  Workspace buffers keep limbs tile-major: element (r, c) at
// wpos(r, c) = 4096 (r mod 16) + 16 c + r / 16, so each row group is one contiguous 32 KiB run
// ([column][m]) that the rows kernels read and write whole, while a cols-kernel thread holding rows
// 16 j + k (k = 0..15) of column c finds them at 4096 k + 16 c + j: 16 lanes touch 128 consecutive
// bytes (256 per column pair).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "internal.hpp"

namespace hck {

// ----------------------------------------------------------------- column slots (16 threads)
// A "slot" of 16 threads owns one 256-point column; thread j holds 16 values, either rows
// j + 16k (layout A) or rows 16j + k (layout B).  R is the slot's LDS run of 272 words.
__device__ __forceinline__ int cpad(int r) { return r + (r >> 4); }

// The 16 threads of a slot are 16 consecutive lanes of one wave and R is private to the slot, so
// an exchange needs only wave-level ordering of its LDS accesses, not a workgroup barrier: waves
// of the block run through their transforms independently.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <typename E>
__device__ __forceinline__ void col_a_to_b(E (&x)[16], E* R, int j) {
#pragma unroll
  for (int k = 0; k < 16; ++k) R[cpad(j + 16 * k)] = x[k];
  wave_sync();
#pragma unroll
  for (int k = 0; k < 16; ++k) x[k] = R[cpad(16 * j + k)];
  wave_sync();
}

template <typename E>
__device__ __forceinline__ void col_b_to_a(E (&x)[16], E* R, int j) {
#pragma unroll
  for (int k = 0; k < 16; ++k) R[cpad(16 * j + k)] = x[k];
  wave_sync();
#pragma unroll
  for (int k = 0; k < 16; ++k) x[k] = R[cpad(j + 16 * k)];
  wave_sync();
}

// ----------------------------------------------------------------- row groups (256 threads)
// The block owns row group g: rows b = g + 16 rb, rb = 0..15.  Two thread mappings: "N"
// (rb = t >> 4, j = t & 15) makes 16 consecutive lanes touch 16 consecutive words of a
// natural-layout row; "T" (rb = t & 15, j = t >> 4) makes them touch the 16 consecutive positions
// 16 g + rb of a workspace column.
__device__ __forceinline__ int ridx(int rb, int c) { return rb * 273 + c + (c >> 4); }
constexpr int kRowLds = 16 * 273 + 16;

struct RowMap {
  int rb, j;
};
__device__ __forceinline__ RowMap map_n() { return RowMap{(int)threadIdx.x >> 4, (int)threadIdx.x & 15}; }
__device__ __forceinline__ RowMap map_t() { return RowMap{(int)threadIdx.x & 15, (int)threadIdx.x >> 4}; }

// x in layout (from, A or B) -> layout (to, A or B) under mapping `to_map`
template <bool FROM_A, bool TO_A, typename E>
__device__ __forceinline__ void row_xchg(E (&x)[16], E* S, RowMap fm, RowMap tm) {
#pragma unroll
  for (int k = 0; k < 16; ++k) S[ridx(fm.rb, FROM_A ? fm.j + 16 * k : 16 * fm.j + k)] = x[k];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 16; ++k) x[k] = S[ridx(tm.rb, TO_A ? tm.j + 16 * k : 16 * tm.j + k)];
  __syncthreads();
}

// Natural position that lands in slot n under sigma_g: slot n holds the evaluation at
// psi^(2 brv(n) + 1), and sigma_g moves the evaluation at psi^(g (2 brv(n) + 1)) there.
__device__ __forceinline__ long long gal_src(long long n, uint32_t g) {
  const uint32_t e = ((2u * (__brev((uint32_t)n) >> 16) + 1u) * g) & (2u * kN - 1u);
  return (long long)(__brev((e - 1u) >> 1) >> 16);
}

// 16 raw words of one natural-layout limb for the thread at natural offset na (+16k), read through
// sigma_g (g == 1: the identity, plain coalesced loads).  The words are not converted here, so that
// a caller can issue the loads early and convert them where they are used.
__device__ __forceinline__ void load_gal_raw(uint64_t (&r)[16], const uint64_t* __restrict__ limb, long long na,
                                             uint32_t g) {
  if (g == 1u) {
#pragma unroll
    for (int k = 0; k < 16; ++k) r[k] = limb[na + 16 * k];
  } else {
#pragma unroll
    for (int k = 0; k < 16; ++k) r[k] = limb[gal_src(na + 16 * k, g)];
  }
}

// Natural-layout access in layout A under map N: thread (rb, j) owns words j + 16k of row g + 16 rb;
// 16 consecutive lanes touch 128 consecutive bytes.
__device__ __forceinline__ long long nat_a(int g) {
  const RowMap mn = map_n();
  return (long long)(g + 16 * mn.rb) * 256 + mn.j;
}

// Workspace element of row g + 16 rb (map T, layout A: columns j + 16 k): wpos = 4096 g + 16 (j + 16 k) + rb.
__device__ __forceinline__ long long ws_a(int g, int k) {
  const RowMap mt = map_t();
  return 4096LL * g + 16 * (mt.j + 16 * k) + mt.rb;
}

// Loads of one workspace tile go through a buffer descriptor: the 16 loads of a thread are 2 KiB
// apart, and as buffer loads they share one VGPR offset (the per-load part is a scalar) instead of
// 16 live 64-bit addresses.
constexpr int kBufWord3 = 0x00020000;  // raw buffer, 32-bit data format (gfx9 family)

// src_t is a tile's base and the same on every lane of a wave (every caller derives it from the
// workgroup's item and tile only); it is passed through readfirstlane so that the descriptor is
// built in scalar registers even where the compiler cannot prove the address uniform (otherwise it
// wraps each load in a loop over the distinct descriptors of the wave).
template <typename E>
__device__ __forceinline__ void load_t(E (&x)[16], const E* __restrict__ src_t, int g) {
  static_assert(sizeof(E) == 8, "workspace words are 64-bit");
  const uint64_t a = (uint64_t)src_t;
  const uint64_t au = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a) |
                      ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)) << 32);
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)au, 0, kN * 8, kBufWord3);
  const int off = (int)ws_a(g, 0) * 8;
#pragma unroll
  for (int k = 0; k < 16; ++k)
    x[k] = __builtin_bit_cast(E, __builtin_amdgcn_raw_buffer_load_b64(r, off, k * 16 * 16 * 8, 0));
}

// Grids of the tile kernels: one linear id per (ciphertext, tile).  Workgroups are dealt to the 8
// XCDs round-robin; the decode keeps every ciphertext of one tile on one XCD, one after another, so
// a key shared by the batch (a giant step) is read from HBM once per tile and served from that
// XCD's L2 to the other ciphertexts.
struct TileId {
  int tile, b;
};
__device__ __forceinline__ TileId decode_tile(int batch, int lin) {
  const int xcd = lin % kXcds, q = lin / kXcds;
  return TileId{(q / batch) * kXcds + xcd, q % batch};
}

}  // namespace hck
