// Exchange tiles of the fused backward kernels: P' = a P and G of a 64-query
// tile, written query-centric (phase 1) and read back transposed as the B
// operands of the key-centric dK/dV products (phase 2).
//
// Layout: for query group j and band slot sl (key group j + sl of the 128
// keys of blocks t-1, t), a [16 query][16 key] bf16 sub-tile with a 32-byte
// row whose 8-byte piece p (keys 4p .. 4p+3) sits at position p ^ xsw(r).
// Phase-1 stores (lane (g,c): query c, keys 4g..4g+3) and phase-2
// transposed reads (16 lanes: 4 rows x 16 keys) each touch 512 contiguous
// bytes per wave instruction.  8-byte accesses are served 32 lanes at a
// time over 64 four-byte banks: unswizzled, the stores of lanes 0-31 (keys
// 0..7 of rows 0..15) put rows r and r + 8 on the same banks; xsw moves rows
// 8..15 to the other half of the row (bank conflicts per LDS access of the
// fused backward 0.41 -> 0.20), and the transposed reads still cover 256
// contiguous bytes per 32 lanes.
#pragma once

#include "mfma_common.h"

namespace tension {

constexpr int kXSlots = 5;                    // 16-key groups in the band of 16 queries (W <= 64)
constexpr int kXSub = 16 * 16;                // bf16 elements of one sub-tile
constexpr int kXElems = 4 * kXSlots * kXSub;  // one exchange tensor (4 query groups)

__device__ __forceinline__ int xsw(int r) { return ((r >> 3) & 1) << 1; }

__device__ __forceinline__ void x_put(bf16* X, int j, int sl, int g, int c, const float* v4) {
  u16x4 o;
#pragma unroll
  for (int r = 0; r < 4; ++r) o[r] = bf16_bits((bf16)v4[r]);
  *(u16x4*)(X + (j * kXSlots + sl) * kXSub + c * 16 + 4 * (g ^ xsw(c))) = o;
}

__device__ __forceinline__ void x_put_bits(bf16* X, int j, int sl, int g, int c, u16x4 v) {
  *(u16x4*)(X + (j * kXSlots + sl) * kXSub + c * 16 + 4 * (g ^ xsw(c))) = v;
}

__device__ __forceinline__ u16x4 bf16x4_bits(float a, float b, float c, float d) {
  u16x4 o;
  o[0] = bf16_bits((bf16)a); o[1] = bf16_bits((bf16)b);
  o[2] = bf16_bits((bf16)c); o[3] = bf16_bits((bf16)d);
  return o;
}

__device__ __forceinline__ bf16x8 join_bits(u16x4 lo, u16x4 hi) {
  u16x8 r;
  r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
  r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
  return __builtin_bit_cast(bf16x8, r);
}

// B operand of a product contracting over the 32 queries of groups j0, j0+1:
// lane (g, c) gets key c of the sub-tiles, queries {4g..4g+3} of group j0
// and of group j0+1 (the tile-row order dt_tr8 gives the A operand).  An
// absent sub-tile (no slot of that query group covers the key group) reads
// as zeros.
__device__ __forceinline__ bf16x8 x_pair(const bf16* X, int j0, int sl0, bool ok0, int sl1, bool ok1, int g,
                                         int l16) {
  const int row = 4 * g + (l16 >> 2);
  const int off = row * 16 + 4 * ((l16 & 3) ^ xsw(row));
  s16x4 lo = {0, 0, 0, 0}, hi = {0, 0, 0, 0};
  if (ok0) lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(X + (j0 * kXSlots + sl0) * kXSub + off));
  if (ok1)
    hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(X + ((j0 + 1) * kXSlots + sl1) * kXSub + off));
  u16x8 r;
  r[0] = (unsigned short)lo[0]; r[1] = (unsigned short)lo[1];
  r[2] = (unsigned short)lo[2]; r[3] = (unsigned short)lo[3];
  r[4] = (unsigned short)hi[0]; r[5] = (unsigned short)hi[1];
  r[6] = (unsigned short)hi[2]; r[7] = (unsigned short)hi[3];
  return __builtin_bit_cast(bf16x8, r);
}

}  // namespace tension
