// Compress arguments and device helpers shared by the general compress kernel
// (tq_codec.hip) and the MFMA compress kernel (tq_compress_fast.hip).
#pragma once

#include "tq_common.h"

namespace tq {

struct CompressArgs {
  const void* x;
  int x_dtype;
  int64_t x_hs;
  tq_span span;
  tq_store dst;
  const float* rot;
  const float* bnd_hi;
  const float* bnd_lo;
  const float* cen_hi;
  const float* cen_lo;
  const float* proj;
  int d;  // head_dim
  int bits_hi, bits_lo, split, qjl_m;
  int row_hi, row_lo, row_sign;
};

// float64 sum of squares of row[0, D) in the library's norm order: 32-dim
// blocks, each summed sequentially from 0, block sums combined pairwise level
// by level ((B0+B1)+(B2+B3) for D = 128). Squares of fp16 / fp32 values are
// exact in float64, so fma(x, x, s) rounds once like s + x*x.
template <int D>
__device__ inline double sumsq_blocks(const float* row) {
  constexpr int NB = D / 32;
  double blk[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    double s = 0.0;
    for (int i = 0; i < 32; ++i) {
      const double xi = (double)row[32 * b + i];
      s = fma(xi, xi, s);
    }
    blk[b] = s;
  }
#pragma unroll
  for (int w = 1; w < NB; w *= 2)
#pragma unroll
    for (int b = 0; b + w < NB; b += 2 * w) blk[b] += blk[b + w];
  return blk[0];
}

template <int BITS>
__device__ inline void store_codes(uint8_t* dst, const uint32_t (&code)[32]) {
  uint32_t w[BITS];
  pack32<BITS>(code, w);
  uint32_t* d32 = reinterpret_cast<uint32_t*>(dst);
#pragma unroll
  for (int i = 0; i < BITS; ++i) d32[i] = w[i];
}

// MFMA compress for fp16 inputs with head_dim 128 and no QJL sketch; returns
// 1 when it launched, 0 when the arguments need the general kernel.
int launch_compress_fast(const CompressArgs& a, hipStream_t s);

}  // namespace tq
