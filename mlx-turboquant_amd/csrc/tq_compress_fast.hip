// MFMA compress for TurboQuant on gfx950: fp16 vectors of head_dim 128 ->
// norm, rotation, quantization and bit packing in one persistent kernel
// (replaces TurboQuantKVCache._quantize_kv / _quantize_kv_fractional,
// mlx_turboquant/cache.py:232-274, for fp16 inputs without a QJL sketch).
//
// Rotation (rotation.py:55-65, y = x_n R^T) runs on 16x16x32 f16 MFMAs against
// 256*R split into an fp16 high part H and an fp16 remainder L. The input x is
// exact in fp16, so z = x (256 R)^T = x H^T + x L^T takes two passes and no
// split of x; the factor 256 keeps L clear of the fp16 subnormal range. Then
// y = z / (256 max(n, 1e-10)). The result differs from the exact y by about
// 2^-22 of sum_i |x_n,i R_ji| plus the float32 accumulation, inside the float32
// dot-product band within which the reference's own GEMM does not fix a code.
//
// Work split: a workgroup of 4 waves walks tiles of 64 vectors of one (batch,
// head) row. Wave w owns rotated dims [32w, 32w+32) and keeps its rows of 256R
// as MFMA A operands in registers for the whole launch. Per tile:
//   1. the x tile (16 KB, loaded one tile ahead) is stored to LDS;
//   2. each thread sums the squares of 32 dims of one vector in float64 and
//      lanes 4v..4v+3 combine them pairwise (the library's norm order);
//   3. each wave multiplies its A operands by the tile (B = x^T read from LDS):
//      D[m][n] = rotated dim 32w + 16*n2 + m of vector n; lane (n = l & 15,
//      g = l >> 4) holds dims 32w + 16*n2 + 4g + e, e = 0..3;
//   4. coordinates are scaled, quantized (count of boundaries below, ties low,
//      NaN -> 0; codebook.py:220-223) and written as code bytes to LDS;
//   5. each thread packs 32 codes of one vector into BITS dwords (LSB-first
//      bitstream, packing.py) and stores them.

#include <math.h>

#include "tq_codec.h"

namespace tq {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int CD = 128;        // head_dim
constexpr int CT = 64;         // vectors per tile
constexpr int CTHR = 256;      // threads per workgroup (4 waves)
constexpr int XS = 272;        // LDS row stride of the x tile, bytes (256 + 16: conflict-free b128 reads)
constexpr int CS = 144;        // LDS row stride of the code tile, bytes
constexpr float RSC = 256.f;   // scale of R before the fp16 split

constexpr uint32_t L_X0 = 0;
constexpr uint32_t L_X1 = CT * XS;
constexpr uint32_t L_CODES = 2 * CT * XS;
constexpr uint32_t L_SCALE = L_CODES + CT * CS;
constexpr uint32_t L_TOTAL = L_SCALE + CT * 4;

__device__ inline half8 as_h8(u4 v) { return __builtin_bit_cast(half8, v); }

struct Tile {
  int id;          // tile index; >= total: none left
  int row;         // (batch, head) row
  int nv;          // vectors in the tile
  int src0, dst0;  // first source / destination token of the tile
};

template <int NB>
__device__ inline uint32_t quant(float y, const float (&b)[NB]) {
  uint32_t idx = 0;
#pragma unroll
  for (int k = 0; k < NB; ++k) idx += y > b[k] ? 1u : 0u;
  return idx;
}

template <int BH, int BL>
__global__ __launch_bounds__(CTHR) void compress_fast_kernel(CompressArgs a, int tiles_per_row, int total) {
  __shared__ __align__(16) uint8_t smem[L_TOTAL];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int m = lane & 15, g = lane >> 4;
  const bool whi = 32 * w < a.split;  // this wave's dims use the high-width codebook

  // A operands: rows 32w + 16*n2 + m of 256R, k-slots 32*kb + 8*g + e
  half8 ah[2][4], al[2][4];
#pragma unroll
  for (int n2 = 0; n2 < 2; ++n2)
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const float* src = a.rot + (32 * w + 16 * n2 + m) * CD + 32 * kb + 8 * g;
      const float4 f0 = *reinterpret_cast<const float4*>(src);
      const float4 f1 = *reinterpret_cast<const float4*>(src + 4);
      const float f[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = RSC * f[e];
        const _Float16 h = (_Float16)v;
        ah[n2][kb][e] = h;
        al[n2][kb][e] = (_Float16)(v - (float)h);
      }
    }
  constexpr int NBH = (1 << BH) - 1, NBL = (1 << BL) - 1;
  float bh[NBH], bl[NBL];
#pragma unroll
  for (int k = 0; k < NBH; ++k) bh[k] = a.bnd_hi[k];
#pragma unroll
  for (int k = 0; k < NBL; ++k) bl[k] = a.bnd_lo[k];

  // next non-empty tile at or after `id` in this workgroup's sequence
  auto make_tile = [&](int id) {
    Tile t;
    t.id = id;
    t.row = t.nv = t.src0 = t.dst0 = 0;
    for (; t.id < total; t.id += gridDim.x) {
      t.row = t.id / tiles_per_row;
      const int t0 = (t.id - t.row * tiles_per_row) * CT;
      const int b = t.row / a.span.heads;
      const int n = a.span.n_tok_b ? a.span.n_tok_b[b] : a.span.n_tok;
      t.nv = min(CT, n - t0);
      if (t.nv > 0) {
        t.src0 = (a.span.src_tok0_b ? a.span.src_tok0_b[b] : 0) + t0;
        t.dst0 = (a.span.dst_tok0_b ? a.span.dst_tok0_b[b] : 0) + t0;
        break;
      }
    }
    return t;
  };

  // x tile: 1024 chunks of 16 bytes, chunk c = vector c >> 4, bytes 16*(c & 15);
  // vectors past the tile's end re-read its last vector (results not stored)
  u4 xr[4];
  auto load_x = [&](const Tile& t) {
    const uint8_t* base = static_cast<const uint8_t*>(a.x) + ((int64_t)t.row * a.x_hs + (int64_t)t.src0 * CD) * 2;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + CTHR * i;
      const int v = min(c >> 4, t.nv - 1);
      xr[i] = *reinterpret_cast<const u4*>(base + v * 256 + (c & 15) * 16);
    }
  };

  Tile cur = make_tile(blockIdx.x);
  if (cur.id >= total) return;
  load_x(cur);
  uint32_t xoff = L_X0;
  float* scl = reinterpret_cast<float*>(smem + L_SCALE);
  while (true) {
    uint8_t* xb = smem + xoff;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + CTHR * i;
      *reinterpret_cast<u4*>(xb + (c >> 4) * XS + (c & 15) * 16) = xr[i];
    }
    const Tile nxt = make_tile(cur.id + gridDim.x);
    if (nxt.id < total) load_x(nxt);
    __syncthreads();

    // norms: thread (v, quarter p) sums dims [32p, 32p+32) in order; lanes
    // combine (Q0 + Q1) + (Q2 + Q3)
    {
      const int v = tid >> 2, p = tid & 3;
      const uint8_t* rp = xb + v * XS + 64 * p;
      double s = 0.0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const half8 h = as_h8(*reinterpret_cast<const u4*>(rp + 16 * i));
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const double xv = (double)(float)h[e];
          s = fma(xv, xv, s);
        }
      }
      s += __shfl_xor(s, 1);
      s += __shfl_xor(s, 2);
      if (p == 0) {
        const float n = (float)sqrt(s);
        if (v < cur.nv) a.dst.norms[(int64_t)cur.row * a.dst.norm_head_stride + cur.dst0 + v] = n;
        scl[v] = 1.f / (RSC * fmaxf(n, 1e-10f));
      }
    }

    // rotation: z^T tiles of 16 dims x 16 vectors
    f4 acc[4][2];
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      half8 bx[4];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
        bx[kb] = as_h8(*reinterpret_cast<const u4*>(xb + (16 * s4 + m) * XS + 64 * kb + 16 * g));
#pragma unroll
      for (int n2 = 0; n2 < 2; ++n2) {
        f4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[n2][kb], bx[kb], c, 0, 0, 0);
          c = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[n2][kb], bx[kb], c, 0, 0, 0);
        }
        acc[s4][n2] = c;
      }
    }
    __syncthreads();  // scales of every vector are in LDS

    // quantize: 4 codes (dims 32w + 16*n2 + 4g + e) per word, as bytes
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      const float sc = scl[16 * s4 + m];
#pragma unroll
      for (int n2 = 0; n2 < 2; ++n2) {
        uint32_t word = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float y = acc[s4][n2][e] * sc;
          uint32_t c;
          if constexpr (BH == BL) c = quant(y, bh);
          else c = whi ? quant(y, bh) : quant(y, bl);
          word |= c << (8 * e);
        }
        *reinterpret_cast<uint32_t*>(smem + L_CODES + (16 * s4 + m) * CS + 32 * w + 16 * n2 + 4 * g) = word;
      }
    }
    __syncthreads();

    // pack 32 codes (dims [32p, 32p+32) of vector v) and store them
    {
      const int v = tid >> 2, p = tid & 3;
      if (v < cur.nv) {
        const uint8_t* cp = smem + L_CODES + v * CS + 32 * p;
        const u4 c0 = *reinterpret_cast<const u4*>(cp);
        const u4 c1 = *reinterpret_cast<const u4*>(cp + 16);
        uint32_t code[32];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          code[i] = (c0[i >> 2] >> (8 * (i & 3))) & 0xFFu;
          code[16 + i] = (c1[i >> 2] >> (8 * (i & 3))) & 0xFFu;
        }
        if (32 * p < a.split) {
          uint8_t* dst = a.dst.codes_hi + (int64_t)cur.row * a.dst.hi_head_stride +
                         (int64_t)(cur.dst0 + v) * a.row_hi + 4 * BH * p;
          store_codes<BH>(dst, code);
        } else {
          uint8_t* dst = a.dst.codes_lo + (int64_t)cur.row * a.dst.lo_head_stride +
                         (int64_t)(cur.dst0 + v) * a.row_lo + 4 * BL * (p - a.split / 32);
          store_codes<BL>(dst, code);
        }
      }
    }
    if (nxt.id >= total) break;
    cur = nxt;
    xoff ^= (L_X0 ^ L_X1);
  }
}

template <int BH, int BL>
int launch_bh(const CompressArgs& a, hipStream_t s) {
  static int occ = 0;  // workgroups per CU (same for every gfx950 device)
  if (occ == 0 &&
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, compress_fast_kernel<BH, BL>, CTHR, 0) != hipSuccess)
    occ = 1;
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess &&
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    cus = 256;
  const int tpr = (a.span.n_tok + CT - 1) / CT;
  const int64_t total = (int64_t)tpr * a.span.rows;
  if (total <= 0 || total > (int64_t)0x7FFFFFFF) return 0;
  const int grid = (int)std::min<int64_t>(total, (int64_t)cus * std::max(occ, 1));
  hipLaunchKernelGGL((compress_fast_kernel<BH, BL>), dim3(grid), dim3(CTHR), 0, s, a, tpr, (int)total);
  return 1;
}

}  // namespace

int launch_compress_fast(const CompressArgs& a, hipStream_t s) {
  if (a.x_dtype != TQ_F16 || a.proj) return 0;
  if ((reinterpret_cast<uintptr_t>(a.x) & 15) || (a.x_hs & 7)) return 0;
  if (a.split != CD && a.split != CD / 2) return 0;
  const int bh = a.bits_hi, bl = a.bits_lo;
  if (bh == bl) {
    switch (bh) {
      case 1: return launch_bh<1, 1>(a, s);
      case 2: return launch_bh<2, 2>(a, s);
      case 3: return launch_bh<3, 3>(a, s);
      case 4: return launch_bh<4, 4>(a, s);
    }
  } else if (bh == bl + 1) {
    switch (bh) {
      case 2: return launch_bh<2, 1>(a, s);
      case 3: return launch_bh<3, 2>(a, s);
      case 4: return launch_bh<4, 3>(a, s);
    }
  }
  return 0;
}

}  // namespace tq
