// MFMA compress for TurboQuant on gfx950: fp16 vectors of head_dim 128 at 2-4
// bits (integer, or fractional with split d/2) ->
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
// Work split: a workgroup of 4 waves (three workgroups per CU) walks tiles of
// 64 vectors of one (batch, head) row, the next tile's x in flight. Wave w owns
// rotated dims [32w, 32w+32) and keeps its rows of 256R as MFMA A operands in
// registers for the whole launch. Per tile:
//   1. the x tile (16 KB) is stored to LDS;
//   2. each thread sums the squares of 32 dims of one vector in float64 and
//      lanes 4v..4v+3 combine them pairwise (the library's norm order);
//   3. each wave multiplies its A operands by the tile (B = x^T read from LDS).
//      A row r of output block n2 is rotated dim 32w + 8(r >> 2) + 4*n2 + (r & 3),
//      so lane (vector n = l & 15, g = l >> 4) ends up holding the 8
//      consecutive dims 32w + 8g .. 32w + 8g + 7 of vector n;
//   4. coordinates are scaled and quantized (count of boundaries below, ties
//      low, NaN -> 0; codebook.py:220-223) through a cell table (cell width
//      1/64 over |y| <= 1 plus a margin, so a cell index never needs a clamp;
//      with at most one boundary per cell, code = base + (y > boundary); a
//      codebook that puts two boundaries in one cell is counted instead);
//   5. the lane's 8 codes form 8*BITS consecutive bits of the LSB-first row
//      bitstream (packing.py); lanes assemble whole dwords and store them.

#include <math.h>

#include <type_traits>

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
constexpr float RSC = 256.f;   // scale of R before the fp16 split
// Quantizer cells c = round(64 y + 32), c in [CELL_LO, CELL_LO + NCELL): y is
// a coordinate of a unit vector (|y| <= 1 up to rounding, so c in [-32, 96]),
// or 0 for a vector whose norm is not finite
constexpr int CELL_LO = -40;
constexpr int NCELL = 144;
constexpr float MAGIC = 12582912.f;  // 1.5 * 2^23: fma(y, 64, 32 + MAGIC) holds round(64 y + 32) in its low bits
constexpr uint32_t MAGIC_BITS = 0x4B400000u;

constexpr uint32_t L_X0 = 0;
constexpr uint32_t L_X1 = CT * XS;
constexpr uint32_t L_SCALE = 2 * CT * XS;
constexpr uint32_t L_QT = L_SCALE + CT * 4;         // [2 codebooks][NCELL] {boundary, base}
constexpr uint32_t L_BND = L_QT + 2 * NCELL * 8;    // [2 codebooks][16] boundaries
constexpr uint32_t L_FLAG = L_BND + 2 * 16 * 4;
constexpr uint32_t L_TOTAL = L_FLAG + 16;

__device__ inline half8 as_h8(u4 v) { return __builtin_bit_cast(half8, v); }

// p[i] through the constant address space: the per-batch span arrays are
// read-only while the kernel runs, so uniform reads become scalar loads (and
// never wait on the vector-memory counter that tracks the prefetched tiles)
__device__ inline int ld_span(const int32_t* p, int i) {
  return ((const __attribute__((address_space(4))) int32_t*)(p))[i];
}

// n / d for uniform 0 <= n < 2^30 and d >= 1, with m = (2^32 - 1) / d from
// the host: umulhi(n, m) is floor(n / d) or one less, fixed by one remainder
// test; the operations stay on the scalar unit
__device__ inline int udiv_uniform(int n, int d, uint32_t m) {
  int q = (int)__umulhi((uint32_t)n, m);
  if (n - q * d >= d) ++q;
  return q;
}

struct Div {
  int d;       // divisor
  uint32_t m;  // (2^32 - 1) / d
};

struct Tile {
  int id;          // tile index; >= total: none left
  int row;         // (batch, head) row
  int nv;          // vectors in the tile
  int src0, dst0;  // first source / destination token of the tile
};

struct QCell {
  float bnd;      // the one boundary that can fall inside the cell, or +inf
  uint32_t base;  // boundaries below every value of the cell
};

// code of y (|y| <= 1 + 2^-20) from the cell table at LDS byte offset
// `tbl_adj` + 8 * (MAGIC_BITS + CELL_LO) (smem is the kernel's only LDS
// object, at offset 0; the magic bias and the first cell are folded into the
// base so the cell address is one shift-add)
__device__ inline uint32_t quant_table(float y, const uint8_t* smem, uint32_t tbl_adj) {
  const uint32_t r = __float_as_uint(fmaf(y, 64.f, 32.f + MAGIC));
  const QCell q = *reinterpret_cast<const QCell*>(smem + (tbl_adj + 8u * r));
  return q.base + (y > q.bnd ? 1u : 0u);
}

// a * b with 0 * anything = 0 (also for an infinite or NaN a): the legacy
// multiply, through its LLVM intrinsic (clang has no builtin for it)
extern "C" __device__ float tq_fmul_legacy(float, float) __asm("llvm.amdgcn.fmul.legacy");
__device__ inline float mul_zero_wins(float a, float b) { return tq_fmul_legacy(a, b); }

template <int BH, int BL>
__global__ __launch_bounds__(CTHR, 3) void compress_fast_kernel(CompressArgs a, Div tiles_per_row, Div heads,
                                                                int total) {
  __shared__ __align__(16) uint8_t smem[L_TOTAL];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int m = lane & 15, g = lane >> 4;
  const bool whi = 32 * w < a.split;  // this wave's dims use the high-width codebook
  constexpr int NBH = (1 << BH) - 1, NBL = (1 << BL) - 1;

  // quantizer tables of both codebooks; the flag records a cell holding two
  // boundaries (then every code is counted instead)
  uint32_t* flag = reinterpret_cast<uint32_t*>(smem + L_FLAG);
  if (tid == 0) *flag = 0u;
  __syncthreads();
  if (tid < 32) {  // boundaries for the counting fallback: [hi 16][lo 16]
    const int cb = tid >> 4, k = tid & 15;
    reinterpret_cast<float*>(smem + L_BND)[tid] = k < (cb ? NBL : NBH) ? (cb ? a.bnd_lo : a.bnd_hi)[k] : 0.f;
  }
  for (int i = tid; i < 2 * NCELL; i += CTHR) {
    const int cb = i / NCELL, ci = i % NCELL, c = CELL_LO + ci;
    const float* bp = cb ? a.bnd_lo : a.bnd_hi;
    const int nb = cb ? NBL : NBH;
    const float eps = 0x1p-20f;  // > the rounding of the cell index near a cell edge, in y units
    const float lo = ci == 0 ? -INFINITY : ((float)c - 32.5f) * (1.f / 64.f) - eps;
    const float hi = ci == NCELL - 1 ? INFINITY : ((float)c - 31.5f) * (1.f / 64.f) + eps;
    uint32_t base = 0, amb = 0;
    float bnd = INFINITY;
    for (int k = 0; k < nb; ++k) {
      const float b = bp[k];
      if (b < lo) ++base;
      else if (b <= hi) { ++amb; bnd = b; }
    }
    QCell* q = reinterpret_cast<QCell*>(smem + L_QT) + cb * NCELL + ci;
    q->bnd = bnd;
    q->base = base;
    if (amb > 1) atomicOr(flag, 1u);
  }

  // A operands: output row r of block n2 = rotated dim 32w + 8(r >> 2) + 4*n2 + (r & 3)
  // of 256R, k-slots 32*kb + 8*g + e
  half8 ah[2][4], al[2][4];
#pragma unroll
  for (int n2 = 0; n2 < 2; ++n2)
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const int j = 32 * w + 8 * (m >> 2) + 4 * n2 + (m & 3);
      const float* src = a.rot + j * CD + 32 * kb + 8 * g;
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
  __syncthreads();
  const bool table = *flag == 0u;
  const uint32_t qtab_adj = L_QT + (whi ? 0u : NCELL * 8u) - 8u * (MAGIC_BITS + (uint32_t)CELL_LO);  // wraps: see quant_table

  // next non-empty tile at or after `id` in this workgroup's sequence
  auto make_tile = [&](int id) {
    Tile t;
    t.id = id;
    t.row = t.nv = t.src0 = t.dst0 = 0;
    for (; t.id < total; t.id += gridDim.x) {
      t.row = udiv_uniform(t.id, tiles_per_row.d, tiles_per_row.m);
      const int t0 = (t.id - t.row * tiles_per_row.d) * CT;
      const int b = udiv_uniform(t.row, heads.d, heads.m);
      const int n = a.span.n_tok_b ? ld_span(a.span.n_tok_b, b) : a.span.n_tok;
      t.nv = min(CT, n - t0);
      if (t.nv > 0) {
        t.src0 = (a.span.src_tok0_b ? ld_span(a.span.src_tok0_b, b) : 0) + t0;
        t.dst0 = (a.span.dst_tok0_b ? ld_span(a.span.dst_tok0_b, b) : 0) + t0;
        break;
      }
    }
    return t;
  };

  // x tile: 1024 chunks of 16 bytes, chunk c = vector c >> 4, bytes 16*(c & 15);
  // vectors past the tile's end re-read its last vector (results not stored)
  auto load_x = [&](u4 (&xr)[4], const Tile& t) {
    const uint8_t* base = static_cast<const uint8_t*>(a.x) + ((int64_t)t.row * a.x_hs + (int64_t)t.src0 * CD) * 2;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + CTHR * i;
      const int v = min(c >> 4, t.nv - 1);
      xr[i] = *reinterpret_cast<const u4*>(base + v * 256 + (c & 15) * 16);
    }
  };

  const int split_w = a.split / 32;  // waves whose dims use the high-width codebook

  // x registers -> LDS tile at xoff
  auto write_x = [&](const u4 (&xr)[4], uint32_t xoff) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + CTHR * i;
      *reinterpret_cast<u4*>(smem + xoff + (c >> 4) * XS + (c & 15) * 16) = xr[i];
    }
  };

  // Norms of the tile at xoff: thread (v, quarter p) sums dims [32p, 32p+32)
  // in order; lanes combine (Q0 + Q1) + (Q2 + Q3). The four lanes of a vector
  // hold the same value and all store it (lanes past the tile's end store the
  // last vector's norm: their inputs are copies of it). The per-vector scale
  // 1 / (256 max(n, 1e-10)) goes to LDS at scl; 0 marks a non-finite norm.
  auto norms = [&](uint32_t xoff, const Tile& t, float* scl) {
    const int v = tid >> 2, p = tid & 3;
    const uint8_t* rp = smem + xoff + v * XS + 64 * p;
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
    const float n = (float)sqrt(s);
    a.dst.norms[(int64_t)t.row * a.dst.norm_head_stride + t.dst0 + min(v, t.nv - 1)] = n;
    scl[v] = __builtin_isfinite(n) ? 1.f / (RSC * fmaxf(n, 1e-10f)) : 0.f;
  };

  // rotation of the tile at xoff: z^T blocks of 16 dims x 16 vectors
  struct Acc {
    f4 v[4][2];
  };
  auto rotate = [&](uint32_t xoff) {
    Acc r;
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      half8 bx[4];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
        bx[kb] = as_h8(*reinterpret_cast<const u4*>(smem + xoff + (16 * s4 + m) * XS + 64 * kb + 16 * g));
#pragma unroll
      for (int n2 = 0; n2 < 2; ++n2) {
        f4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[n2][kb], bx[kb], c, 0, 0, 0);
          c = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[n2][kb], bx[kb], c, 0, 0, 0);
        }
        r.v[s4][n2] = c;
      }
    }
    return r;
  };

  // Quantize the lane's 8 consecutive dims of each sub-tile, pack, store.
  // The wave's 32 codes of vector v are B dwords at byte 4*B*wl of its row;
  // lane g holds bits [8Bg, 8Bg + 8B) of them. Lanes past the tile's end write
  // the last vector's row (their inputs are copies of it).
  const int B = whi ? BH : BL;  // wave-uniform
  uint8_t* const codes = whi ? a.dst.codes_hi : a.dst.codes_lo;
  const int64_t head_stride = whi ? a.dst.hi_head_stride : a.dst.lo_head_stride;
  const int row_bytes = whi ? a.row_hi : a.row_lo;
  const int wl = whi ? w : w - split_w;
  const float* bnd_l = reinterpret_cast<const float*>(smem + L_BND) + (whi ? 0 : 16);
  const int nbnd = (1 << B) - 1;
  auto quant_store = [&](auto table_tag, const Acc& acc, const Tile& t, const float* scl) {
    constexpr bool TABLE = decltype(table_tag)::value;
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      const int v = 16 * s4 + m;
      const float sc = scl[v];
      uint32_t V = 0;  // codes of dims 32w + 8g + k at bits B*k
#pragma unroll
      for (int n2 = 0; n2 < 2; ++n2)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float y = mul_zero_wins(acc.v[s4][n2][e], sc);  // 0 for a non-finite norm (sc = 0)
          uint32_t c;
          if constexpr (TABLE) {
            c = quant_table(y, smem, qtab_adj);
          } else {
            c = 0;
            for (int k = 0; k < nbnd; ++k) c += y > bnd_l[k] ? 1u : 0u;
          }
          V |= c << (B * (4 * n2 + e));
        }
      if (sc == 0.f) V = 0u;  // non-finite norm: every coordinate is NaN -> code 0
      uint32_t* rowp = reinterpret_cast<uint32_t*>(codes + (int64_t)t.row * head_stride +
                                                   (int64_t)(t.dst0 + min(v, t.nv - 1)) * row_bytes + 4 * B * wl);
      if constexpr (BH == BL && BH == 4) {
        rowp[g] = V;
      } else if constexpr (BH == BL && BH == 2) {
        // lanes g = 2k, 2k + 1 both store dword k
        const auto pr = __builtin_amdgcn_permlane16_swap(V, V, false, false);
        rowp[g >> 1] = pr[0] | (pr[1] << 16);
      } else {
        // dword k = min(g, B - 1) holds bits of lanes la = 4k / B and la + 1
        // (a lane past the last dword repeats it)
        const int k = min(g, B - 1);
        const int la = (4 * k) / B;
        const int off = 32 * k - 8 * B * la;
        const int sh2 = 8 * B - off;
        const uint32_t Va = __shfl(V, m + 16 * la);
        const uint32_t Vb = __shfl(V, m + 16 * min(la + 1, 3));
        rowp[k] = (Va >> off) | (sh2 < 32 ? Vb << sh2 : 0u);
      }
    }
  };

  // Tiles t, t + grid, ... of this workgroup. Per tile: the x tile already
  // in LDS gets its norms and rotation, the next tile's x (loaded during the
  // previous tile) goes to the other LDS buffer and the one after is loaded,
  // then the tile is quantized and stored. One accumulator set per wave keeps
  // the kernel at three workgroups per CU (12 waves); the MFMAs of one wave
  // overlap the quantization of the others. Every global load and store is
  // issued in the same order on every path through the loop, so the
  // compiler's memory-counter waits keep the prefetched tile in flight.
  auto run_tiles = [&](auto table_tag) {
    Tile cur = make_tile(blockIdx.x);
    if (cur.id >= total) return;
    Tile nxt = make_tile(cur.id + gridDim.x);
    u4 xr[4];
    {
      u4 x0[4];
      load_x(x0, cur);
      load_x(xr, nxt.id < total ? nxt : cur);
      write_x(x0, L_X0);
    }
    float* scl = reinterpret_cast<float*>(smem + L_SCALE);
    uint32_t xo = L_X0;
    for (;;) {
      __syncthreads();  // x of cur in LDS; every wave is done with the previous tile
      norms(xo, cur, scl);
      const Acc acc = rotate(xo);
      const bool more = nxt.id < total;
      const Tile far = more ? make_tile(nxt.id + gridDim.x) : nxt;
      if (more) {
        write_x(xr, xo ^ (L_X0 ^ L_X1));
        load_x(xr, far.id < total ? far : nxt);
      }
      __syncthreads();  // scales of cur
      quant_store(table_tag, acc, cur, scl);
      if (!more) break;
      cur = nxt;
      nxt = far;
      xo ^= (L_X0 ^ L_X1);
    }
  };
  if (table)
    run_tiles(std::true_type{});
  else
    run_tiles(std::false_type{});
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
  if (total <= 0 || total >= ((int64_t)1 << 30)) return 0;  // tile ids + 2 grids stay within int
  const int grid = (int)std::min<int64_t>(total, (int64_t)cus * std::max(occ, 1));
  const Div dt{tpr, 0xFFFFFFFFu / (uint32_t)tpr}, dh{a.span.heads, 0xFFFFFFFFu / (uint32_t)a.span.heads};
  hipLaunchKernelGGL((compress_fast_kernel<BH, BL>), dim3(grid), dim3(CTHR), 0, s, a, dt, dh, (int)total);
  return 1;
}

}  // namespace

int launch_compress_fast(const CompressArgs& a, hipStream_t s) {
  if (a.x_dtype != TQ_F16 || a.proj) return 0;
  if ((reinterpret_cast<uintptr_t>(a.x) & 15) || (a.x_hs & 7)) return 0;
  const int bh = a.bits_hi, bl = a.bits_lo;
  if (bh == bl && a.split == CD) {
    switch (bh) {
      case 2: return launch_bh<2, 2>(a, s);
      case 3: return launch_bh<3, 3>(a, s);
      case 4: return launch_bh<4, 4>(a, s);
    }
  } else if (bh == bl + 1 && a.split == CD / 2) {
    switch (bh) {
      case 3: return launch_bh<3, 2>(a, s);
      case 4: return launch_bh<4, 3>(a, s);
    }
  }
  return 0;  // 1-bit widths and other splits: the general kernel
}

}  // namespace tq
