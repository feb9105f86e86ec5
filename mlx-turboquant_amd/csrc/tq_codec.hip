// TurboQuant codec kernels for gfx950: compress (norm -> normalise -> rotate
// -> quantize -> pack [-> QJL sketch]), dequantize, bit packing utilities.
//
// Numeric contract (matches the CPU restatement used by the tests):
//   n   = f32(sqrt(S)), S the float64 sum of squares in 32-dim blocks (each
//         summed sequentially) combined pairwise (sumsq_blocks in tq_codec.h;
//         mlx_turboquant/cache.py:235-236 computes mx.linalg.norm of the f32 cast);
//   x_n = f32(x) / max(n, 1e-10f), IEEE float32 division (cache.py:237-238);
//   y_j = sum_i x_n[i] * R[j][i] accumulated in float32 (rotation.py:65);
//   idx = #{k : y > b_k} (codebook.py:220-223);
//   codes packed as an LSB-first bitstream per row (packing.py:9-173).

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include <type_traits>

#include "tq_common.h"
#include "tq_codec.h"

namespace tq {

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_codec(const tq_codec* c) {
  if (!c) return set_error(TQ_ERR_INVALID, "codec is NULL");
  if (c->d < 16 || c->d > 256 || (c->d % 16) != 0)
    return set_error(TQ_ERR_UNSUPPORTED, "head_dim %d not supported (a multiple of 16 in [16, 256])", c->d);
  if (c->bits_hi < 1 || c->bits_hi > 4 || c->bits_lo < 1 || c->bits_lo > 4)
    return set_error(TQ_ERR_UNSUPPORTED, "Unsupported bit-width: %d/%d. Use 1, 2, 3, or 4.",
                     c->bits_hi, c->bits_lo);
  if (c->split <= 0 || c->split > c->d || (c->split % 16) != 0)
    return set_error(TQ_ERR_UNSUPPORTED, "split %d must be a positive multiple of 16 <= d", c->split);
  if (!c->rotation || !c->centroids_hi || !c->boundaries_hi)
    return set_error(TQ_ERR_INVALID, "codec rotation / codebook pointer is NULL");
  if (c->split < c->d && (!c->centroids_lo || !c->boundaries_lo))
    return set_error(TQ_ERR_INVALID, "fractional codec needs the low-width codebook");
  if (c->qjl_proj && (c->qjl_m <= 0 || (c->qjl_m % 32) != 0 || c->qjl_m > 256))
    return set_error(TQ_ERR_UNSUPPORTED, "qjl_m %d must be a multiple of 32 in [32, 256]", c->qjl_m);
  return TQ_OK;
}

// ---------------------------------------------------------------------------
// Tiled float32 row-vector x matrix products for VPW vectors of dimension D.
// Thread (v, q) owns output columns [32q, 32q+32) of vector v. The matrix tile
// is staged in LDS with each 32-column segment padded to 36 floats so that the
// NSEG segments of a wave read distinct LDS banks.
// ---------------------------------------------------------------------------
// Thread (v, q) = (tid / NSEG, tid % NSEG); when NSEG does not divide 256
// (D = 96, 160, 192, 224) the last threads have no vector (v == VPW): they
// read vector VPW - 1 and write nothing. DP is the head_dim rounded up to a
// multiple of 32 (the tile width); a head_dim that is an odd multiple of 16
// leaves the upper half of the last segment: its columns of the vector tile
// and the matrix tiles hold zeros, and its codes are neither stored nor read.
template <int DP>
struct Geo {
  static_assert(DP % 32 == 0 && DP <= 256, "padded head_dim");
  static constexpr int NSEG = DP / 32;         // 32-column segments
  static constexpr int VPW = 256 / NSEG;       // vectors per workgroup
  static constexpr int XS = DP + 1;            // padded row of the vector tile
  static constexpr int SEGP = 36;              // padded segment
  static constexpr int MROW = NSEG * SEGP;     // padded matrix row
  static constexpr int TI = 32;                // matrix rows per LDS tile
};

__device__ inline void store_codes_dyn(int bits, uint8_t* dst, const uint32_t (&code)[32]) {
  switch (bits) {
    case 1: store_codes<1>(dst, code); break;
    case 2: store_codes<2>(dst, code); break;
    case 3: store_codes<3>(dst, code); break;
    default: store_codes<4>(dst, code); break;
  }
}

template <int BITS>
__device__ inline void load_codes(const uint8_t* src, uint32_t (&code)[32]) {
  uint32_t w[BITS];
  const uint32_t* s32 = reinterpret_cast<const uint32_t*>(src);
#pragma unroll
  for (int i = 0; i < BITS; ++i) w[i] = s32[i];
  unpack32<BITS>(w, code);
}

__device__ inline void load_codes_dyn(int bits, const uint8_t* src, uint32_t (&code)[32]) {
  switch (bits) {
    case 1: load_codes<1>(src, code); break;
    case 2: load_codes<2>(src, code); break;
    case 3: load_codes<3>(src, code); break;
    default: load_codes<4>(src, code); break;
  }
}

// Codes c0 .. c0 + 15 of a segment as 2 BITS bytes of the LSB-first
// bitstream, written / read byte by byte (rows whose byte offsets are not
// dword multiples: head_dim 96 split in halves of 48 codes).
__device__ inline void store_half(int bits, uint8_t* dst, const uint32_t (&code)[32], int c0) {
  uint64_t w = 0;
#pragma unroll
  for (int k = 0; k < 16; ++k) w |= (uint64_t)code[c0 + k] << (bits * k);
  for (int i = 0; i < 2 * bits; ++i) dst[i] = (uint8_t)(w >> (8 * i));
}

__device__ inline void load_half(int bits, const uint8_t* src, uint32_t (&code)[32], int c0) {
  uint64_t w = 0;
  for (int i = 0; i < 2 * bits; ++i) w |= (uint64_t)src[i] << (8 * i);
  const uint32_t mask = (1u << bits) - 1u;
#pragma unroll
  for (int k = 0; k < 16; ++k) code[c0 + k] = (uint32_t)(w >> (bits * k)) & mask;
}

// count of boundaries strictly below y (ties go low, NaN -> 0)
__device__ inline uint32_t quantize_one(float y, const float* b, int nb) {
  uint32_t idx = 0;
  for (int k = 0; k < nb; ++k) idx += (y > b[k]) ? 1u : 0u;
  return idx;
}

// acc[c] += sum_{i in tile} xs[v][i] * M[i][32q + c] for the LDS tile M.
template <int DP>
__device__ inline void tile_madd(const float* __restrict__ xs_row, const float* __restrict__ mt,
                                 int i0, int q, float (&acc)[32]) {
  using G = Geo<DP>;
#pragma unroll 4
  for (int ii = 0; ii < G::TI; ++ii) {
    const float xv = xs_row[i0 + ii];
    const float4* m4 = reinterpret_cast<const float4*>(mt + ii * G::MROW + q * G::SEGP);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float4 r = m4[k];
      acc[4 * k + 0] = fmaf(xv, r.x, acc[4 * k + 0]);
      acc[4 * k + 1] = fmaf(xv, r.y, acc[4 * k + 1]);
      acc[4 * k + 2] = fmaf(xv, r.z, acc[4 * k + 2]);
      acc[4 * k + 3] = fmaf(xv, r.w, acc[4 * k + 3]);
    }
  }
}

// Stage rows [i0, i0+TI) of M (row-major d x d, or its transpose when
// TRANSPOSE) into the padded LDS tile mt[ii][seg][SEGP]; rows and columns at
// or past d are zeros.
template <int DP, bool TRANSPOSE>
__device__ inline void stage_tile(const float* __restrict__ m, int d, int i0, float* mt) {
  using G = Geo<DP>;
  for (int e = threadIdx.x; e < G::TI * DP; e += blockDim.x) {
    const int ii = e / DP, j = e % DP;
    const bool ok = i0 + ii < d && j < d;
    const float val = !ok ? 0.f : TRANSPOSE ? m[(int64_t)j * d + (i0 + ii)] : m[(int64_t)(i0 + ii) * d + j];
    mt[ii * G::MROW + (j >> 5) * G::SEGP + (j & 31)] = val;
  }
}

// The codes of the thread's segment q (columns [32 q, 32 q + 32) of a
// d-dim row, the first `split` at bits_hi into rows of row_hi bytes, the rest
// at bits_lo into rows of row_lo bytes): one dword store / load per BITS
// dwords when the segment is whole, of one width, and dword-aligned in its
// row; else 16-code halves byte by byte (columns at or past d skipped).
__device__ inline bool whole_segment(int q, int d, int split, int row_hi, int row_lo) {
  const bool hi = 32 * q < split;
  return (split & 31) == 0 && 32 * q + 32 <= d && ((hi ? row_hi : row_lo) & 3) == 0;
}

// f(std::integral_constant<int, DP>) with DP = d rounded up to a multiple of
// 32 (d a multiple of 16 in [16, 256], checked by check_codec)
template <typename F>
static void launch_padded(int d, F f) {
  switch ((d + 31) / 32) {
    case 1: f(std::integral_constant<int, 32>{}); break;
    case 2: f(std::integral_constant<int, 64>{}); break;
    case 3: f(std::integral_constant<int, 96>{}); break;
    case 4: f(std::integral_constant<int, 128>{}); break;
    case 5: f(std::integral_constant<int, 160>{}); break;
    case 6: f(std::integral_constant<int, 192>{}); break;
    case 7: f(std::integral_constant<int, 224>{}); break;
    default: f(std::integral_constant<int, 256>{}); break;
  }
}

template <int DP>
__global__ __launch_bounds__(256) void compress_kernel(CompressArgs a) {
  using G = Geo<DP>;
  __shared__ float xs[G::VPW * G::XS];
  __shared__ float mt[G::TI * G::MROW];
  __shared__ float nrm[G::VPW];
  __shared__ float bnd[2][16];
  __shared__ float cen[2][16];

  const int D = a.d;
  const int r = blockIdx.y;
  const int b = r / a.span.heads;
  const int n_tok = a.span.n_tok_b ? a.span.n_tok_b[b] : a.span.n_tok;
  const int t0 = blockIdx.x * G::VPW;
  if (t0 >= n_tok) return;
  const int nv = min(G::VPW, n_tok - t0);
  const int src0 = (a.span.src_tok0_b ? a.span.src_tok0_b[b] : 0) + t0;
  const int dst0 = (a.span.dst_tok0_b ? a.span.dst_tok0_b[b] : 0) + t0;
  const int tid = threadIdx.x;

  if (tid < 16) {
    const int nbh = (1 << a.bits_hi) - 1, nbl = (1 << a.bits_lo) - 1;
    bnd[0][tid] = tid < nbh ? a.bnd_hi[tid] : 0.f;
    bnd[1][tid] = tid < nbl ? a.bnd_lo[tid] : 0.f;
    cen[0][tid] = tid <= nbh ? a.cen_hi[tid] : 0.f;
    cen[1][tid] = tid <= nbl ? a.cen_lo[tid] : 0.f;
  }

  // Load the tile as float32 (exact); columns past D are zeros.
  const int64_t xrow = (int64_t)r * a.x_hs + (int64_t)src0 * D;
  for (int e = tid; e < G::VPW * DP; e += blockDim.x) {
    const int v = e / DP, i = e % DP;
    xs[v * G::XS + i] = v < nv && i < D ? load_elem(a.x, xrow + (int64_t)v * D + i, a.x_dtype) : 0.f;
  }
  __syncthreads();

  // Norm: float64 sum of squares in the library's block order, rounded square
  // root (the zero columns past D add nothing to the last block).
  if (tid < G::VPW) {
    const float n = (float)sqrt(sumsq_blocks<DP>(xs + tid * G::XS));
    nrm[tid] = n;
    if (tid < nv) a.dst.norms[(int64_t)r * a.dst.norm_head_stride + dst0 + tid] = n;
  }
  __syncthreads();

  // Normalise in place.
  for (int e = tid; e < G::VPW * DP; e += blockDim.x) {
    const int v = e / DP, i = e % DP;
    xs[v * G::XS + i] = xs[v * G::XS + i] / fmaxf(nrm[v], 1e-10f);
  }

  // Rotate: y = x_n @ R^T.
  const int v = tid / G::NSEG, q = tid % G::NSEG;
  const bool vok = v < G::VPW;            // false only for the spare threads when NSEG does not divide 256
  const int vr = vok ? v : G::VPW - 1;    // the vector row it reads
  float acc[32];
#pragma unroll
  for (int c = 0; c < 32; ++c) acc[c] = 0.f;
  for (int i0 = 0; i0 < D; i0 += G::TI) {
    __syncthreads();
    stage_tile<DP, true>(a.rot, D, i0, mt);
    __syncthreads();
    tile_madd<DP>(xs + vr * G::XS, mt, i0, q, acc);
  }

  // Quantize + pack this thread's 32 coordinates (columns 32q + c; column j
  // uses the high-width codebook when j < split).
  uint32_t code[32];
#pragma unroll
  for (int c = 0; c < 32; ++c) {
    const bool hc = 32 * q + c < a.split;
    code[c] = quantize_one(acc[c], bnd[hc ? 0 : 1], (1 << (hc ? a.bits_hi : a.bits_lo)) - 1);
  }
  if (v < nv && 32 * q < D) {
    if (whole_segment(q, D, a.split, a.row_hi, a.row_lo)) {
      const bool hi = 32 * q < a.split;
      const int bits = hi ? a.bits_hi : a.bits_lo;
      uint8_t* dst;
      if (hi) {
        dst = a.dst.codes_hi + (int64_t)r * a.dst.hi_head_stride + (int64_t)(dst0 + v) * a.row_hi +
              (32 * q) * bits / 8;
      } else {
        dst = a.dst.codes_lo + (int64_t)r * a.dst.lo_head_stride + (int64_t)(dst0 + v) * a.row_lo +
              (32 * q - a.split) * bits / 8;
      }
      store_codes_dyn(bits, dst, code);
    } else {
      for (int hh = 0; hh < 2; ++hh) {
        const int j = 32 * q + 16 * hh;
        if (j >= D) break;
        const bool hi = j < a.split;
        const int bits = hi ? a.bits_hi : a.bits_lo;
        uint8_t* dst = hi ? a.dst.codes_hi + (int64_t)r * a.dst.hi_head_stride + (int64_t)(dst0 + v) * a.row_hi +
                                j * bits / 8
                          : a.dst.codes_lo + (int64_t)r * a.dst.lo_head_stride + (int64_t)(dst0 + v) * a.row_lo +
                                (j - a.split) * bits / 8;
        store_half(bits, dst, code, 16 * hh);
      }
    }
  }

  if (!a.proj) return;

  // QJL sketch of the residual r = x - n * (c[idx] @ R) (cache.py:396-427).
  // Reconstruct in rotated space first: xs[v][j] <- c[idx_j] (overwrites x_n;
  // zeros past D).
  __syncthreads();
  if (vok) {
#pragma unroll
    for (int c = 0; c < 32; ++c)
      xs[v * G::XS + 32 * q + c] = 32 * q + c < D ? cen[32 * q + c < a.split ? 0 : 1][code[c]] : 0.f;
  }
#pragma unroll
  for (int c = 0; c < 32; ++c) acc[c] = 0.f;
  for (int i0 = 0; i0 < D; i0 += G::TI) {
    __syncthreads();
    stage_tile<DP, false>(a.rot, D, i0, mt);
    __syncthreads();
    tile_madd<DP>(xs + vr * G::XS, mt, i0, q, acc);
  }
  __syncthreads();
  // residual in xs (float32: x - n * acc; zeros past D)
  if (vok) {
    const float n = nrm[v];
#pragma unroll
    for (int c = 0; c < 32; ++c) {
      const int i = 32 * q + c;
      const float x = v < nv && i < D ? load_elem(a.x, xrow + (int64_t)v * D + i, a.x_dtype) : 0.f;
      xs[v * G::XS + i] = i < D ? x - n * acc[c] : 0.f;
    }
  }
  __syncthreads();
  if (tid < G::VPW) {
    double s = 0.0;
    const float* row = xs + tid * G::XS;
    for (int i = 0; i < D; ++i) {
      const double ri = (double)row[i];
      s = fma(ri, ri, s);
    }
    if (tid < nv) a.dst.gamma[(int64_t)r * a.dst.gamma_head_stride + dst0 + tid] = (float)sqrt(s);
  }
  // proj = r @ S^T, m outputs in segments of 32 (S rows are projections).
  const int nseg_m = a.qjl_m / 32;
  for (int s0 = 0; s0 < nseg_m; s0 += G::NSEG) {
    // Stage S^T columns [32*s0, 32*s0 + DP) in tiles: reuse mt with rows i of S^T.
    const int qs = s0 + q;
#pragma unroll
    for (int c = 0; c < 32; ++c) acc[c] = 0.f;
    for (int i0 = 0; i0 < D; i0 += G::TI) {
      __syncthreads();
      for (int e = tid; e < G::TI * DP; e += blockDim.x) {
        const int ii = e / DP, j = e % DP;  // j indexes projection 32*s0 + j
        const int mrow = 32 * s0 + j;
        mt[ii * G::MROW + (j >> 5) * G::SEGP + (j & 31)] =
            mrow < a.qjl_m && i0 + ii < D ? a.proj[(int64_t)mrow * D + i0 + ii] : 0.f;
      }
      __syncthreads();
      tile_madd<DP>(xs + vr * G::XS, mt, i0, q, acc);
    }
    if (v < nv && qs < nseg_m) {
      uint32_t word = 0;
#pragma unroll
      for (int c = 0; c < 32; ++c) word |= (acc[c] >= 0.f ? 1u : 0u) << c;
      uint32_t* sd = reinterpret_cast<uint32_t*>(a.dst.signs + (int64_t)r * a.dst.sign_head_stride +
                                                 (int64_t)(dst0 + v) * a.row_sign);
      sd[qs] = word;
    }
  }
}

// One vector per wave for small spans (d = 128, with or without a sketch of
// m <= 128): the one-token ragged drains of a decode step, where the tiled
// kernel above (64 vectors per workgroup) spends its time in a long chain of
// dependent phases. The same float32 / float64 operations in the same order
// as compress_kernel, so the outputs are bit-identical: every product is one
// output per lane (lane and lane + 64) summed over i = 0..127 in order with
// fmaf, with R and S staged in LDS (rows padded to 129 floats).
constexpr int DRW = 8;    // waves (vectors) per workgroup
constexpr int DRP = 132;  // padded LDS row: 16-byte aligned, rows of 16 lanes in distinct banks

// LDS of a drain workgroup: R and S (rows padded to DRP floats), the waves'
// vectors and codes, the codebooks
struct DrainLds {
  float rt[128 * DRP];  // R[c][i] at c * DRP + i
  float st[128 * DRP];  // S[k][i] at k * DRP + i
  float vec[DRW][128];
  uint8_t cds[DRW][128];
  float bnd[2][16];
  float cen[2][16];
};

// The drain of vector `vid` (row vid / n_tok, token vid % n_tok) by wave w,
// in two parts: drain_begin, before the workgroup's barrier (the vector's
// indices and loads, whose latency then runs under the staging of R and S),
// and drain_vector after it (R, S and the codebooks of `a` in LDS); seq(b)
// gives sequence b's {token count, first source token, first destination
// token}.
struct DrainIn {
  int r, dst;
  float x0, x1;
  bool ok;  // the wave has a vector
};
template <class Seq>
__device__ __forceinline__ DrainIn drain_begin(const CompressArgs& a, DrainLds& L, int vid, int w, int lane, Seq seq);
__device__ __forceinline__ void drain_vector(const CompressArgs& a, DrainLds& L, int w, int lane, const DrainIn& in);

// R, S and the codebooks of `a` into the workgroup's LDS (before a barrier)
__device__ __forceinline__ void drain_stage(const CompressArgs& a, DrainLds& L, int tid) {
  float* rt = L.rt;
  float* st = L.st;
  // R and S in 16-byte pieces, every load of a thread requested before its
  // first store (8 pieces of R per thread, up to 16 of S)
  {
    const float4* r4 = reinterpret_cast<const float4*>(a.rot);
    float4 x[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) x[k] = r4[tid + k * DRW * 64];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int e = tid + k * DRW * 64, row = e >> 5, c = 4 * (e & 31);
      *reinterpret_cast<float4*>(rt + row * DRP + c) = x[k];
    }
    if (a.qjl_m > 0) {
      const float4* s4 = reinterpret_cast<const float4*>(a.proj);
      const int n4 = a.qjl_m * 32;  // pieces of S (qjl_m <= 128 here)
      float4 y[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int e = tid + k * DRW * 64;
        y[k] = e < n4 ? s4[e] : float4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int e = tid + k * DRW * 64, row = e >> 5, c = 4 * (e & 31);
        if (e < n4) *reinterpret_cast<float4*>(st + row * DRP + c) = y[k];
      }
    }
  }
  if (tid < 16) {
    const int nbh = (1 << a.bits_hi) - 1, nbl = (1 << a.bits_lo) - 1;
    L.bnd[0][tid] = tid < nbh ? a.bnd_hi[tid] : 0.f;
    L.bnd[1][tid] = tid < nbl ? a.bnd_lo[tid] : 0.f;
    L.cen[0][tid] = tid <= nbh ? a.cen_hi[tid] : 0.f;
    L.cen[1][tid] = tid <= nbl ? a.cen_lo[tid] : 0.f;
  }
}

struct SeqRange {
  int n_tok, src0, dst0;
};

__global__ __launch_bounds__(DRW * 64) void drain_kernel(CompressArgs a) {
  __shared__ __align__(16) DrainLds L;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const DrainIn in = drain_begin(a, L, blockIdx.x * DRW + w, w, lane, [&](int b) {
    return SeqRange{a.span.n_tok_b ? a.span.n_tok_b[b] : a.span.n_tok, a.span.src_tok0_b ? a.span.src_tok0_b[b] : 0,
                    a.span.dst_tok0_b ? a.span.dst_tok0_b[b] : 0};
  });
  drain_stage(a, L, tid);
  __syncthreads();  // the only barrier: waves without a vector leave after it
  if (in.ok) drain_vector(a, L, w, lane, in);
}

template <class Seq>
__device__ __forceinline__ DrainIn drain_begin(const CompressArgs& a, DrainLds& L, int vid, int w, int lane, Seq seq) {
  DrainIn in{0, 0, 0.f, 0.f, false};
  const int r = vid / a.span.n_tok, t = vid % a.span.n_tok;
  if (r >= a.span.rows) return in;
  const int b = r / a.span.heads;
  const SeqRange sr = seq(b);
  if (t >= sr.n_tok) return in;
  const int src = sr.src0 + t;
  in.r = r;
  in.dst = sr.dst0 + t;
  in.ok = true;
  const int64_t xrow = (int64_t)r * a.x_hs + (int64_t)src * 128;
  in.x0 = load_elem(a.x, xrow + lane, a.x_dtype);
  in.x1 = load_elem(a.x, xrow + 64 + lane, a.x_dtype);
  return in;
}

__device__ __forceinline__ void drain_vector(const CompressArgs& a, DrainLds& L, int w, int lane, const DrainIn& in) {
  const float* rt = L.rt;
  const float* st = L.st;
  auto& vec = L.vec;
  auto& cds = L.cds;
  auto& bnd = L.bnd;
  auto& cen = L.cen;
  const int r = in.r, dst = in.dst;
  const float x0 = in.x0, x1 = in.x1;
  float* xv = vec[w];
  xv[lane] = x0;
  xv[64 + lane] = x1;
  // norm: float64 block sums (every lane, the same value)
  const float n = (float)sqrt(sumsq_blocks<128>(xv));
  if (lane == 0) a.dst.norms[(int64_t)r * a.dst.norm_head_stride + dst] = n;
  xv[lane] = x0 / fmaxf(n, 1e-10f);
  xv[64 + lane] = x1 / fmaxf(n, 1e-10f);
  // rotate: y_c = sum_i x_n[i] * R[c][i] (i in order; four i per LDS read)
  float y0 = 0.f, y1 = 0.f;
#pragma unroll 4
  for (int i = 0; i < 128; i += 4) {
    const float4 xi = *reinterpret_cast<const float4*>(xv + i);
    const float4 ra = *reinterpret_cast<const float4*>(rt + lane * DRP + i);
    const float4 rb = *reinterpret_cast<const float4*>(rt + (lane + 64) * DRP + i);
    y0 = fmaf(xi.w, ra.w, fmaf(xi.z, ra.z, fmaf(xi.y, ra.y, fmaf(xi.x, ra.x, y0))));
    y1 = fmaf(xi.w, rb.w, fmaf(xi.z, rb.z, fmaf(xi.y, rb.y, fmaf(xi.x, rb.x, y1))));
  }
  const bool hi0 = lane < a.split, hi1 = lane + 64 < a.split;
  const uint32_t c0 = quantize_one(y0, bnd[hi0 ? 0 : 1], (1 << (hi0 ? a.bits_hi : a.bits_lo)) - 1);
  const uint32_t c1 = quantize_one(y1, bnd[hi1 ? 0 : 1], (1 << (hi1 ? a.bits_hi : a.bits_lo)) - 1);
  cds[w][lane] = (uint8_t)c0;
  cds[w][64 + lane] = (uint8_t)c1;
  if (lane < 4) {  // lane q packs the 32 codes of segment q
    const int q = lane;
    const bool hi = 32 * q < a.split;
    const int bits = hi ? a.bits_hi : a.bits_lo;
    uint32_t code[32];
#pragma unroll
    for (int c = 0; c < 32; ++c) code[c] = cds[w][32 * q + c];
    uint8_t* d = hi ? a.dst.codes_hi + (int64_t)r * a.dst.hi_head_stride + (int64_t)dst * a.row_hi + (32 * q) * bits / 8
                    : a.dst.codes_lo + (int64_t)r * a.dst.lo_head_stride + (int64_t)dst * a.row_lo +
                          (32 * q - a.split) * bits / 8;
    store_codes_dyn(bits, d, code);
  }
  if (!a.proj) return;
  // QJL sketch of the residual r = x - n * (c[idx] @ R)
  xv[lane] = cen[hi0 ? 0 : 1][c0];
  xv[64 + lane] = cen[hi1 ? 0 : 1][c1];
  float a0 = 0.f, a1 = 0.f;
#pragma unroll 4
  for (int i = 0; i < 128; i += 4) {
    const float4 ci = *reinterpret_cast<const float4*>(xv + i);
    a0 = fmaf(ci.x, rt[i * DRP + lane], a0);
    a1 = fmaf(ci.x, rt[i * DRP + lane + 64], a1);
    a0 = fmaf(ci.y, rt[(i + 1) * DRP + lane], a0);
    a1 = fmaf(ci.y, rt[(i + 1) * DRP + lane + 64], a1);
    a0 = fmaf(ci.z, rt[(i + 2) * DRP + lane], a0);
    a1 = fmaf(ci.z, rt[(i + 2) * DRP + lane + 64], a1);
    a0 = fmaf(ci.w, rt[(i + 3) * DRP + lane], a0);
    a1 = fmaf(ci.w, rt[(i + 3) * DRP + lane + 64], a1);
  }
  const float r0 = x0 - n * a0;
  const float r1 = x1 - n * a1;
  xv[lane] = r0;
  xv[64 + lane] = r1;
  double s2 = 0.0;
#pragma unroll 4
  for (int i = 0; i < 128; i += 4) {
    const float4 r4 = *reinterpret_cast<const float4*>(xv + i);
    s2 = fma((double)r4.x, (double)r4.x, s2);
    s2 = fma((double)r4.y, (double)r4.y, s2);
    s2 = fma((double)r4.z, (double)r4.z, s2);
    s2 = fma((double)r4.w, (double)r4.w, s2);
  }
  if (lane == 0) a.dst.gamma[(int64_t)r * a.dst.gamma_head_stride + dst] = (float)sqrt(s2);
  float p0 = 0.f, p1 = 0.f;
  const int k1 = min(lane + 64, a.qjl_m - 1);
#pragma unroll 4
  for (int i = 0; i < 128; i += 4) {
    const float4 ri = *reinterpret_cast<const float4*>(xv + i);
    const float4 sa = *reinterpret_cast<const float4*>(st + lane * DRP + i);
    const float4 sb = *reinterpret_cast<const float4*>(st + k1 * DRP + i);
    p0 = fmaf(ri.w, sa.w, fmaf(ri.z, sa.z, fmaf(ri.y, sa.y, fmaf(ri.x, sa.x, p0))));
    p1 = fmaf(ri.w, sb.w, fmaf(ri.z, sb.z, fmaf(ri.y, sb.y, fmaf(ri.x, sb.x, p1))));
  }
  const uint64_t s_lo = __ballot(p0 >= 0.f), s_hi = __ballot(p1 >= 0.f);
  if (lane == 0) {
    uint32_t* sd = reinterpret_cast<uint32_t*>(a.dst.signs + (int64_t)r * a.dst.sign_head_stride + (int64_t)dst * a.row_sign);
    const int nw = a.qjl_m / 32;
    sd[0] = (uint32_t)s_lo;
    if (nw > 1) sd[1] = (uint32_t)(s_lo >> 32);
    if (nw > 2) sd[2] = (uint32_t)s_hi;
    if (nw > 3) sd[3] = (uint32_t)(s_hi >> 32);
  }
}

struct DequantArgs {
  tq_store src;
  tq_span span;
  float* out;
  int64_t out_hs;
  const float* rot;
  const float* cen_hi;
  const float* cen_lo;
  const float* proj;
  int d;  // head_dim
  int bits_hi, bits_lo, split, qjl_m, apply_qjl;
  int row_hi, row_lo, row_sign;
};

template <int DP>
__global__ __launch_bounds__(256) void dequant_kernel(DequantArgs a) {
  using G = Geo<DP>;
  __shared__ float ys[G::VPW * G::XS];
  __shared__ float mt[G::TI * G::MROW];
  __shared__ float cen[2][16];
  const int D = a.d;
  const int r = blockIdx.y;
  const int b = r / a.span.heads;
  const int n_tok = a.span.n_tok_b ? a.span.n_tok_b[b] : a.span.n_tok;
  const int t0 = blockIdx.x * G::VPW;
  if (t0 >= n_tok) return;
  const int nv = min(G::VPW, n_tok - t0);
  const int src0 = (a.span.src_tok0_b ? a.span.src_tok0_b[b] : 0) + t0;
  const int dst0 = (a.span.dst_tok0_b ? a.span.dst_tok0_b[b] : 0) + t0;
  const int tid = threadIdx.x;
  if (tid < 16) {
    cen[0][tid] = tid < (1 << a.bits_hi) ? a.cen_hi[tid] : 0.f;
    cen[1][tid] = tid < (1 << a.bits_lo) ? a.cen_lo[tid] : 0.f;
  }
  __syncthreads();
  const int v = tid / G::NSEG, q = tid % G::NSEG;
  const bool vok = v < G::VPW;            // false only for the spare threads when NSEG does not divide 256
  const int vr = vok ? v : G::VPW - 1;
  uint32_t code[32];
#pragma unroll
  for (int c = 0; c < 32; ++c) code[c] = 0;
  if (v < nv && 32 * q < D) {
    if (whole_segment(q, D, a.split, a.row_hi, a.row_lo)) {
      const bool hi = 32 * q < a.split;
      const int bits = hi ? a.bits_hi : a.bits_lo;
      const uint8_t* src = hi ? a.src.codes_hi + (int64_t)r * a.src.hi_head_stride +
                                    (int64_t)(src0 + v) * a.row_hi + (32 * q) * bits / 8
                              : a.src.codes_lo + (int64_t)r * a.src.lo_head_stride +
                                    (int64_t)(src0 + v) * a.row_lo + (32 * q - a.split) * bits / 8;
      load_codes_dyn(bits, src, code);
    } else {  // halves of 16 codes, byte loads
      for (int hh = 0; hh < 2; ++hh) {
        const int j = 32 * q + 16 * hh;
        if (j >= D) break;
        const bool hi = j < a.split;
        const int bits = hi ? a.bits_hi : a.bits_lo;
        const uint8_t* src = hi ? a.src.codes_hi + (int64_t)r * a.src.hi_head_stride +
                                      (int64_t)(src0 + v) * a.row_hi + j * bits / 8
                                : a.src.codes_lo + (int64_t)r * a.src.lo_head_stride +
                                      (int64_t)(src0 + v) * a.row_lo + (j - a.split) * bits / 8;
        load_half(bits, src, code, 16 * hh);
      }
    }
  }
  if (vok) {
#pragma unroll
    for (int c = 0; c < 32; ++c)
      ys[v * G::XS + 32 * q + c] = 32 * q + c < D ? cen[32 * q + c < a.split ? 0 : 1][code[c]] : 0.f;
  }
  float acc[32];
#pragma unroll
  for (int c = 0; c < 32; ++c) acc[c] = 0.f;
  for (int i0 = 0; i0 < D; i0 += G::TI) {
    __syncthreads();
    stage_tile<DP, false>(a.rot, D, i0, mt);
    __syncthreads();
    tile_madd<DP>(ys + vr * G::XS, mt, i0, q, acc);
  }
  const float n = v < nv ? a.src.norms[(int64_t)r * a.src.norm_head_stride + src0 + v] : 0.f;
#pragma unroll
  for (int c = 0; c < 32; ++c) acc[c] *= n;

  if (a.apply_qjl) {
    // + sqrt(pi/2)/D * gamma * (z @ S), z = +-1 from the stored signs, in
    // passes of DP projections (the segments of the tile).
    __syncthreads();
    const int nseg_m = a.qjl_m / 32;
    float corr[32];
#pragma unroll
    for (int c = 0; c < 32; ++c) corr[c] = 0.f;
    for (int m0 = 0; m0 < a.qjl_m; m0 += DP) {
      __syncthreads();
      if (v < nv) {
        const uint32_t* sg = reinterpret_cast<const uint32_t*>(
            a.src.signs + (int64_t)r * a.src.sign_head_stride + (int64_t)(src0 + v) * a.row_sign);
        const int seg = m0 / 32 + q;
        const uint32_t w = seg < nseg_m ? sg[seg] : 0u;
#pragma unroll
        for (int c = 0; c < 32; ++c)
          ys[v * G::XS + 32 * q + c] = seg < nseg_m ? (((w >> c) & 1u) ? 1.f : -1.f) : 0.f;
      } else if (vok) {
#pragma unroll
        for (int c = 0; c < 32; ++c) ys[v * G::XS + 32 * q + c] = 0.f;
      }
      // rows m0 + i of S (i < DP), columns < D
      const int mi = min(DP, a.qjl_m - m0);
      for (int i0 = 0; i0 < mi; i0 += G::TI) {
        __syncthreads();
        for (int e = tid; e < G::TI * DP; e += blockDim.x) {
          const int ii = e / DP, j = e % DP;
          mt[ii * G::MROW + (j >> 5) * G::SEGP + (j & 31)] =
              i0 + ii < mi && j < D ? a.proj[(int64_t)(m0 + i0 + ii) * D + j] : 0.f;
        }
        __syncthreads();
        tile_madd<DP>(ys + vr * G::XS, mt, i0, q, corr);
      }
    }
    if (v < nv) {
      const float g = a.src.gamma[(int64_t)r * a.src.gamma_head_stride + src0 + v];
      const float sc = 1.2533141373155003f / (float)D * g;  // sqrt(pi/2)/D * gamma
#pragma unroll
      for (int c = 0; c < 32; ++c) acc[c] = fmaf(sc, corr[c], acc[c]);
    }
  }
  if (v < nv && 32 * q < D) {
    float4* o = reinterpret_cast<float4*>(a.out + (int64_t)r * a.out_hs + (int64_t)(dst0 + v) * D + 32 * q);
    const int nk = min(8, (D - 32 * q) / 4);
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (k < nk) o[k] = make_float4(acc[4 * k], acc[4 * k + 1], acc[4 * k + 2], acc[4 * k + 3]);
  }
}

__global__ void pack_kernel(const uint8_t* __restrict__ idx, int64_t n_rows, int d, int bits,
                            uint8_t* __restrict__ out) {
  const int rb = d * bits / 8;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n_rows * rb) return;
  const int64_t row = e / rb;
  const int k = (int)(e % rb);
  const uint8_t* in = idx + row * d;
  uint32_t byte = 0;
  const int jlo = (8 * k) / bits, jhi = (8 * k + 7) / bits;
  for (int j = jlo; j <= jhi && j < d; ++j) {
    const int p = bits * j - 8 * k;  // bit offset of code j relative to this byte
    const uint32_t c = in[j] & ((1u << bits) - 1u);
    byte |= p >= 0 ? (c << p) : (c >> (-p));
  }
  out[e] = (uint8_t)(byte & 0xFFu);
}

__global__ void unpack_kernel(const uint8_t* __restrict__ in, int64_t n_rows, int d, int bits,
                              uint8_t* __restrict__ idx) {
  const int rb = d * bits / 8;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n_rows * d) return;
  const int64_t row = e / d;
  const int j = (int)(e % d);
  const uint8_t* p = in + row * rb;
  const int bit = bits * j;
  uint32_t v = p[bit >> 3] >> (bit & 7);
  if ((bit & 7) + bits > 8) v |= (uint32_t)p[(bit >> 3) + 1] << (8 - (bit & 7));
  idx[e] = (uint8_t)(v & ((1u << bits) - 1u));
}

__global__ void quantize_scalar_kernel(const float* __restrict__ y, int64_t n,
                                       const float* __restrict__ b, int nb, uint8_t* __restrict__ idx) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n) return;
  idx[e] = (uint8_t)quantize_one(y[e], b, nb);
}

static int check_span(const tq_span* s) {
  if (!s) return set_error(TQ_ERR_INVALID, "span is NULL");
  if (s->rows < 0 || s->n_tok < 0 || s->heads <= 0 || (s->rows % s->heads) != 0)
    return set_error(TQ_ERR_INVALID, "bad span rows=%d heads=%d n_tok=%d", s->rows, s->heads, s->n_tok);
  if (s->rows > 65535) return set_error(TQ_ERR_UNSUPPORTED, "rows %d > 65535", s->rows);
  return TQ_OK;
}

static bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }

}  // namespace tq

using namespace tq;

extern "C" {

int tq_abi_version(void) { return TQ_ABI_VERSION; }

int tq_codec_decode_table(const tq_codec* c, uint64_t* t) {
  if (!c || !t) return set_error(TQ_ERR_INVALID, "codec / table is NULL");
  auto h16 = [](float x) { return (uint64_t)__builtin_bit_cast(uint16_t, (_Float16)x); };
  if (c->n_host_centroids == 16) {
    uint64_t hi[16], lo[16];
    for (int i = 0; i < 16; ++i) {
      const float x = c->host_centroids[i];
      const _Float16 xh = (_Float16)x;
      hi[i] = __builtin_bit_cast(uint16_t, xh);
      lo[i] = h16(x - (float)xh);
    }
    for (int e = 0; e < 256; ++e) t[e] = hi[e & 15] | (hi[e >> 4] << 16) | (lo[e & 15] << 32) | (lo[e >> 4] << 48);
    return TQ_OK;
  }
  if (c->n_host_centroids == 4) {
    for (int e = 0; e < 256; ++e) {
      uint64_t v = 0;
      for (int i = 0; i < 4; ++i) v |= (uint64_t)c->value_table[(e >> (2 * i)) & 3] << (16 * i);
      t[e] = v;
    }
    return TQ_OK;
  }
  return set_error(TQ_ERR_UNSUPPORTED, "decode table: codebook of %d entries", c->n_host_centroids);
}

int tq_codec_prepare(tq_codec* c, const float* cen, int32_t n) {
  if (!c) return set_error(TQ_ERR_INVALID, "codec is NULL");
  c->n_host_centroids = 0;
  for (int i = 0; i < 16; ++i) c->host_centroids[i] = 0.f;
  if (cen && n > 0 && n <= 16) {
    for (int i = 0; i < n; ++i) c->host_centroids[i] = cen[i];
    c->n_host_centroids = n;
  }
  c->value_table[0] = c->value_table[1] = c->value_table[2] = c->value_table[3] = 0;
  c->value_scale = 0.f;
  c->value_table_err = INFINITY;
  if (!cen || n != 4) return TQ_OK;
  // The largest centroid is anchored at an fp16 number m * 2^-14 (m an
  // 11-bit significand); the others are the nearest fp16 numbers of c_i /
  // scale. Of the 1024 anchors the one with the smallest worst relative error
  // (scale rounded to float32 included) is kept.
  int a = 0;
  for (int i = 1; i < 4; ++i)
    if (fabs((double)cen[i]) > fabs((double)cen[a])) a = i;
  const double ca = cen[a];
  if (!(fabs(ca) > 0.0) || !std::isfinite(ca)) return TQ_OK;
  double best = INFINITY;
  for (int m = 1024; m < 2048; ++m) {
    const double ta = (ca < 0 ? -m : m) * 0x1p-14;
    const float scale = (float)(ca / ta);
    uint16_t tab[4];
    double err = 0.0;
    for (int i = 0; i < 4; ++i) {
      const _Float16 t = (_Float16)((double)cen[i] / (double)scale);
      tab[i] = __builtin_bit_cast(uint16_t, t);
      const double got = (double)scale * (double)(float)t;
      const double e = cen[i] == 0.f ? fabs(got) : fabs(got - (double)cen[i]) / fabs((double)cen[i]);
      err = e > err ? e : err;
    }
    if (err < best) {
      best = err;
      for (int i = 0; i < 4; ++i) c->value_table[i] = tab[i];
      c->value_scale = scale;
    }
  }
  c->value_table_err = (float)best;
  return TQ_OK;
}

namespace tq {
// Ring append: workgroup (b*heads + h), thread t < d/8 copies 16 bytes of the
// key, thread d/8 + t the same bytes of the value, into slot slot_b[b].
__global__ __launch_bounds__(256) void ring_append_kernel(const uint4* k, const uint4* v, uint4* rk, uint4* rv,
                                                           int64_t rhs16, int cap, int heads, int d16,
                                                           const int32_t* slot_b) {
  const int row = blockIdx.x, b = row / heads, t = threadIdx.x;
  const int slot = slot_b[b];
  if (slot < 0 || slot >= cap || t >= 2 * d16) return;
  const bool val = t >= d16;
  const int j = val ? t - d16 : t;
  const int64_t dst = (int64_t)row * rhs16 + (int64_t)slot * d16 + j;
  const int64_t src = (int64_t)row * d16 + j;
  if (val)
    rv[dst] = v[src];
  else
    rk[dst] = k[src];
}

// One decode step of a ragged batch in one launch (tq_ragged_step): the
// step's key and value vectors appended to the residual rings, and the
// one-token drains of both sides. Workgroups [0, dwg) drain keys, [dwg, 2 dwg)
// values (the drain workgroup of drain_kernel: the general compress kernel's
// operations, so the stored codes, norms, signs and gamma are bit-identical
// to tq_compress's with a sketch, and to its general kernel without one),
// the rest append. The per-sequence ints are [slot | drain | src | dst |
// caller's extra] (batch each); up to STEP_INL of them travel in the kernel
// arguments and are copied to ints_dev by the first append workgroup,
// otherwise the caller's copy in ints_dev is read.
constexpr int STEP_INL = 512;

struct StepArgs {
  CompressArgs side[2];  // key / value drains over the rings (span arrays unused)
  const uint4* k;
  const uint4* v;
  uint4* rk;
  uint4* rv;
  int64_t rhs16;         // ring head stride, 16-byte units
  int cap, heads, d16, rows, batch;
  int dwg;               // drain workgroups per side
  int awg;               // append workgroups
  int n_ints;
  int inl;               // the ints are in `ints` (else only in ints_dev)
  int32_t* ints_dev;
  int32_t ints[STEP_INL];
};
static_assert(sizeof(StepArgs) <= 4096, "kernel arguments of at most 4 KB");

__global__ __launch_bounds__(DRW * 64) void step_kernel(StepArgs A) {
  __shared__ __align__(16) DrainLds L;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wg = blockIdx.x;
  const int32_t* seqi = A.inl ? A.ints : A.ints_dev;
  if (wg >= 2 * A.dwg) {
    // 16-byte piece e of the keys (e < rows d16) or of the values
    const int np = A.rows * A.d16;
    for (int e = (wg - 2 * A.dwg) * (DRW * 64) + tid; e < 2 * np; e += A.awg * (DRW * 64)) {
      const bool val = e >= np;
      const int f = val ? e - np : e;
      const int row = f / A.d16, j = f - row * A.d16;
      const int slot = seqi[row / A.heads];
      if (slot < 0 || slot >= A.cap) continue;
      const int64_t dst = (int64_t)row * A.rhs16 + (int64_t)slot * A.d16 + j;
      if (val)
        A.rv[dst] = A.v[f];
      else
        A.rk[dst] = A.k[f];
    }
    if (wg == 2 * A.dwg && A.inl)
      for (int i = tid; i < A.n_ints; i += DRW * 64) A.ints_dev[i] = A.ints[i];
    return;
  }
  const int sd = wg >= A.dwg ? 1 : 0;
  const CompressArgs& a = A.side[sd];
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int B = A.batch;
  const DrainIn in = drain_begin(a, L, (wg - sd * A.dwg) * DRW + w, w, lane,
                                 [&](int b) { return SeqRange{seqi[B + b], seqi[2 * B + b], seqi[3 * B + b]}; });
  drain_stage(a, L, tid);
  __syncthreads();  // the only barrier: waves without a vector leave after it
  if (in.ok) drain_vector(a, L, w, lane, in);
}
}  // namespace tq

const char* tq_last_error(void) { return tq::g_err; }

int tq_ring_append(const void* k, const void* v, int32_t dtype, void* ring_k, void* ring_v, int64_t ring_head_stride,
                   int32_t ring_cap, int32_t batch, int32_t heads, int32_t d, const int32_t* slot_b, void* stream) {
  using namespace tq;
  if (dtype != TQ_F16 && dtype != TQ_BF16) return set_error(TQ_ERR_UNSUPPORTED, "ring_append: dtype %d", dtype);
  if (!k || !v || !ring_k || !ring_v || !slot_b) return set_error(TQ_ERR_INVALID, "ring_append: NULL pointer");
  if (batch < 0 || heads <= 0 || d <= 0 || d % 8 || d > 1024 || ring_cap <= 0 || ring_head_stride % 8 ||
      ring_head_stride < (int64_t)ring_cap * d)
    return set_error(TQ_ERR_INVALID, "ring_append: bad shape (batch %d heads %d d %d cap %d stride %lld)", batch, heads,
                     d, ring_cap, (long long)ring_head_stride);
  const auto a16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  if (!a16(k) || !a16(v) || !a16(ring_k) || !a16(ring_v))
    return set_error(TQ_ERR_INVALID, "ring_append: pointers must be 16-byte aligned");
  if (batch == 0) return TQ_OK;
  const int64_t rows = (int64_t)batch * heads;
  if (rows >= ((int64_t)1 << 31)) return set_error(TQ_ERR_INVALID, "ring_append: too many rows");
  const int d16 = d / 8;
  hipLaunchKernelGGL(ring_append_kernel, dim3((unsigned)rows), dim3(((2 * d16 + 63) / 64) * 64), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint4*>(k), static_cast<const uint4*>(v),
                     static_cast<uint4*>(ring_k), static_cast<uint4*>(ring_v), ring_head_stride / 8, (int)ring_cap,
                     (int)heads, d16, slot_b);
  TQ_LAUNCH_CHECK("tq_ring_append");
  return TQ_OK;
}

int tq_ragged_step(const tq_codec* kcodec, const tq_codec* vcodec, const void* k, const void* v, int32_t dtype,
                   void* ring_k, void* ring_v, int64_t ring_head_stride, int32_t ring_cap, const tq_store* kstore,
                   const tq_store* vstore, int32_t batch, int32_t heads, const int32_t* seq_ints, int32_t n_ints,
                   int32_t* seq_ints_dev, void* stream) {
  using namespace tq;
  int rc = check_codec(kcodec);
  if (rc || (rc = check_codec(vcodec))) return rc;
  if (dtype != TQ_F16 && dtype != TQ_BF16) return set_error(TQ_ERR_UNSUPPORTED, "ragged_step: dtype %d", dtype);
  if (!k || !v || !ring_k || !ring_v || !kstore || !vstore || !seq_ints || !seq_ints_dev)
    return set_error(TQ_ERR_INVALID, "ragged_step: NULL pointer");
  if (batch < 0 || heads <= 0 || ring_cap <= 0 || (ring_head_stride & 7) || ring_head_stride < (int64_t)ring_cap * 128 ||
      n_ints < 4 * batch || (int64_t)batch * heads >= ((int64_t)1 << 24))
    return set_error(TQ_ERR_INVALID, "ragged_step: bad shape (batch %d heads %d cap %d stride %lld ints %d)", batch, heads,
                     ring_cap, (long long)ring_head_stride, n_ints);
  // the one-token drain workgroup serves d = 128, with a sketch of at most
  // 128 projections or none (the general compress kernel's operations, as in
  // the tq_compress drain route); other codecs use tq_ring_append + tq_compress
  const tq_codec* cs[2] = {kcodec, vcodec};
  const tq_store* ss[2] = {kstore, vstore};
  bool sk[2];
  for (int i = 0; i < 2; ++i) {
    const tq_codec* c = cs[i];
    const tq_store* st = ss[i];
    sk[i] = c->qjl_proj && st->signs;  // the sketch is stored where the store has sign rows
    if (c->d != 128 || (sk[i] && c->qjl_m > 128) || (reinterpret_cast<uintptr_t>(c->rotation) & 15) ||
        (sk[i] && (reinterpret_cast<uintptr_t>(c->qjl_proj) & 15)))
      return set_error(TQ_ERR_UNSUPPORTED, "ragged_step: codec (d %d, qjl_m %d) has no one-launch step", c->d, c->qjl_m);
    if (!st->codes_hi || !st->norms || (sk[i] && !st->gamma) || (c->split < c->d && !st->codes_lo))
      return set_error(TQ_ERR_INVALID, "ragged_step: store without codes / norms (or gamma with a sketch)");
    if (!aligned4(st->codes_hi) || (st->hi_head_stride & 3) || (st->codes_lo && (!aligned4(st->codes_lo) || (st->lo_head_stride & 3))) ||
        (sk[i] && (!aligned4(st->signs) || (st->sign_head_stride & 3))))
      return set_error(TQ_ERR_INVALID, "ragged_step: packed outputs must be 4-byte aligned");
  }
  const auto a16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  if (!a16(k) || !a16(v) || !a16(ring_k) || !a16(ring_v))
    return set_error(TQ_ERR_INVALID, "ragged_step: k, v and the rings must be 16-byte aligned");
  // a drained ring position is read while the appends write: never the same slot
  for (int b = 0; b < batch; ++b) {
    const int slot = seq_ints[b], dr = seq_ints[batch + b], src = seq_ints[2 * batch + b], dst = seq_ints[3 * batch + b];
    if (dr != 0 && dr != 1) return set_error(TQ_ERR_INVALID, "ragged_step: drain count %d of sequence %d", dr, b);
    if (dr && (src < 0 || src >= ring_cap || dst < 0 || slot == src))
      return set_error(TQ_ERR_INVALID, "ragged_step: sequence %d drains ring slot %d to token %d (append slot %d)", b, src,
                       dst, slot);
  }
  if (batch == 0) return TQ_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  StepArgs A;
  for (int i = 0; i < 2; ++i) {
    const tq_codec* c = cs[i];
    CompressArgs& a = A.side[i];
    a.x = i ? ring_v : ring_k;
    a.x_dtype = dtype;
    a.x_hs = ring_head_stride;
    a.span = tq_span{batch * heads, heads, 1, 0, nullptr, nullptr, nullptr};
    a.dst = *ss[i];
    a.rot = c->rotation;
    a.bnd_hi = c->boundaries_hi;
    a.bnd_lo = c->split < c->d ? c->boundaries_lo : c->boundaries_hi;
    a.cen_hi = c->centroids_hi;
    a.cen_lo = c->split < c->d ? c->centroids_lo : c->centroids_hi;
    a.proj = sk[i] ? c->qjl_proj : nullptr;
    a.qjl_m = sk[i] ? c->qjl_m : 0;
    a.d = c->d;
    a.bits_hi = c->bits_hi;
    a.bits_lo = c->split < c->d ? c->bits_lo : c->bits_hi;
    a.split = c->split;
    a.row_hi = row_bytes(c->split, c->bits_hi);
    a.row_lo = row_bytes(c->d - c->split, a.bits_lo);
    a.row_sign = a.qjl_m / 8;
  }
  A.k = static_cast<const uint4*>(k);
  A.v = static_cast<const uint4*>(v);
  A.rk = static_cast<uint4*>(ring_k);
  A.rv = static_cast<uint4*>(ring_v);
  A.rhs16 = ring_head_stride / 8;
  A.cap = ring_cap;
  A.heads = heads;
  A.d16 = 16;
  A.rows = batch * heads;
  A.batch = batch;
  A.dwg = (A.rows + DRW - 1) / DRW;
  A.awg = (2 * A.rows * A.d16 + DRW * 64 - 1) / (DRW * 64);
  A.n_ints = n_ints;
  A.ints_dev = seq_ints_dev;
  A.inl = n_ints <= STEP_INL;
  if (A.inl) {
    memcpy(A.ints, seq_ints, sizeof(int32_t) * n_ints);
  } else if (hipMemcpyAsync(seq_ints_dev, seq_ints, sizeof(int32_t) * n_ints, hipMemcpyHostToDevice, s) != hipSuccess) {
    return set_error(TQ_ERR_LAUNCH, "ragged_step: copy of the sequence ints: %s", hipGetErrorString(hipGetLastError()));
  }
  hipLaunchKernelGGL(step_kernel, dim3((unsigned)(2 * A.dwg + A.awg)), dim3(DRW * 64), 0, s, A);
  TQ_LAUNCH_CHECK("tq_ragged_step");
  return TQ_OK;
}

int tq_device_supported(void) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  hipDeviceProp_t p;
  if (hipGetDeviceProperties(&p, dev) != hipSuccess) return 0;
  return strncmp(p.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

int tq_compress(const tq_codec* codec, const void* x, int32_t x_dtype, int64_t x_head_stride,
                const tq_span* span, const tq_store* dst, void* stream) {
  int rc = check_codec(codec);
  if (rc) return rc;
  if ((rc = check_span(span))) return rc;
  if (x_dtype != TQ_F16 && x_dtype != TQ_BF16 && x_dtype != TQ_F32)
    return set_error(TQ_ERR_UNSUPPORTED, "compress: unknown input dtype %d", x_dtype);
  if (!x || !dst || !dst->codes_hi || !dst->norms)
    return set_error(TQ_ERR_INVALID, "compress: NULL input/output pointer");
  if (codec->split < codec->d && !dst->codes_lo)
    return set_error(TQ_ERR_INVALID, "compress: fractional codec needs codes_lo");
  const bool qjl = codec->qjl_proj && dst->signs;
  if (qjl && !dst->gamma) return set_error(TQ_ERR_INVALID, "compress: QJL needs gamma output");
  if (!aligned4(dst->codes_hi) || (dst->hi_head_stride & 3) ||
      (dst->codes_lo && (!aligned4(dst->codes_lo) || (dst->lo_head_stride & 3))) ||
      (qjl && (!aligned4(dst->signs) || (dst->sign_head_stride & 3))))
    return set_error(TQ_ERR_INVALID, "compress: packed outputs must be 4-byte aligned");
  if (span->rows == 0 || span->n_tok == 0) return TQ_OK;
  CompressArgs a;
  a.x = x;
  a.x_dtype = x_dtype;
  a.x_hs = x_head_stride;
  a.span = *span;
  a.dst = *dst;
  a.rot = codec->rotation;
  a.bnd_hi = codec->boundaries_hi;
  a.bnd_lo = codec->split < codec->d ? codec->boundaries_lo : codec->boundaries_hi;
  a.cen_hi = codec->centroids_hi;
  a.cen_lo = codec->split < codec->d ? codec->centroids_lo : codec->centroids_hi;
  a.proj = qjl ? codec->qjl_proj : nullptr;
  a.qjl_m = qjl ? codec->qjl_m : 0;
  a.d = codec->d;
  a.bits_hi = codec->bits_hi;
  a.bits_lo = codec->split < codec->d ? codec->bits_lo : codec->bits_hi;
  a.split = codec->split;
  a.row_hi = row_bytes(codec->split, codec->bits_hi);
  a.row_lo = row_bytes(codec->d - codec->split, a.bits_lo);
  a.row_sign = a.qjl_m / 8;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // small spans with the QJL sketch (one-token decode drains): one vector per
  // wave (without a sketch the MFMA kernel below is as fast on such spans)
  if (codec->d == 128 && qjl && codec->qjl_m <= 128 && span->n_tok <= 8 && !(codec->flags & TQ_CODEC_GENERAL_COMPRESS) &&
      !(reinterpret_cast<uintptr_t>(codec->rotation) & 15) && !(reinterpret_cast<uintptr_t>(codec->qjl_proj) & 15)) {
    const int64_t nvec = (int64_t)span->rows * span->n_tok;
    hipLaunchKernelGGL(drain_kernel, dim3((unsigned)((nvec + DRW - 1) / DRW)), dim3(DRW * 64), 0, s, a);
    TQ_LAUNCH_CHECK("tq_compress (drain)");
    return TQ_OK;
  }
  // fp16, head_dim 128, no QJL sketch: the MFMA kernel (tq_compress_fast.hip)
  if (codec->d == 128 && !(codec->flags & TQ_CODEC_GENERAL_COMPRESS) && launch_compress_fast(a, s)) {
    TQ_LAUNCH_CHECK("tq_compress");
    return TQ_OK;
  }
  launch_padded(codec->d, [&](auto dp) {
    constexpr int DP = decltype(dp)::value;
    dim3 g((span->n_tok + Geo<DP>::VPW - 1) / Geo<DP>::VPW, span->rows);
    hipLaunchKernelGGL(compress_kernel<DP>, g, dim3(256), 0, s, a);
  });
  TQ_LAUNCH_CHECK("tq_compress");
  return TQ_OK;
}

int tq_dequantize(const tq_codec* codec, const tq_store* src, const tq_span* span, float* out,
                  int64_t out_head_stride, int32_t apply_qjl, void* stream) {
  int rc = check_codec(codec);
  if (rc) return rc;
  if ((rc = check_span(span))) return rc;
  if (!src || !src->codes_hi || !src->norms || !out)
    return set_error(TQ_ERR_INVALID, "dequantize: NULL input/output pointer");
  if (codec->split < codec->d && !src->codes_lo)
    return set_error(TQ_ERR_INVALID, "dequantize: fractional codec needs codes_lo");
  const bool qjl = apply_qjl && codec->qjl_proj && src->signs && src->gamma;
  if (apply_qjl && !qjl) return set_error(TQ_ERR_INVALID, "dequantize: QJL needs projection, signs, gamma");
  if ((reinterpret_cast<uintptr_t>(out) & 15) || (out_head_stride & 3))
    return set_error(TQ_ERR_INVALID, "dequantize: output must be 16-byte aligned");
  if (span->rows == 0 || span->n_tok == 0) return TQ_OK;
  DequantArgs a;
  a.src = *src;
  a.span = *span;
  a.out = out;
  a.out_hs = out_head_stride;
  a.rot = codec->rotation;
  a.cen_hi = codec->centroids_hi;
  a.cen_lo = codec->split < codec->d ? codec->centroids_lo : codec->centroids_hi;
  a.proj = qjl ? codec->qjl_proj : nullptr;
  a.qjl_m = qjl ? codec->qjl_m : 0;
  a.apply_qjl = qjl ? 1 : 0;
  a.d = codec->d;
  a.bits_hi = codec->bits_hi;
  a.bits_lo = codec->split < codec->d ? codec->bits_lo : codec->bits_hi;
  a.split = codec->split;
  a.row_hi = row_bytes(codec->split, codec->bits_hi);
  a.row_lo = row_bytes(codec->d - codec->split, a.bits_lo);
  a.row_sign = a.qjl_m / 8;
  hipStream_t s = static_cast<hipStream_t>(stream);
  launch_padded(codec->d, [&](auto dp) {
    constexpr int DP = decltype(dp)::value;
    dim3 g((span->n_tok + Geo<DP>::VPW - 1) / Geo<DP>::VPW, span->rows);
    hipLaunchKernelGGL(dequant_kernel<DP>, g, dim3(256), 0, s, a);
  });
  TQ_LAUNCH_CHECK("tq_dequantize");
  return TQ_OK;
}

int tq_pack_codes(const uint8_t* idx, int64_t n_rows, int32_t d, int32_t bits, uint8_t* packed,
                  void* stream) {
  if (bits < 1 || bits > 4)
    return set_error(TQ_ERR_UNSUPPORTED, "Unsupported bit-width: %d. Use 1, 2, 3, or 4.", bits);
  if (d <= 0 || (d * bits) % 8 != 0)
    return set_error(TQ_ERR_INVALID, "Last dimension %d cannot be packed at %d bits", d, bits);
  if (n_rows < 0) return set_error(TQ_ERR_INVALID, "n_rows < 0");
  const int64_t n = n_rows * (int64_t)(d * bits / 8);
  if (n == 0) return TQ_OK;
  if (!idx || !packed) return set_error(TQ_ERR_INVALID, "pack: NULL pointer");
  hipLaunchKernelGGL(pack_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), idx, n_rows, d, bits, packed);
  TQ_LAUNCH_CHECK("tq_pack_codes");
  return TQ_OK;
}

int tq_unpack_codes(const uint8_t* packed, int64_t n_rows, int32_t d, int32_t bits, uint8_t* idx,
                    void* stream) {
  if (bits < 1 || bits > 4)
    return set_error(TQ_ERR_UNSUPPORTED, "Unsupported bit-width: %d. Use 1, 2, 3, or 4.", bits);
  if (d <= 0 || (d * bits) % 8 != 0)
    return set_error(TQ_ERR_INVALID, "Last dimension %d cannot be unpacked at %d bits", d, bits);
  if (n_rows < 0) return set_error(TQ_ERR_INVALID, "n_rows < 0");
  const int64_t n = n_rows * (int64_t)d;
  if (n == 0) return TQ_OK;
  if (!idx || !packed) return set_error(TQ_ERR_INVALID, "unpack: NULL pointer");
  hipLaunchKernelGGL(unpack_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), packed, n_rows, d, bits, idx);
  TQ_LAUNCH_CHECK("tq_unpack_codes");
  return TQ_OK;
}

int tq_quantize_scalar(const float* y, int64_t n, const float* boundaries, int32_t n_boundaries,
                       uint8_t* idx, void* stream) {
  if (n < 0 || n_boundaries < 0 || n_boundaries > 255)
    return set_error(TQ_ERR_INVALID, "quantize_scalar: bad sizes");
  if (n == 0) return TQ_OK;
  if (!y || !idx || (n_boundaries && !boundaries))
    return set_error(TQ_ERR_INVALID, "quantize_scalar: NULL pointer");
  hipLaunchKernelGGL(quantize_scalar_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), y, n, boundaries, n_boundaries, idx);
  TQ_LAUNCH_CHECK("tq_quantize_scalar");
  return TQ_OK;
}

}  // extern "C"
