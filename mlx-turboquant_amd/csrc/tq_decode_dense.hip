// Decode attention over uncompressed K/V (fp16 or bf16) on gfx950: the layers
// a TurboQuant model keeps uncompressed (outlier and skipped layers, which the
// reference hands a plain KVCache, patch.py:337-338) and TurboQuant caches whose
// tokens all still sit in the fp16 sink and residual window.
//
// Grid (nwg, hkv, batch), DENSE_WAVES waves per workgroup. The tokens of
// sequence b and kv head g form up to three contiguous pieces: the sink
// [0, S), the residual ring from its start slot to the ring's end, and the
// part of the ring that wrapped to slot 0. Each piece is cut into 32-token
// blocks (the last one partial and masked), so a block always reads
// contiguous rows. Workgroup c owns blocks [c*W*bpw, (c+1)*W*bpw) of the
// concatenated block list and wave w takes every W-th of them, with the next
// block's loads in flight while it computes the current one.
//
// Scores, transposed: S^T = K q^T with MFMA 16x16x32 (f16, or bf16 for bf16
// caches). A = 16 tokens x 32 dims of keys loaded straight from memory;
// B = 32 dims x 16 query columns, column c < 8 the high part of query head c
// (pre-scaled by scale * log2 e) and column c + 8 its remainder, so adding
// the value 8 lanes over (a DPP row rotation) gives the full score in both
// lanes. Lane (column c, group q4) then holds the scores of tokens 4q4 + i
// (tile 0) and 16 + 4q4 + i (tile 1), i < 4, which are the k-slots 8q4 + j of
// the A operand of O = P V: rows c < 8 take the high part of p, rows c >= 8
// its remainder. B of O = P V is V with 16 dims as columns: lane (n, q4)
// loads dims 8n .. 8n + 7 of its 8 tokens (16 bytes of each row) and v_perm
// pairs the tokens, so MFMA m produces dims 8n + m. Output rows h and h + 8
// are added at the end.
//
// Online softmax in base 2 with a lazily raised running max (raised with a
// margin, so most blocks need no rescale). The waves of a workgroup combine
// through LDS into one partial per query head (max, sum, output / sum); the
// K4/V2 path's merge kernel combines the partials, or a lone workgroup writes
// the output itself.

#include <math.h>

#include "tq_common.h"
#include "tq_decode_fast.h"

namespace tq {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int DD = 128;                  // head dim
constexpr int DW = DENSE_WAVES;          // waves per workgroup
constexpr int DT = DW * 64;              // threads per workgroup
constexpr int PS = FAST_PART_FLOATS;     // floats per (workgroup, head) partial
constexpr int P_OUT = 4;                 // partial: [M, L, pad, pad, out[128]]
constexpr float M_INIT = -1e30f;         // running max before the first block
constexpr float RESCALE_MARGIN = 3.f;    // the running max is raised to block max + margin

template <bool BF>
__device__ inline f4 mma(u4 a, u4 b, f4 c) {
  if constexpr (BF)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf8, a), __builtin_bit_cast(bf8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0, 0, 0);
}

// float -> element bits (round to nearest even) and back
template <bool BF>
__device__ inline uint32_t to_e(float x) {
  if constexpr (BF)
    return __builtin_bit_cast(uint16_t, (__bf16)x);
  else
    return __builtin_bit_cast(uint16_t, (_Float16)x);
}

template <bool BF>
__device__ inline float from_e(uint32_t h) {
  if constexpr (BF)
    return __uint_as_float(h << 16);
  else
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// high part of x (hi_lane) or the remainder x - high part, as element bits
template <bool BF>
__device__ inline uint32_t split_e(float x, bool lo_lane) {
  const uint32_t hi = to_e<BF>(x);
  return lo_lane ? to_e<BF>(x - from_e<BF>(hi)) : hi;
}

__device__ inline float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }

// value of lane (i - 8) mod 16 of the same 16-lane row
__device__ inline float row_ror8(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, true));
}

// max / sum over the four 16-lane rows (lanes l, l^16, l^32, l^48)
__device__ inline float rows_max(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ inline float rows_sum(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// v + the value of lane l ^ 32
__device__ inline float add_half32(float v) {
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// token of k-slot 8 q4 + j of a 32-token block
__device__ inline int slot_token(int q4, int j) { return j < 4 ? 4 * q4 + j : 16 + 4 * q4 + (j - 4); }

// The tokens of one (sequence, kv head): pieces sink, ring head, ring wrap.
// Named fields and selects only: a dynamically indexed array would live in
// scratch memory, whose loads share the vector-memory counter with the tile
// prefetch and would make every wait on them drain it.
struct Seq {
  const uint16_t *k0, *k1, *k2;
  const uint16_t *v0, *v1, *v2;
  int len0, len1, len2;
  int nb0, nb01, nb;  // block counts: piece 0, pieces 0-1, all
};

struct Blk {
  const uint16_t* k;
  const uint16_t* v;
  int off, len;  // first token of the block within its piece, piece length
};

__device__ inline Blk block_at(const Seq s, int j) {
  const bool in0 = j < s.nb0, in1 = !in0 && j < s.nb01;
  Blk b;
  b.k = in0 ? s.k0 : (in1 ? s.k1 : s.k2);
  b.v = in0 ? s.v0 : (in1 ? s.v1 : s.v2);
  b.len = in0 ? s.len0 : (in1 ? s.len1 : s.len2);
  b.off = 32 * (j - (in0 ? 0 : (in1 ? s.nb0 : s.nb01)));
  return b;
}

// Loads of one block, lane (r, q4): key rows off + r and off + 16 + r, dims
// 32 kb + 8 q4 .. + 8 (A of the score MFMA kb); value rows of the 8 k-slots,
// dims 8 r .. 8 r + 7. Rows past the piece re-read its last row (masked).
struct Tile {
  u4 k[2][4];
  u4 v[8];
};

// Tile loads: 16-byte non-temporal loads the compiler sees (it inserts
// every wait itself).
template <int OFF>
__device__ inline u4 gload(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u4*>(static_cast<const uint8_t*>(p) + OFF));
}

__device__ inline void load_tile(Tile& t, const Blk& bk, int r, int q4) {
  const int last = bk.len - 1;
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const uint16_t* p = bk.k + (int64_t)min(bk.off + 16 * tt + r, last) * DD + 8 * q4;
    t.k[tt][0] = gload<0>(p);
    t.k[tt][1] = gload<64>(p);
    t.k[tt][2] = gload<128>(p);
    t.k[tt][3] = gload<192>(p);
  }
#pragma unroll
  for (int j = 0; j < 8; ++j)
    t.v[j] = gload<0>(bk.v + (int64_t)min(bk.off + slot_token(q4, j), last) * DD + 8 * r);
}

template <int G, bool BF>
__global__ __launch_bounds__(DT) __attribute__((amdgpu_waves_per_eu(2))) void dense_decode_kernel(DenseArgs a) {
  __shared__ __align__(16) float cmb[DW][8][DD];  // per (wave, head) output, unnormalised
  __shared__ float cml[DW][2][8];                 // per (wave, head) running max, sum
  const int c = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, r = lane & 15, q4 = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: block choice stays scalar
  const int64_t row = (int64_t)b * a.hkv + g;

  Seq sq;
  {
    // per-sequence values clamped to the bounds the host checked (reads stay in the buffers)
    const int S = a.sink_len_b ? min(max(a.sink_len_b[b], 0), a.max_sink) : a.max_sink;
    const int R = a.res_len_b ? min(max(a.res_len_b[b], 0), a.max_res) : a.max_res;
    const int rs = a.res_start_b ? min(max(a.res_start_b[b], 0), max(a.res_cap - 1, 0)) : a.res_start0;
    const int RA = R > 0 ? min(R, a.res_cap - rs) : 0;
    const uint16_t* sk = static_cast<const uint16_t*>(a.sink_k) + row * a.sink_hs;
    const uint16_t* sv = static_cast<const uint16_t*>(a.sink_v) + row * a.sink_hs;
    const uint16_t* rk = static_cast<const uint16_t*>(a.res_k) + row * a.res_hs;
    const uint16_t* rv = static_cast<const uint16_t*>(a.res_v) + row * a.res_hs;
    sq.k0 = sk; sq.v0 = sv; sq.len0 = S;
    sq.k1 = rk + (int64_t)rs * DD; sq.v1 = rv + (int64_t)rs * DD; sq.len1 = RA;
    sq.k2 = rk; sq.v2 = rv; sq.len2 = R - RA;
    sq.nb0 = (S + 31) >> 5;
    sq.nb01 = sq.nb0 + ((RA + 31) >> 5);
    sq.nb = sq.nb01 + ((R - RA + 31) >> 5);
  }

  // B operand of the score MFMAs: column r holds part (r >= 8) of head r & 7,
  // dims 32 kb + 8 q4 .. + 8 (16-byte pieces of the query row, 16-byte
  // aligned: checked on the host); zero for heads past G. The raw query
  // pieces and the first two blocks are loaded together, then converted.
  const bool lo_lane = r >= 8;
  const int h = r & 7;
  const int64_t qo = ((int64_t)b * a.hq + g * G + min(h, G - 1)) * DD + 8 * q4;
  const bool q32 = a.q_dtype == TQ_F32;
  u4 qr[8];
  {
    // 8 loads in both cases (fp16 / bf16 rows re-read their 4 pieces), so
    // the explicit wait below counts the same loads
    const uint8_t* p = static_cast<const uint8_t*>(a.q) + qo * (q32 ? 4 : 2);
    const int step = q32 ? 128 : 64;  // bytes between the pieces of consecutive kb
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int kb = q32 ? (i >> 1) : (i & 3);
      qr[i] = gload<0>(p + kb * step + (q32 ? 16 * (i & 1) : 0));
    }
  }

  const int jbeg = c * DW * a.bpw + w;
  const int jend = min(sq.nb, (c + 1) * DW * a.bpw);
  Tile t0, t1;
  {
    // a wave without blocks loads the first 256 bytes of its query rows instead (unused)
    const uint16_t* qrow = static_cast<const uint16_t*>(a.q) + ((int64_t)b * a.hq + g * G) * DD * (q32 ? 2 : 1);
    const bool any = jbeg < jend;
    const Blk first = any ? block_at(sq, jbeg) : Blk{qrow, qrow, 0, 1};
    const Blk second = any ? block_at(sq, min(jbeg + DW, jend - 1)) : first;
    load_tile(t0, first, r, q4);
    load_tile(t1, second, r, q4);
  }

  u4 qop[4];
  {
    float x[4][8];
    if (q32) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 8; ++e) x[kb][e] = __uint_as_float(qr[2 * kb + (e >> 2)][e & 3]);
    } else if (a.q_dtype == TQ_BF16) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 8; ++e) x[kb][e] = __uint_as_float(((qr[kb][e >> 1] >> (16 * (e & 1))) & 0xFFFFu) << 16);
    } else {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 8; ++e)
          x[kb][e] = (float)__builtin_bit_cast(_Float16, (uint16_t)(qr[kb][e >> 1] >> (16 * (e & 1))));
    }
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        uint32_t x0 = 0u, x1 = 0u;
        if (h < G) {
          x0 = split_e<BF>(x[kb][2 * e] * a.qscale, lo_lane);
          x1 = split_e<BF>(x[kb][2 * e + 1] * a.qscale, lo_lane);
        }
        qop[kb][e] = x0 | (x1 << 16);
      }
  }

  f4 acc[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) acc[m] = f4{0.f, 0.f, 0.f, 0.f};
  float m_run = M_INIT, l_run = 0.f;

  auto compute = [&](const Tile& t, const Blk& bk) {
    f4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = s0;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      s0 = mma<BF>(t.k[0][kb], qop[kb], s0);
      s1 = mma<BF>(t.k[1][kb], qop[kb], s1);
    }
    float s[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s[i] = s0[i] + row_ror8(s0[i]);
      s[4 + i] = s1[i] + row_ror8(s1[i]);
    }
    if (bk.off + 32 > bk.len) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (bk.off + slot_token(q4, j) >= bk.len) s[j] = -INFINITY;
    }
    float bm = s[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) bm = fmaxf(bm, s[j]);
    bm = rows_max(bm);
    if (__any(bm > m_run)) {
      const float mnew = bm > m_run ? bm + RESCALE_MARGIN : m_run;
      const float al = fexp2(m_run - mnew);
      m_run = mnew;
      l_run *= al;
      // accumulator row 4 q4 + i is query column 4 q4 + i, whose factor lane 4 q4 + i holds
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float ai = __shfl(al, 4 * q4 + i);
#pragma unroll
        for (int m = 0; m < 8; ++m) acc[m][i] *= ai;
      }
    }
    float p[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      p[j] = fexp2(s[j] - m_run);
      l_run += p[j];
    }
    u4 pa;
#pragma unroll
    for (int e = 0; e < 4; ++e) pa[e] = split_e<BF>(p[2 * e], lo_lane) | (split_e<BF>(p[2 * e + 1], lo_lane) << 16);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const uint32_t sel = (m & 1) ? 0x07060302u : 0x05040100u;
      u4 bv;
#pragma unroll
      for (int e = 0; e < 4; ++e) bv[e] = __builtin_amdgcn_perm(t.v[2 * e + 1][m >> 1], t.v[2 * e][m >> 1], sel);
      acc[m] = mma<BF>(pa, bv, acc[m]);
    }
  };

  // Two tiles rotate in fixed registers: each is refilled with the block two
  // steps ahead right after it has been consumed, so one block is in flight
  // while the other is computed (16 loads issued after the ones waited for).
  // Refills past the wave's last block re-read an earlier block (L2); an odd
  // block count ends with a fully masked step (len 0).
  if (jbeg < jend) {
    const int npair = ((jend - jbeg + DW - 1) / DW + 1) / 2;
    for (int it = 0; it < npair; ++it) {
      const int j = jbeg + 2 * DW * it;
      compute(t0, block_at(sq, j));
      load_tile(t0, block_at(sq, min(j + 2 * DW, jend - 1)), r, q4);
      compute(t1, j + DW < jend ? block_at(sq, j + DW) : Blk{nullptr, nullptr, 0, 0});
      load_tile(t1, block_at(sq, min(j + 3 * DW, jend - 1)), r, q4);
    }
  }

  // column sums over the four groups; high part + remainder rows (h, h + 8)
  l_run = rows_sum(l_run);
#pragma unroll
  for (int m = 0; m < 8; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[m][i] = add_half32(acc[m][i]);
  if (q4 == 0 && r < G) {
    cml[w][0][r] = m_run;
    cml[w][1][r] = l_run;
  }
  if (q4 < 2) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * q4 + i;
      if (h < G) {
        float4* dst = reinterpret_cast<float4*>(&cmb[w][h][8 * r]);
        dst[0] = make_float4(acc[0][i], acc[1][i], acc[2][i], acc[3][i]);
        dst[1] = make_float4(acc[4][i], acc[5][i], acc[6][i], acc[7][i]);
      }
    }
  }
  __syncthreads();
  for (int e = tid; e < G * DD; e += DT) {
    const int h = e / DD, d = e % DD;
    float M = M_INIT;
#pragma unroll
    for (int v = 0; v < DW; ++v) M = fmaxf(M, cml[v][0][h]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int v = 0; v < DW; ++v) {
      const float wt = fexp2(cml[v][0][h] - M);
      L += wt * cml[v][1][h];
      O += wt * cmb[v][h][d];
    }
    const float val = L > 0.f ? O / L : 0.f;
    if (a.nwg == 1) {
      a.out[((int64_t)b * a.hq + g * G + h) * DD + d] = val;
    } else {
      float* part = a.part + ((row * a.nwg + c) * G + h) * PS;
      part[P_OUT + d] = val;
      if (d == 0) {
        part[0] = M;
        part[1] = L;
      }
    }
  }
}

template <int G>
void launch_g(const DenseArgs& a, bool bf, int batch, hipStream_t s) {
  const dim3 grid(a.nwg, a.hkv, batch);
  if (bf)
    hipLaunchKernelGGL((dense_decode_kernel<G, true>), grid, dim3(DT), 0, s, a);
  else
    hipLaunchKernelGGL((dense_decode_kernel<G, false>), grid, dim3(DT), 0, s, a);
}

}  // namespace

// Workgroups per (sequence, kv head) and blocks per wave: about one
// workgroup per CU in total (measured: 5.6 TB/s at 65536 tokens against 5.2
// with two per CU and 4.8 with four), at least one block per wave, at most
// FAST_MAX_WG partials for the merge.
void dense_geometry(int batch, int hkv, int max_sink, int max_res, int cus, int& nwg, int& bpw) {
  const int nb = (max_sink + 31) / 32 + (max_res + 31) / 32 + (max_res > 0 ? 1 : 0);
  const int groups = batch * hkv > 0 ? batch * hkv : 1;
  const int target = (cus + groups - 1) / groups;
  int hi = (nb + DW - 1) / DW;
  if (hi < 1) hi = 1;
  nwg = target < hi ? target : hi;
  if (nwg < 1) nwg = 1;
  if (nwg > FAST_MAX_WG) nwg = FAST_MAX_WG;
  bpw = (nb + nwg * DW - 1) / (nwg * DW);
  if (bpw < 1) bpw = 1;
  nwg = (nb + bpw * DW - 1) / (bpw * DW);  // drop workgroups left without blocks
  if (nwg < 1) nwg = 1;
}

int launch_dense_decode(const DenseArgs& a, int G, bool bf, int batch, int merge, hipStream_t s) {
  switch (G) {
    case 1: launch_g<1>(a, bf, batch, s); break;
    case 2: launch_g<2>(a, bf, batch, s); break;
    case 4: launch_g<4>(a, bf, batch, s); break;
    default: launch_g<8>(a, bf, batch, s); break;
  }
  if (hipGetLastError() != hipSuccess) return -1;
  if (a.nwg > 1 && merge) return launch_partial_merge(a.part, a.nwg, G, a.hq, a.hkv, batch, a.out, s);
  return 0;
}

}  // namespace tq
