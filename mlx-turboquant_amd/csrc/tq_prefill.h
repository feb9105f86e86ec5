// Prefill attention over a TurboQuant cache on gfx950: n_q > 1 query tokens
// per sequence, the cache's last n_q tokens, attending causally (query i sees
// positions <= total - n_q + i; cache.py:722-724), head_dim 128, integer key /
// value widths KB, VB in 2..4, no QJL sketch.
//
// Query rows are (query token, head of the kv group) pairs: row r of kv head
// (b, g) is token r / G of query head g G + r % G. A wave owns NT 16-row tiles
// (the MFMA columns; NT = PREFILL_TILES) and walks a range of 32-token key
// blocks; each block's code rows are decoded once per wave and serve all its
// rows:
//  - scores S^T = K q^T (MFMA 16x16x32 f16, A = 16 keys x 32 dims, B = 32
//    dims x 16 rows): k-slot 8 q4 + e of step s is rotated dim 32 q4 + 8 s + e,
//    so lane (key r, q4) reads the 32 contiguous codes of dims [32 q4, 32 q4 +
//    32) of its key (4 KB bytes) and looks up 2 dims per LDS pair-table entry,
//    (c_hi[a], c_hi[b]) and (c_lo[a], c_lo[b]) (c_hi = fp16(c), c_lo = fp16(c -
//    c_hi)): the high parts make one A operand and the remainders another;
//    the rotated query (scaled by a per-wave power of two) is split the same
//    way, and three MFMAs per step add c_hi q_hi + c_lo q_hi + c_hi q_lo
//    (fp32-class scores);
//  - output O^T += V^T P^T: k-slot 8 q4 + e is key 4 q4 + e of tile 0 (e < 4)
//    or of tile 1, exactly the scores lane (row j, q4) holds, so p * n_v
//    (fp16, round to nearest) is the B operand as it stands; A row i of PV
//    MFMA nb is rotated dim 8 i + nb, its k-slot pairs are token pairs, and one
//    pair-table entry indexed by (code of token a, code of token b) gives the
//    high parts and the remainders of both;
//  - the accumulator of lane (row j, q4), MFMA nb, register e is rotated dim
//    32 q4 + 8 e + nb.
// Online softmax in base 2 with a rescale margin; p * n_v is kept in the fp16
// range by a per-wave power of two (value norms are the same for every row).
//
// The uncompressed tokens (sink and residual ring) take the same path: a
// preparation kernel rotates them into the compressed tokens' space (k R^T,
// v R^T), stores each as a norm and a unit vector in fp16 high part /
// remainder form, keys row-major and values transposed in the PV k-slot
// order, and rotates the queries (q R^T, float32). The key range of a (kv
// head, row group) is split over workgroups; each writes per-row partials
// (max, sum, output / sum) and a merge kernel combines them and applies the
// inverse rotation (value codec R) once per row.
#pragma once

#include <type_traits>

#include "tq_decode_uniform.h"

namespace tq {
namespace pf {

using uk::as_h8;
using uk::f4;
using uk::fexp2;
using uk::half8;
using uk::mfma;
using uk::rows_max;
using uk::rows_sum;
using uk::rsrc;
using uk::u2;
using uk::u3;
using uk::u4;

constexpr int D = 128;
constexpr int NT = PREFILL_TILES;    // 16-row query tiles per wave
constexpr int WR = PREFILL_WAVE_ROWS;  // query rows per wave
constexpr int PW = PREFILL_WAVES;    // waves per workgroup
constexpr int PT = 64 * PW;          // threads per workgroup
constexpr int PART = PREFILL_PART_FLOATS;
constexpr float M_INIT = -1e30f;
constexpr float MARGIN = 3.f;        // base-2 headroom added when the running max rises
constexpr float PV_LIMIT = 32768.f;  // p * n_v 2^-vx above this: vx grows
constexpr float PV_SET = 2048.f;     // the first block with values sets vx so its largest n_v 2^-vx is near this
constexpr float LOG2E = 1.4426950408889634f;

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// fp16 pair (round to nearest even) as one dword
__device__ inline uint32_t pack_rn(float a, float b) {
  const h2 v = {(_Float16)a, (_Float16)b};
  return __builtin_bit_cast(uint32_t, v);
}

// LDS of the prefill kernel: the value pair table at 0 and the key pair table
// at 64 KB. Row e of a table (256 bytes) holds 32 replicas of the entry's
// fp16 high parts (c_hi[e & M], c_hi[e >> B]) in bytes [0, 128) and 32 of its
// remainders in [128, 256): lane l reads replica l & 31 at base + 256 e +
// 4 (l & 31) (+ 128), one dword each, straight into its MFMA operand (the
// address is one byte permute of a code byte when the entry is a byte).
// Then each wave's norm staging, the codebooks, and each wave's accumulator
// rescale area.
template <int KB, int VB>
struct PLds {
  static constexpr uint32_t vlut = 0;
  static constexpr uint32_t klut = 0x10000;
  static constexpr uint32_t nst = klut + (256u << (2 * KB));  // [PW][2][32] f32 key / value norms
  static constexpr uint32_t cen = nst + PW * 256;             // [2][16] f32 key / value centroids
  static constexpr uint32_t rsc = cen + 128;                  // [PW][2][64] f4: a quarter of a query tile
  static constexpr uint32_t total = rsc + PW * 2048;
  static_assert((256u << (2 * VB)) <= klut, "value table below the key table");
  static_assert(total <= 160 * 1024, "LDS of one workgroup");
};

// Pair table of B-bit codes (layout above) from the codebook in LDS.
template <int B>
__device__ inline void pair_table(uint8_t* tab, const float* c, int tid) {
  constexpr int NR = 1 << (2 * B), M = (1 << B) - 1;
  for (int x = tid; x < NR * 16; x += PT) {
    const int e = x >> 4, part = (x >> 3) & 1;
    const float ca = c[e & M], cb = c[e >> B];
    const _Float16 ha = (_Float16)ca, hb = (_Float16)cb;
    const uint32_t v = part == 0 ? pack_rn((float)ha, (float)hb) : pack_rn(ca - (float)ha, cb - (float)hb);
    *reinterpret_cast<u4*>(tab + e * 256 + (x & 15) * 16) = u4{v, v, v, v};
  }
}

// The two dwords of a table entry at `addr` into element m of the high-part
// and remainder operands
__device__ inline void entry(const uint8_t* smem, uint32_t addr, u4& hi, u4& lo, int m) {
  hi[m] = *reinterpret_cast<const uint32_t*>(smem + addr);
  lo[m] = *reinterpret_cast<const uint32_t*>(smem + addr + 128);
}

// byte-address of byte `by` of w with the replica offset c0 (bits 0-7) and
// table base bits 16-23 of c0: one v_perm
__device__ inline uint32_t byte_addr(uint32_t w, uint32_t c0, int by) {
  return __builtin_amdgcn_perm(w, c0, 0x0C020000u | ((4u + by) << 8));
}

// Element i of a row of dtype dt (TQ_F16 / TQ_BF16 / TQ_F32) as float32.
__device__ inline float load_elem(const void* p, int dt, int64_t i) {
  if (dt == TQ_F32) return static_cast<const float*>(p)[i];
  const uint16_t u = static_cast<const uint16_t*>(p)[i];
  if (dt == TQ_BF16) return __uint_as_float((uint32_t)u << 16);
  return (float)__builtin_bit_cast(_Float16, u);
}

__device__ inline int clamp_len(const int32_t* v, int b, int mx) {
  return v ? min(max(v[b], 0), mx) : mx;
}

// Rotation of the query rows and of the uncompressed tokens. Grid (x, kind,
// kv row): kind 0 rotates query rows [32 x, 32 x + 32) with the key codec's R
// (float32 rows of qr); kind 1 / 2 rotates the sink + residual keys / values
// [32 x, 32 x + 32) of the sequence (key codec R / value codec R) and stores
// norm and unit vector (fp16 high part / remainder): keys in rows of dk,
// values transposed per 32-token block in the PV k-slot order (dv). Rows and
// tokens past the call's are written as zeros.
__global__ __launch_bounds__(256) void prefill_prep_kernel(PrefillArgs a) {
  constexpr int RS = D + 4;  // R rows padded against bank conflicts (16-byte aligned)
  __shared__ __align__(16) float rs[D * RS];
  __shared__ __align__(16) float xs[32][D];
  __shared__ float nrm[32];
  const int kind = blockIdx.y, x = blockIdx.x, row = blockIdx.z, tid = threadIdx.x;
  const int n = kind == 0 ? a.nrows_pad : a.nd_pad;
  if (32 * x >= n) return;
  const int b = row / a.hkv, g = row % a.hkv;
  const int sl = clamp_len(a.sink_len, b, a.max_sink), rl = clamp_len(a.res_len, b, a.max_res);
  const int nd = sl + rl;
  int rs0 = a.res_start ? a.res_start[b] : a.res_start0;
  rs0 = min(max(rs0, 0), max(a.res_cap - 1, 0));
  const float* R = kind == 2 ? a.rv : a.rk;
  for (int e = tid; e < D * D / 4; e += 256)
    *reinterpret_cast<float4*>(rs + (e >> 5) * RS + 4 * (e & 31)) = reinterpret_cast<const float4*>(R)[e];
  for (int e = tid; e < 32 * D; e += 256) {
    const int r = e >> 7, i = e & 127, idx = 32 * x + r;
    float v = 0.f;
    if (kind == 0) {
      if (idx < a.nrows) {
        const int qi = idx / a.G, h = idx % a.G;
        v = load_elem(a.q, a.q_dtype, (((int64_t)b * a.hq + g * a.G + h) * a.n_q + qi) * D + i);
      }
    } else if (idx < nd) {
      if (idx < sl) {
        v = load_elem(kind == 1 ? a.sink_k : a.sink_v, a.kv_dtype, (int64_t)row * a.sink_hs + (int64_t)idx * D + i);
      } else {
        int slot = rs0 + idx - sl;
        slot = slot >= a.res_cap ? slot - a.res_cap : slot;
        v = load_elem(kind == 1 ? a.res_k : a.res_v, a.kv_dtype, (int64_t)row * a.res_hs + (int64_t)slot * D + i);
      }
    }
    xs[r][i] = v;
  }
  __syncthreads();
  // y[u] = (x R^T)_j = sum_i R[j][i] x[i] for rows 16 hh + u, dim j
  const int j = tid & 127, hh = tid >> 7;
  float y[16];
#pragma unroll
  for (int u = 0; u < 16; ++u) y[u] = 0.f;
  for (int i = 0; i < D; i += 4) {
    const float4 rr = *reinterpret_cast<const float4*>(rs + j * RS + i);
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const float4 xv = *reinterpret_cast<const float4*>(&xs[16 * hh + u][i]);
      y[u] = fmaf(rr.x, xv.x, fmaf(rr.y, xv.y, fmaf(rr.z, xv.z, fmaf(rr.w, xv.w, y[u]))));
    }
  }
  if (kind == 0) {
#pragma unroll
    for (int u = 0; u < 16; ++u) a.qr[((int64_t)row * a.nrows_pad + 32 * x + 16 * hh + u) * D + j] = y[u];
    return;
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < 16; ++u) xs[16 * hh + u][j] = y[u];
  __syncthreads();
  if (tid < 32) {
    float s = 0.f;
    for (int i = 0; i < D; ++i) s = fmaf(xs[tid][i], xs[tid][i], s);
    nrm[tid] = sqrtf(s);
    (kind == 1 ? a.dnk : a.dnv)[(int64_t)row * a.nd_pad + 32 * x + tid] = nrm[tid];
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const int tb = 16 * hh + u;  // token within the block
    const float nv = nrm[tb];
    const float uv = nv > 0.f ? y[u] / nv : 0.f;
    const _Float16 hi = (_Float16)uv;
    const _Float16 lo = (_Float16)(uv - (float)hi);
    if (kind == 1) {
      _Float16* p = reinterpret_cast<_Float16*>(a.dk) + ((int64_t)row * a.nd_pad + 32 * x + tb) * 2 * D;
      p[j] = hi;
      p[D + j] = lo;
    } else {
      // k-slot of token tb: tile tb >> 4, key k = tb & 15 -> slot 8 (k >> 2) + 4 (tb >> 4) + (k & 3)
      const int k = tb & 15, slot = 8 * (k >> 2) + 4 * (tb >> 4) + (k & 3);
      _Float16* p = reinterpret_cast<_Float16*>(a.dv) + (((int64_t)row * a.nbd + x) * 2 * D + j) * 32 + slot;
      p[0] = hi;
      p[D * 32] = lo;
    }
  }
}

// The partials kernel. Grid (split, row group, kv row), PW waves; wave w of
// row group y owns rows [(y PW + w) 64, + 64) of the kv row and the blocks
// [split bps, (split + 1) bps) of the kv row's block list (the nbd blocks of
// uncompressed tokens, then the nbc compressed blocks).
template <int KB, int VB>
__global__ __launch_bounds__(PT, 1) void prefill_kernel(PrefillArgs a) {
  using L = PLds<KB, VB>;
  __shared__ __align__(16) uint8_t smem[L::total];
  const int split = blockIdx.x, row = blockIdx.z;
  const int b = row / a.hkv;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 15, q4 = lane >> 4;

  // ---- codebooks, then the pair tables (every wave takes part)
  float* cs = reinterpret_cast<float*>(smem + L::cen);
  if (tid < 16) cs[tid] = tid < (1 << KB) ? a.kcen[tid] : 0.f;
  else if (tid < 32) cs[tid] = tid - 16 < (1 << VB) ? a.vcen[tid - 16] : 0.f;
  __syncthreads();
  pair_table<KB>(smem + L::klut, cs, tid);
  pair_table<VB>(smem + L::vlut, cs + 16, tid);
  __syncthreads();

  const int r0 = (blockIdx.y * PW + w) * WR;  // first query row of the wave
  const int nbt = a.nbd + a.nbc;
  const int blo = split * a.bps, bhi = min(nbt, blo + a.bps);
  if (r0 >= a.nrows || blo >= bhi) return;

  const int cl = clamp_len(a.comp_len, b, a.max_comp);
  const int sl = clamp_len(a.sink_len, b, a.max_sink);
  const int rl = clamp_len(a.res_len, b, a.max_res);
  const int nd = sl + rl, total = nd + cl;
  const int base = total - a.n_q;  // position of query token 0
  int qpos[NT];
#pragma unroll
  for (int rt = 0; rt < NT; ++rt) {
    const int rr = r0 + 16 * rt + j;
    qpos[rt] = rr < a.nrows ? base + rr / a.G : -1;
  }
  const int qlo = base + r0 / a.G;                            // smallest query position of the wave
  const int qhi = base + (min(r0 + WR, a.nrows) - 1) / a.G;  // largest

  // ---- query operands: lane (j, q4) of tile rt, step s holds rotated dims
  // 32 q4 + 8 s .. + 7 of row r0 + 16 rt + j, scaled by 2^e (per wave) so the
  // largest |coordinate| is in [2^13, 2^14)
  u4 qb[NT][4], qbl[NT][4];  // fp16 high parts and remainders
  float qscale;
  {
    // two passes over the rows (the second from cache): the wave's largest
    // |coordinate|, then the fp16 operands
    const float* qr = a.qr + ((int64_t)row * a.nrows_pad + r0) * D + j * D + 32 * q4;
    float qm = 0.f;
#pragma unroll
    for (int rt = 0; rt < NT; ++rt)
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float4 x = *reinterpret_cast<const float4*>(qr + 16 * rt * D + 8 * s + 4 * h);
          qm = fmaxf(qm, fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w))));
        }
    qm = uk::wave_max(qm);
    const int e = qm > 0.f ? 14 - __builtin_amdgcn_frexp_expf(qm) : 0;  // qm 2^e in [2^13, 2^14)
    const float sc = __builtin_amdgcn_ldexpf(1.f, e);
#pragma unroll
    for (int rt = 0; rt < NT; ++rt)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const float4 x0 = *reinterpret_cast<const float4*>(qr + 16 * rt * D + 8 * s);
        const float4 x1 = *reinterpret_cast<const float4*>(qr + 16 * rt * D + 8 * s + 4);
        const float v[8] = {x0.x * sc, x0.y * sc, x0.z * sc, x0.w * sc, x1.x * sc, x1.y * sc, x1.z * sc, x1.w * sc};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t hp = pack_rn(v[2 * k], v[2 * k + 1]);
          const h2 hv = __builtin_bit_cast(h2, hp);
          qb[rt][s][k] = hp;
          qbl[rt][s][k] = pack_rn(v[2 * k] - (float)hv[0], v[2 * k + 1] - (float)hv[1]);
        }
      }
    qscale = a.scale * LOG2E * __builtin_amdgcn_ldexpf(1.f, -e);
  }

  float m_run[NT], l_run[NT];
  f4 acc[NT][8];
#pragma unroll
  for (int rt = 0; rt < NT; ++rt) {
    m_run[rt] = M_INIT;
    l_run[rt] = 0.f;
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) acc[rt][nb] = f4{0.f, 0.f, 0.f, 0.f};
  }
  int vx = 0;
  bool vset = false;

  // LDS addresses of table entries: replica lane & 31
  const uint32_t cp = (uint32_t)(lane & 31) * 4;
  const uint32_t cpk = cp | L::klut;
  float* nst = reinterpret_cast<float*>(smem + L::nst + w * 256);
  f4* rsb = reinterpret_cast<f4*>(smem + L::rsc + w * 2048);
  // acc[rt] *= f, through the wave's LDS area: the accumulators are only
  // stored and reloaded here (the products are formed on loaded copies), so
  // they can stay in the MFMA result registers, which VALU instructions
  // cannot read
  auto scale_tile = [&](int rt, float f) {
#pragma unroll
    for (int h = 0; h < 8; h += 2) {
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) rsb[nb * 64 + lane] = acc[rt][h + nb];
      asm volatile("" ::: "memory");
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const f4 x = rsb[nb * 64 + lane];
        rsb[nb * 64 + lane] = x * f;
      }
      asm volatile("" ::: "memory");
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) acc[rt][h + nb] = rsb[nb * 64 + lane];
    }
  };

  // One block: kop(t, s, hi, lo) gives the key A operands of tile t, step s;
  // vop(nb, hi, lo) the value A operands of PV MFMA nb; nk / nv the norms of
  // the lane's 8 keys (k-slot order); kpos their positions (-1: no token),
  // read only when MASK (a block with tokens past the sequence or past some
  // row's query position).
  auto block = [&](auto kop, auto vop, const float (&nk)[8], const float (&nv)[8], const int (&kpos)[8],
                   auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    f4 sc[2][NT];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int rt = 0; rt < NT; ++rt) sc[t][rt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      u4 kh[2], kl[2];
      kop(0, s, kh[0], kl[0]);
      kop(1, s, kh[1], kl[1]);
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int rt = 0; rt < NT; ++rt) sc[t][rt] = mfma(as_h8(kh[t]), as_h8(qb[rt][s]), sc[t][rt]);
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int rt = 0; rt < NT; ++rt) sc[t][rt] = mfma(as_h8(kl[t]), as_h8(qb[rt][s]), sc[t][rt]);
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int rt = 0; rt < NT; ++rt) sc[t][rt] = mfma(as_h8(kh[t]), as_h8(qbl[rt][s]), sc[t][rt]);
    }
    // value scale: the block's largest n_v is the same for every row
    float nvm = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) nvm = fmaxf(nvm, nv[i]);
    nvm = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(rows_max(nvm))));
    if (!vset) {
      if (nvm > 0.f) {
        vx = max((int)ceilf(log2f(nvm / PV_SET)), -110);
        vset = true;
      }
    } else {
      const float pm = nvm * __builtin_amdgcn_ldexpf(1.f, -vx);
      if (pm > PV_LIMIT) {
        const int dx = (int)ceilf(log2f(pm / PV_LIMIT));
        const float f = __builtin_amdgcn_ldexpf(1.f, -dx);
#pragma unroll
        for (int rt = 0; rt < NT; ++rt) scale_tile(rt, f);
        vx += dx;
      }
    }
    const float down = __builtin_amdgcn_ldexpf(1.f, -vx);
    float ck[8], nvs[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      ck[i] = nk[i] * qscale;
      nvs[i] = nv[i] * down;
    }
    u4 pb[NT];
#pragma unroll
    for (int rt = 0; rt < NT; ++rt) {
      float sv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) sv[i] = fmaf(sc[i >> 2][rt][i & 3], ck[i], -m_run[rt]);
      if constexpr (MASK) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (kpos[i] < 0 || kpos[i] > qpos[rt]) sv[i] = -INFINITY;
      }
      float bm = sv[0];
#pragma unroll
      for (int i = 1; i < 8; ++i) bm = fmaxf(bm, sv[i]);
      if (__builtin_amdgcn_ballot_w64(bm > 0.f) != 0) {
        // a row's max rose: the scores again without the old max, the new max
        // (with the margin) from the row's four lanes
        float tv[8], tm = -INFINITY;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          tv[i] = sv[i] == -INFINITY ? -INFINITY : sc[i >> 2][rt][i & 3] * ck[i];
          tm = fmaxf(tm, tv[i]);
        }
        tm = rows_max(tm);
        const float mnew = tm > m_run[rt] ? tm + MARGIN : m_run[rt];
        const float corr = fexp2(m_run[rt] - mnew);
        l_run[rt] *= corr;
        scale_tile(rt, corr);
        m_run[rt] = mnew;
#pragma unroll
        for (int i = 0; i < 8; ++i) sv[i] = tv[i] - mnew;
      }
      float p[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        p[i] = fexp2(sv[i]);
        l_run[rt] += p[i];
      }
      pb[rt] = u4{pack_rn(p[0] * nvs[0], p[1] * nvs[1]), pack_rn(p[2] * nvs[2], p[3] * nvs[3]),
                  pack_rn(p[4] * nvs[4], p[5] * nvs[5]), pack_rn(p[6] * nvs[6], p[7] * nvs[7])};
    }
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
      u4 vh, vl;
      vop(nb, vh, vl);
#pragma unroll
      for (int rt = 0; rt < NT; ++rt) acc[rt][nb] = mfma(as_h8(vh), as_h8(pb[rt]), acc[rt][nb]);
#pragma unroll
      for (int rt = 0; rt < NT; ++rt) acc[rt][nb] = mfma(as_h8(vl), as_h8(pb[rt]), acc[rt][nb]);
    }
  };
  using masked = std::integral_constant<bool, true>;
  using unmasked = std::integral_constant<bool, false>;

  // position of the lane's key i (k-slot order: tile i >> 2, key 4 q4 + (i & 3))
  auto slot_tok = [&](int i) { return 16 * (i >> 2) + 4 * q4 + (i & 3); };

  // ---- uncompressed tokens: blocks [blo, min(bhi, nbd)), all with the mask
  {
    const _Float16* dk = reinterpret_cast<const _Float16*>(a.dk) + (int64_t)row * a.nd_pad * 2 * D;
    const _Float16* dv = reinterpret_cast<const _Float16*>(a.dv) + (int64_t)row * a.nbd * 2 * D * 32;
    const float* dnk = a.dnk + (int64_t)row * a.nd_pad;
    const float* dnv = a.dnv + (int64_t)row * a.nd_pad;
    for (int db = blo; db < min(bhi, a.nbd); ++db) {
      const int t0 = 32 * db;
      if (t0 >= nd) break;
      auto dpos = [&](int tok) { return tok < sl ? tok : tok + cl; };
      if (dpos(t0) > qhi) break;  // later blocks are later positions
      float nk[8], nv[8];
      int kpos[8];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float4 k4 = *reinterpret_cast<const float4*>(dnk + t0 + 16 * h + 4 * q4);
        const float4 v4 = *reinterpret_cast<const float4*>(dnv + t0 + 16 * h + 4 * q4);
        nk[4 * h] = k4.x; nk[4 * h + 1] = k4.y; nk[4 * h + 2] = k4.z; nk[4 * h + 3] = k4.w;
        nv[4 * h] = v4.x; nv[4 * h + 1] = v4.y; nv[4 * h + 2] = v4.z; nv[4 * h + 3] = v4.w;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int tok = t0 + slot_tok(i);
        kpos[i] = tok < nd ? dpos(tok) : -1;
      }
      auto kop = [&](int t, int s, u4& hi, u4& lo) {
        const _Float16* p = dk + (int64_t)(t0 + 16 * t + j) * 2 * D + 32 * q4 + 8 * s;
        hi = *reinterpret_cast<const u4*>(p);
        lo = *reinterpret_cast<const u4*>(p + D);
      };
      auto vop = [&](int nb, u4& hi, u4& lo) {
        const _Float16* p = dv + ((int64_t)db * 2 * D + 8 * j + nb) * 32 + 8 * q4;
        hi = *reinterpret_cast<const u4*>(p);
        lo = *reinterpret_cast<const u4*>(p + D * 32);
      };
      block(kop, vop, nk, nv, kpos, masked{});
    }
  }

  // ---- compressed blocks [max(blo, nbd), bhi) - nbd, one block's loads in
  // flight while the previous one is computed: first the blocks that need no
  // mask (whole, and before every row's query position), then the others
  const int c0 = max(blo, a.nbd) - a.nbd, c1 = bhi - a.nbd;
  const int ncl = min(c1, (cl + 31) >> 5);  // blocks holding tokens of this sequence
  int cend = ncl;
  // blocks whose first position is past the wave's last query are skipped
  if (c0 < cend) cend = min(cend, max(c0, ((qhi - sl) >> 5) + 1));
  // block cb needs no mask when 32 cb + 32 <= cl and sl + 32 cb + 31 <= qlo
  const int cfree = max(c0, min(cend, min(cl >> 5, qlo - sl - 31 >= 0 ? ((qlo - sl - 31) >> 5) + 1 : 0)));
  if (c0 < cend) {
    constexpr int RK = 16 * KB, RV = 16 * VB;
    const uint8_t* kcodes = a.kc + (int64_t)row * a.k_hs;
    const uint8_t* vcodes = a.vc + (int64_t)row * a.v_hs;
    const float* knorm = a.kn + (int64_t)row * a.kn_hs;
    const float* vnorm = a.vn + (int64_t)row * a.vn_hs;
    // lane byte offsets within a block: key bytes 4 KB q4 .. of token j (tile
    // 1 at + 16 RK); value bits 8 VB j .. of token 4 q4 + i (i < 4) and 16 + 4
    // q4 + i (VB = 3: the dword holding bit 24 j and the next); norm of token
    // lane & 31
    const int ko = j * RK + 4 * KB * q4;
    const int vo = q4 * 4 * RV + (VB == 3 ? 4 * ((3 * j) >> 2) : VB * j);
    const int no = (lane & 31) * 4;
    struct CB {
      u4 k[2];
      uint32_t v[8];
      uint32_t vx[VB == 3 ? 8 : 1];
      float nk, nv;
    };
    auto load = [&](int cb, CB& B) {
      const int t0 = cb << 5;
      const int n = cl - t0;
      const __amdgpu_buffer_rsrc_t rk = rsrc(kcodes + (int64_t)t0 * RK, n * RK);
      const __amdgpu_buffer_rsrc_t rv = rsrc(vcodes + (int64_t)t0 * RV, n * RV);
      const __amdgpu_buffer_rsrc_t rkn = rsrc(knorm + t0, n * 4);
      const __amdgpu_buffer_rsrc_t rvn = rsrc(vnorm + t0, n * 4);
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if constexpr (KB == 4) {
          B.k[t] = __builtin_amdgcn_raw_buffer_load_b128(rk, ko + 16 * RK * t, 0, 0);
        } else if constexpr (KB == 3) {
          const u3 x = __builtin_amdgcn_raw_buffer_load_b96(rk, ko + 16 * RK * t, 0, 0);
          B.k[t] = u4{x[0], x[1], x[2], 0u};
        } else {
          const u2 x = __builtin_amdgcn_raw_buffer_load_b64(rk, ko + 16 * RK * t, 0, 0);
          B.k[t] = u4{x[0], x[1], 0u, 0u};
        }
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int off = vo + (i < 4 ? RV * i : 16 * RV + RV * (i - 4));
        if constexpr (VB == 2) {
          B.v[i] = __builtin_amdgcn_raw_buffer_load_b16(rv, off, 0, 0);
        } else if constexpr (VB == 4) {
          B.v[i] = __builtin_amdgcn_raw_buffer_load_b32(rv, off, 0, 0);
        } else {
          const u2 x = __builtin_amdgcn_raw_buffer_load_b64(rv, off, 0, 0);
          B.v[i] = x[0];
          B.vx[i] = x[1];
        }
      }
      B.nk = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rkn, no, 0, 0));
      B.nv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rvn, no, 0, 0));
    };
    CB cur, nxt;
    load(c0, cur);
    auto run = [&](int from, int to, auto mask_tag) {
      for (int cb = from; cb < to; ++cb) {
        if (cb + 1 < cend) load(cb + 1, nxt);
        const int t0 = cb << 5;
        // norms of the lane's keys through the wave's LDS staging
        nst[lane & 31] = cur.nk;  // lanes l and l + 32 store the same value
        nst[32 + (lane & 31)] = cur.nv;
        __builtin_amdgcn_wave_barrier();
        float nk[8], nv[8];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float4 k4 = *reinterpret_cast<const float4*>(nst + 16 * h + 4 * q4);
          const float4 v4 = *reinterpret_cast<const float4*>(nst + 32 + 16 * h + 4 * q4);
          nk[4 * h] = k4.x; nk[4 * h + 1] = k4.y; nk[4 * h + 2] = k4.z; nk[4 * h + 3] = k4.w;
          nv[4 * h] = v4.x; nv[4 * h + 1] = v4.y; nv[4 * h + 2] = v4.z; nv[4 * h + 3] = v4.w;
        }
        __builtin_amdgcn_wave_barrier();
        int kpos[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int tok = t0 + slot_tok(i);
          kpos[i] = tok < cl ? sl + tok : -1;
        }
        // key entries: pair m of step s = codes 8 s + 2 m, 8 s + 2 m + 1 of the
        // lane's 32 (a byte for 4 bits, a nibble for 2, 6 bits for 3)
        uint32_t kn2[2][4][2];  // KB = 2: the nibbles of each dword spread to bytes (even, odd)
        if constexpr (KB == 2) {
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int d = 0; d < 2; ++d) {
              kn2[t][d][0] = cur.k[t][d] & 0x0F0F0F0Fu;
              kn2[t][d][1] = (cur.k[t][d] >> 4) & 0x0F0F0F0Fu;
            }
        }
        auto kop = [&](int t, int s, u4& hi, u4& lo) {
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            uint32_t addr;
            if constexpr (KB == 4) {
              addr = byte_addr(cur.k[t][s], cpk, m);
            } else if constexpr (KB == 2) {
              const int n = 4 * (s & 1) + m;  // nibble of dword s >> 1
              addr = byte_addr(kn2[t][s >> 1][n & 1], cpk, n >> 1);
            } else {
              constexpr int W = 6;
              const int off = W * (4 * s + m), wd = off >> 5, sh = off & 31;
              const uint32_t xw = sh + W <= 32 ? cur.k[t][wd] >> sh
                                               : __builtin_amdgcn_alignbit(cur.k[t][wd + 1], cur.k[t][wd], sh);
              addr = cpk | ((xw & 63u) << 8);
            }
            entry(smem, addr, hi, lo, m);
          }
        };
        // value entries: dim 8 j + nb of the token pairs (2 m, 2 m + 1); the
        // pair indices of all 8 dims of a token pair first
        uint32_t vp[4][2];
        {
          const uint32_t sh3 = (24u * (uint32_t)j) & 31u;
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            uint32_t wa = cur.v[2 * m], wb = cur.v[2 * m + 1];
            if constexpr (VB == 3) {
              wa = __builtin_amdgcn_alignbit(cur.vx[VB == 3 ? 2 * m : 0], wa, sh3);
              wb = __builtin_amdgcn_alignbit(cur.vx[VB == 3 ? 2 * m + 1 : 0], wb, sh3);
            }
            if constexpr (VB == 4) {
              // byte k: dims 2 k (even word), 2 k + 1 (odd word)
              vp[m][0] = (wa & 0x0F0F0F0Fu) | ((wb << 4) & 0xF0F0F0F0u);
              vp[m][1] = ((wa >> 4) & 0x0F0F0F0Fu) | (wb & 0xF0F0F0F0u);
            } else if constexpr (VB == 2) {
              // nibble k: dim 2 k (k < 4), dim 2 (k - 4) + 1; then spread to bytes
              const uint32_t te = (wa & 0x3333u) | ((wb & 0x3333u) << 2);
              const uint32_t to = ((wa >> 2) & 0x3333u) | (wb & 0xCCCCu);
              const uint32_t x = te | (to << 16);
              vp[m][0] = x & 0x0F0F0F0Fu;
              vp[m][1] = (x >> 4) & 0x0F0F0F0Fu;
            } else {
              vp[m][0] = wa;
              vp[m][1] = wb;
            }
          }
        }
        auto vop = [&](int nb, u4& hi, u4& lo) {
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            uint32_t addr;
            if constexpr (VB == 4) {
              addr = byte_addr(vp[m][nb & 1], cp, nb >> 1);
            } else if constexpr (VB == 2) {
              const int n = (nb & 1) ? 4 + (nb >> 1) : (nb >> 1);
              addr = byte_addr(vp[m][n & 1], cp, n >> 1);
            } else {
              const uint32_t ca = (vp[m][0] >> (3 * nb)) & 7u, cb2 = (vp[m][1] >> (3 * nb)) & 7u;
              addr = cp | ((ca | (cb2 << 3)) << 8);
            }
            entry(smem, L::vlut + addr, hi, lo, m);
          }
        };
        block(kop, vop, nk, nv, kpos, mask_tag);
        if (cb + 1 < cend) cur = nxt;
      }
    };
    run(c0, cfree, unmasked{});
    run(cfree, cend, masked{});
  }

  // ---- partials: row r0 + 16 rt + j, dims 32 q4 + 8 e + nb
  float* pbase = a.part + (((int64_t)split * a.kvrows + row) * a.nrows_pad + r0) * PART;
  const float up = __builtin_amdgcn_ldexpf(1.f, vx);
#pragma unroll
  for (int rt = 0; rt < NT; ++rt) {
    const float lt = rows_sum(l_run[rt]);
    const int rr = r0 + 16 * rt + j;
    if (rr >= a.nrows) continue;
    float* pp = pbase + (16 * rt + j) * PART;
    const float inv = lt > 0.f ? up / lt : 0.f;
    if (q4 == 0) {
      pp[0] = lt > 0.f ? m_run[rt] : -INFINITY;
      pp[1] = lt;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float* o = pp + 4 + 32 * q4 + 8 * e;
      *reinterpret_cast<float4*>(o) = make_float4(acc[rt][0][e] * inv, acc[rt][1][e] * inv, acc[rt][2][e] * inv,
                                                  acc[rt][3][e] * inv);
      *reinterpret_cast<float4*>(o + 4) = make_float4(acc[rt][4][e] * inv, acc[rt][5][e] * inv,
                                                      acc[rt][6][e] * inv, acc[rt][7][e] * inv);
    }
  }
}

// Merge: rows [16 x, 16 x + 16) of kv row blockIdx.y; combines the nsplit
// partials of each row with their softmax weights and applies the inverse
// rotation (out = o R, the value codec's R).
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillArgs a) {
  __shared__ float orot[16][D];
  const int row = blockIdx.y, tid = threadIdx.x, j = tid & 127, hh = tid >> 7;
  const int b = row / a.hkv, g = row % a.hkv;
  const int64_t pstride = (int64_t)a.kvrows * a.nrows_pad * PART;  // between splits
#pragma unroll 1
  for (int u = 0; u < 8; ++u) {
    const int rr = 16 * blockIdx.x + 8 * hh + u;
    float o = 0.f;
    if (rr < a.nrows) {
      const float* pp = a.part + ((int64_t)row * a.nrows_pad + rr) * PART;
      float M = -INFINITY;
      for (int s = 0; s < a.nsplit; ++s) {
        const float* q = pp + s * pstride;
        if (q[1] > 0.f) M = fmaxf(M, q[0]);
      }
      float W = 0.f;
      for (int s = 0; s < a.nsplit; ++s) {
        const float* q = pp + s * pstride;
        if (q[1] > 0.f) {
          const float wgt = q[1] * fexp2(q[0] - M);
          W += wgt;
          o = fmaf(wgt, q[4 + j], o);
        }
      }
      o = W > 0.f ? o / W : 0.f;
    }
    orot[8 * hh + u][j] = o;
  }
  __syncthreads();
  float y[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) y[u] = 0.f;
  for (int i = 0; i < D; ++i) {
    const float r = a.rv[i * D + j];
#pragma unroll
    for (int u = 0; u < 8; ++u) y[u] = fmaf(orot[8 * hh + u][i], r, y[u]);
  }
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int rr = 16 * blockIdx.x + 8 * hh + u;
    if (rr >= a.nrows) break;
    const int qi = rr / a.G, h = rr % a.G;
    a.out[(((int64_t)b * a.hq + g * a.G + h) * a.n_q + qi) * D + j] = y[u];
  }
}

}  // namespace pf
}  // namespace tq
