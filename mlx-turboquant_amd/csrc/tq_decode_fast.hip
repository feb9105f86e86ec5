// Single-launch fused decode attention for K4/V2 TurboQuant caches on gfx950.
//
// One workgroup (8 waves) per (token range, kv head g, sequence b). The
// token range is a run of 32-token blocks of the sequence's
// [compressed | sink | residual] block list; wave w takes every 8th block.
// A wave issues the loads of its first four compressed blocks before any
// set-up work and keeps three blocks in flight while it computes.
//
// Compressed block (rotated space, docs/FUSED_ATTENTION_DESIGN.md:62-67):
//   S^T[h][t] = n_k[t] * sum_j q_rot[h][j] c4[idx[t][j]]       (MFMA 16x16x32 f16)
//     A = q_rot split into fp16 hi/lo (rows = query heads of g),
//     B = keys decoded through an LDS table byte -> (c_hi pair, c_lo pair),
//     three products q_hi*c_hi + q_hi*c_lo + q_lo*c_hi, float32 accumulate.
//   acc_rot[h][j] += sum_t p[h][t] n_v[t] c2[idx[t][j]]        (MFMA 16x16x32 f16)
//     A = p * n_v split hi/lo (rows [hi heads | lo heads]),
//     B = values decoded through an LDS table indexed by two tokens' code
//     nibbles after an in-wave LDS transpose of the 32x32-byte code tile.
// fp16 block (sink / residual, original space): same MFMAs with exact fp16
// keys/values as B and q (hi/lo) as A, accumulated into acc_orig.
// Online softmax in base 2 (scale * log2 e folded into q).
//
// q_rot = q @ R^T and the per-workgroup inverse rotation acc_rot @ R are
// MFMAs too (R and R^T split into fp16 hi/lo; wave w owns output dims
// [16w, 16w+16)). Each workgroup writes (max, sum, out_partial) per query
// head in original space with device-coherent stores; the last workgroup of
// each (b, g) (ticket counter in the workspace, reset by that workgroup)
// merges them (docs/FULL_FUSED_ATTENTION_RESULTS.md:34-40).
//
// Rotated dims are permuted inside the MFMAs: QK lane (col t, group q4) step
// kb holds dims 32*q4 + 8*kb + i; PV N-block nb column n holds dim 8*n + nb.

#include <math.h>

#include "tq_common.h"
#include "tq_decode_fast.h"

namespace tq {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int FD = 128;
constexpr int FW = 8;            // waves per workgroup (FW * 16 == FD)
constexpr int FT = FW * 64;      // threads
constexpr int NCOPY = 16;        // LDS table replicas (lane % NCOPY)
constexpr int VTS = 40;          // halfwords per row of the transposed V tile
constexpr int PS = FAST_PART_FLOATS;  // floats per (head) partial: m, l, out[128], pad
constexpr int MAXWG = 128;       // workgroups per (sequence, kv head)

__device__ inline half8 as_h8(u4 v) { return __builtin_bit_cast(half8, v); }

__device__ inline f4 mfma(half8 a, half8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ inline float max16(float v) {
  v = fmaxf(v, __shfl_xor(v, 1));
  v = fmaxf(v, __shfl_xor(v, 2));
  v = fmaxf(v, __shfl_xor(v, 4));
  v = fmaxf(v, __shfl_xor(v, 8));
  return v;
}

__device__ inline float sum16(float v) {
  v += __shfl_xor(v, 1);
  v += __shfl_xor(v, 2);
  v += __shfl_xor(v, 4);
  v += __shfl_xor(v, 8);
  return v;
}

__device__ inline uint32_t pack_h2(float lo, float hi) {
  const _Float16 a = (_Float16)lo, b = (_Float16)hi;
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// 8 floats -> fp16 hi part and fp16 remainder
__device__ inline void split8(const float4& x0, const float4& x1, half8& hi, half8& lo) {
  const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const _Float16 h = (_Float16)v[i];
    hi[i] = h;
    lo[i] = (_Float16)(v[i] - (float)h);
  }
}

__device__ inline void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ inline float load_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct Layout {
  static constexpr size_t lut_k = 0;
  static constexpr size_t lut_v = lut_k + 256 * NCOPY * 8;
  static constexpr size_t qrs = lut_v + 256 * NCOPY * 8;        // [8][128] f32 rotated q
  static constexpr size_t qsh = qrs + 8 * FD * 4;                // [8][128] f32 scaled q
  static constexpr size_t fin = qsh + 8 * FD * 4;                // [2][8][128] f32 rot / orig
  static constexpr size_t vt = fin + 2 * 8 * FD * 4;             // FW x 16 x VTS u16
  static constexpr size_t pb = vt + FW * 16 * VTS * 2;           // FW x 8 x 32 f32
  static constexpr size_t misc = pb + FW * 8 * 32 * 4;           // scalars, merge tables
  static constexpr size_t total = misc + 4 * 2 * MAXWG * 8 + 1024;
  static constexpr size_t accb_bytes = lut_v + 256 * NCOPY * 8;  // reusable after the loop
};

struct PackedLoad {
  u4 k0, k1, v;
  float nk0, nk1, nv0, nv1;
};

template <int G>
__global__ __launch_bounds__(FT) void fast_decode_kernel(FastArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  uint2* lut_k = reinterpret_cast<uint2*>(smem + Layout::lut_k);
  uint2* lut_v = reinterpret_cast<uint2*>(smem + Layout::lut_v);
  float* qrs = reinterpret_cast<float*>(smem + Layout::qrs);
  float* qsh = reinterpret_cast<float*>(smem + Layout::qsh);
  float* fin = reinterpret_cast<float*>(smem + Layout::fin);
  float* misc = reinterpret_cast<float*>(smem + Layout::misc);

  const int c = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int r = lane & 15, q4 = lane >> 4, cp = lane % NCOPY;
  const int row = b * a.hkv + g;
  const int j0 = 16 * w;  // output-dim tile of this wave for the rotations

  const int comp = a.comp_len_b ? a.comp_len_b[b] : a.max_comp;
  const int sink = a.sink_len_b ? a.sink_len_b[b] : a.max_sink;
  const int res = a.res_len_b ? a.res_len_b[b] : a.max_res;
  const int rstart = a.res_start_b ? a.res_start_b[b] : a.res_start0;
  const int nbc = (comp + 31) >> 5, nbs = (sink + 31) >> 5, nbr = (res + 31) >> 5;
  const int nbt = nbc + nbs + nbr;
  const int blk0 = c * a.bpw, blk1 = min(blk0 + a.bpw, nbt);
  const int blkc = min(blk1, nbc);
  // compressed blocks of this wave: blk0 + w + k*FW, k < npk
  const int npk = blkc > blk0 + w ? (blkc - (blk0 + w) + FW - 1) / FW : 0;
  const bool wg_has_fp16 = blk1 > nbc;

  const uint8_t* kcodes = a.kc + (int64_t)row * a.k_hs;
  const float* knorm = a.kn + (int64_t)row * a.kn_hs;
  const uint8_t* vcodes = a.vc + (int64_t)row * a.v_hs;
  const float* vnorm = a.vn + (int64_t)row * a.vn_hs;

  auto load_packed = [&](int k) {
    PackedLoad L;
    const int t0 = (blk0 + w + k * FW) << 5;
    const int tA = min(t0 + r, comp - 1), tB = min(t0 + 16 + r, comp - 1);
    L.k0 = *reinterpret_cast<const u4*>(kcodes + (int64_t)tA * 64 + 16 * q4);
    L.k1 = *reinterpret_cast<const u4*>(kcodes + (int64_t)tB * 64 + 16 * q4);
    const int tv = min(t0 + (lane >> 1), comp - 1);
    L.v = *reinterpret_cast<const u4*>(vcodes + (int64_t)tv * 32 + 16 * (lane & 1));
    L.nk0 = knorm[tA];
    L.nk1 = knorm[tB];
    L.nv0 = vnorm[tA];
    L.nv1 = vnorm[tB];
    return L;
  };

  // ---- first loads: four compressed blocks, R rows for q_rot, q rows
  PackedLoad r0, r1, r2, r3;
  if (npk > 0) r0 = load_packed(0);
  if (npk > 1) r1 = load_packed(1);
  if (npk > 2) r2 = load_packed(2);
  if (npk > 3) r3 = load_packed(3);
  float4 rq[8];
  {
    const float* rr = a.rot + (int64_t)(j0 + r) * FD + 8 * q4;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      rq[2 * kb] = *reinterpret_cast<const float4*>(rr + 32 * kb);
      rq[2 * kb + 1] = *reinterpret_cast<const float4*>(rr + 32 * kb + 4);
    }
  }
  // q rows (original space) as MFMA A operands: row r = query head
  half8 qo_hi[4], qo_lo[4];
  {
    const int64_t qb = ((int64_t)b * a.hq + g * G + min(r, G - 1)) * FD + 8 * q4;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float v = r < G ? load_elem(a.q, qb + 32 * kb + i, a.q_dtype) : 0.f;
        const _Float16 h = (_Float16)v;
        qo_hi[kb][i] = h;
        qo_lo[kb][i] = (_Float16)(v - (float)h);  // zero for fp16 queries
      }
    }
  }

  // ---- tables: one entry per thread per table, replicated NCOPY times
  {
    float* cen = misc;  // 16 key + 4 value centroids
    if (tid < 20) cen[tid] = tid < 16 ? a.kcen[tid] : a.vcen[tid - 16];
    __syncthreads();
    const int ent = tid & 255;
    const float c0 = cen[ent & 15], c1 = cen[ent >> 4];
    const float h0 = (float)(_Float16)c0, h1 = (float)(_Float16)c1;
    const uint2 ek = make_uint2(pack_h2(c0, c1), pack_h2(c0 - h0, c1 - h1));
    const uint2 ev = make_uint2(pack_h2(cen[16 + (ent & 3)], cen[16 + ((ent >> 4) & 3)]),
                                pack_h2(cen[16 + ((ent >> 2) & 3)], cen[16 + ((ent >> 6) & 3)]));
#pragma unroll
    for (int k = tid >> 8; k < NCOPY; k += FT / 256) {
      lut_k[ent * NCOPY + k] = ek;
      lut_v[ent * NCOPY + k] = ev;
    }
  }
  // ---- q_rot tile: D[h][n] = sum_i q[h][i] R[j0+n][i]   (B[k=i][n] = R[j0+n][i])
  {
    f4 dq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      half8 bh, bl;
      split8(rq[2 * kb], rq[2 * kb + 1], bh, bl);
      dq = mfma(qo_hi[kb], bh, dq);
      dq = mfma(qo_hi[kb], bl, dq);
      dq = mfma(qo_lo[kb], bh, dq);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * q4 + i;
      if (h < G) qrs[h * FD + j0 + r] = dq[i] * a.qscale;
    }
  }
  // fp16 blocks use q * qscale in original space (kept in LDS)
  if (r < G) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int i = 0; i < 8; ++i)
        qsh[r * FD + 32 * kb + 8 * q4 + i] = ((float)qo_hi[kb][i] + (float)qo_lo[kb][i]) * a.qscale;
  }
  __syncthreads();

  // A operands of the rotated-space QK: row r = query head, k slot (q4, i)
  half8 qa_hi[4], qa_lo[4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float v = r < G ? qrs[r * FD + 32 * q4 + 8 * kb + i] : 0.f;
      const _Float16 hv = (_Float16)v;
      qa_hi[kb][i] = hv;
      qa_lo[kb][i] = (_Float16)(v - (float)hv);
    }
  }

  // ---- per-wave online softmax state (rows 4*q4 + i of the S tile)
  float m_i[4], l_i[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) { m_i[i] = -INFINITY; l_i[i] = 0.f; }
  f4 acc_r[8];
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) acc_r[nb] = f4{0.f, 0.f, 0.f, 0.f};

  uint16_t* vt = reinterpret_cast<uint16_t*>(smem + Layout::vt) + w * 16 * VTS;
  float* pb = reinterpret_cast<float*>(smem + Layout::pb) + w * 8 * 32;

  // Online softmax of one 32-token block (scores s0: tokens 0..15, s1: 16..31
  // of the block, rows = query heads): updates (m, l), returns the PV A operand
  // (p * n_v split hi/lo) and the per-row correction of the accumulators.
  auto softmax_block = [&](const f4& s0, const f4& s1, float nv0, float nv1, half8& pa, float (&cr)[4]) {
    float corr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float mb = max16(fmaxf(s0[i], s1[i]));
      const float mn = fmaxf(m_i[i], mb);
      corr[i] = (m_i[i] == -INFINITY) ? 0.f : exp2f(m_i[i] - mn);
      const float p0 = (s0[i] == -INFINITY) ? 0.f : exp2f(s0[i] - mn);
      const float p1 = (s1[i] == -INFINITY) ? 0.f : exp2f(s1[i] - mn);
      l_i[i] = l_i[i] * corr[i] + p0 + p1;
      m_i[i] = mn;
      const int rho = 4 * q4 + i;
      if (rho < G) {
        pb[rho * 32 + r] = p0 * nv0;
        pb[rho * 32 + 16 + r] = p1 * nv1;
      }
    }
    // Row rho = 4*q4 + i of an accumulator belongs to head rho % G; its
    // softmax state lives in lane 16*(head/4), register head % 4, and that
    // register index depends on i only.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int reg = (G >= 4) ? i : (i % G);
      const int rho = 4 * q4 + i;
      const int src = 16 * ((rho % G) >> 2);
      const float v = __int_as_float(__builtin_amdgcn_ds_bpermute(src << 2, __float_as_int(corr[reg])));
      cr[i] = rho < 2 * G ? v : 0.f;
    }
    __builtin_amdgcn_wave_barrier();
    // row r = [p*n_v hi (heads 0..G-1) | lo (heads 0..G-1)], k slot = token 8*q4 + i
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int t = 8 * q4 + i;
      float v = 0.f;
      if (r < G) v = pb[r * 32 + t];
      else if (r < 2 * G) v = pb[(r - G) * 32 + t];
      const _Float16 hv = (_Float16)v;
      pa[i] = (r < G) ? hv : (_Float16)(v - (float)hv);
    }
  };

  // ---- compressed blocks (rotated space); blocks k+1..k+3 stay in flight
  for (int k = 0; k < npk; ++k) {
    const PackedLoad& cur = r0;
    const int t0 = (blk0 + w + k * FW) << 5;
    // stage the value codes transposed: vt[n][t] = halfword n of token t
#pragma unroll
    for (int j = 0; j < 8; ++j)
      vt[(8 * (lane & 1) + j) * VTS + (lane >> 1)] = (uint16_t)(cur.v[j >> 1] >> (16 * (j & 1)));
    f4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const uint32_t w0 = cur.k0[kb], w1 = cur.k1[kb];
      u4 bh0, bl0, bh1, bl1;
#pragma unroll
      for (int byte = 0; byte < 4; ++byte) {
        const uint2 e0 = lut_k[((w0 >> (8 * byte)) & 0xFF) * NCOPY + cp];
        const uint2 e1 = lut_k[((w1 >> (8 * byte)) & 0xFF) * NCOPY + cp];
        bh0[byte] = e0.x; bl0[byte] = e0.y;
        bh1[byte] = e1.x; bl1[byte] = e1.y;
      }
      s0 = mfma(qa_hi[kb], as_h8(bh0), s0);
      s0 = mfma(qa_hi[kb], as_h8(bl0), s0);
      s0 = mfma(qa_lo[kb], as_h8(bh0), s0);
      s1 = mfma(qa_hi[kb], as_h8(bh1), s1);
      s1 = mfma(qa_hi[kb], as_h8(bl1), s1);
      s1 = mfma(qa_lo[kb], as_h8(bh1), s1);
    }
    const bool ok0 = t0 + r < comp, ok1 = t0 + 16 + r < comp;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s0[i] = ok0 ? s0[i] * cur.nk0 : -INFINITY;
      s1[i] = ok1 ? s1[i] * cur.nk1 : -INFINITY;
    }
    half8 pa;
    float cr[4];
    softmax_block(s0, s1, cur.nv0, cur.nv1, pa, cr);
#pragma unroll
    for (int nb = 0; nb < 8; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc_r[nb][i] *= cr[i];
    const u4 vw = *reinterpret_cast<const u4*>(vt + r * VTS + 8 * q4);
    u4 bv[8];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const uint32_t idx = ((vw[kk] >> (4 * p)) & 0xF) | (((vw[kk] >> (16 + 4 * p)) & 0xF) << 4);
        const uint2 e = lut_v[idx * NCOPY + cp];
        bv[2 * p][kk] = e.x;
        bv[2 * p + 1][kk] = e.y;
      }
    }
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) acc_r[nb] = mfma(pa, as_h8(bv[nb]), acc_r[nb]);
    __builtin_amdgcn_wave_barrier();
    r0 = r1;
    r1 = r2;
    r2 = r3;
    if (k + 4 < npk) r3 = load_packed(k + 4);
  }

  // ---- fp16 blocks of the sink and the residual ring (original space)
  f4 acc_o[8];
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) acc_o[nb] = f4{0.f, 0.f, 0.f, 0.f};
  for (int blk = blk0 + w + npk * FW; blk < blk1; blk += FW) {
    const bool is_sink = blk < nbc + nbs;
    const int ft0 = (is_sink ? blk - nbc : blk - nbc - nbs) << 5;
    const int flen = is_sink ? sink : res;
    const int64_t hs = is_sink ? a.sink_hs : a.res_hs;
    const uint16_t* fk = static_cast<const uint16_t*>(is_sink ? a.sink_k : a.res_k) + (int64_t)row * hs;
    const uint16_t* fv = static_cast<const uint16_t*>(is_sink ? a.sink_v : a.res_v) + (int64_t)row * hs;
    auto slot = [&](int t) {
      t = min(t, flen - 1);
      return is_sink ? t : (rstart + t) % a.res_cap;
    };
    const u4* kA = reinterpret_cast<const u4*>(fk + (int64_t)slot(ft0 + r) * FD + 32 * q4);
    const u4* kB = reinterpret_cast<const u4*>(fk + (int64_t)slot(ft0 + 16 + r) * FD + 32 * q4);
    f4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      half8 qh, ql;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float v = r < G ? qsh[r * FD + 32 * q4 + 8 * kb + i] : 0.f;
        const _Float16 hv = (_Float16)v;
        qh[i] = hv;
        ql[i] = (_Float16)(v - (float)hv);
      }
      const half8 ba = as_h8(kA[kb]), bb = as_h8(kB[kb]);
      s0 = mfma(qh, ba, s0);
      s0 = mfma(ql, ba, s0);
      s1 = mfma(qh, bb, s1);
      s1 = mfma(ql, bb, s1);
    }
    const bool ok0 = ft0 + r < flen, ok1 = ft0 + 16 + r < flen;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (!ok0) s0[i] = -INFINITY;
      if (!ok1) s1[i] = -INFINITY;
    }
    half8 pa;
    float cr[4];
    softmax_block(s0, s1, 1.f, 1.f, pa, cr);
#pragma unroll
    for (int nb = 0; nb < 8; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i) { acc_r[nb][i] *= cr[i]; acc_o[nb][i] *= cr[i]; }
    // B = V rows: lane (n = r, q4) needs dims 8n..8n+7 of tokens 8*q4 + i
    u4 vr[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) vr[i] = *reinterpret_cast<const u4*>(fv + (int64_t)slot(ft0 + 8 * q4 + i) * FD + 8 * r);
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
      const uint32_t sel = (nb & 1) ? 0x07060302u : 0x05040100u;
      u4 bvv;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        bvv[kk] = __builtin_amdgcn_perm(vr[2 * kk + 1][nb >> 1], vr[2 * kk][nb >> 1], sel);
      acc_o[nb] = mfma(pa, as_h8(bvv), acc_o[nb]);
    }
    __builtin_amdgcn_wave_barrier();
  }

  // ---- R^T rows of this wave for the inverse rotation (latency overlaps the combine)
  float4 rt[8];
  {
    const float* tr = a.rot_t + (int64_t)(j0 + r) * FD + 8 * q4;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      rt[2 * kb] = *reinterpret_cast<const float4*>(tr + 32 * kb);
      rt[2 * kb + 1] = *reinterpret_cast<const float4*>(tr + 32 * kb + 4);
    }
  }

  // ---- combine the 8 waves of this workgroup
#pragma unroll
  for (int i = 0; i < 4; ++i) l_i[i] = sum16(l_i[i]);
  float* wm = misc;            // [FW][8]
  float* wl = misc + FW * 8;   // [FW][8]
  float* hM = misc + 2 * FW * 8;
  float* hL = hM + 8;
  int* flag = reinterpret_cast<int*>(hL + 8);
  float* pm = misc + 2 * FW * 8 + 32;  // [MAXWG * 8] merge tables
  float* pl = pm + MAXWG * 8;
  // accumulators of every wave (unscaled) into LDS, reusing the table space
  constexpr int SIDE = FW * 2 * G * FD;                         // floats per side
  constexpr bool ONE_PASS = 2 * SIDE * 4 <= (int)Layout::accb_bytes;
  float* accb = reinterpret_cast<float*>(smem);
  __syncthreads();  // every wave is done with the tables
  if (r == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rho = 4 * q4 + i;
      if (rho < G) { wm[w * 8 + rho] = m_i[i]; wl[w * 8 + rho] = l_i[i]; }
    }
  }
  const int nside = wg_has_fp16 ? 2 : 1;
  for (int side = 0; side < nside; ++side) {
    float* dst = accb + (ONE_PASS ? side * SIDE : 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rho = 4 * q4 + i;
      if (rho < 2 * G) {
#pragma unroll
        for (int nb = 0; nb < 8; ++nb)
          dst[(w * 2 * G + rho) * FD + 8 * r + nb] = side == 0 ? acc_r[nb][i] : acc_o[nb][i];
      }
    }
    __syncthreads();
    for (int e = tid; e < G * FD; e += FT) {
      const int h = e / FD, j = e % FD;
      float M = -INFINITY;
#pragma unroll
      for (int ww = 0; ww < FW; ++ww) M = fmaxf(M, wm[ww * 8 + h]);
      float s = 0.f, L = 0.f;
#pragma unroll
      for (int ww = 0; ww < FW; ++ww) {
        const float mw = wm[ww * 8 + h];
        const float sc = mw > -INFINITY ? exp2f(mw - M) : 0.f;
        s = fmaf(sc, dst[(ww * 2 * G + h) * FD + j] + dst[(ww * 2 * G + G + h) * FD + j], s);
        L = fmaf(sc, wl[ww * 8 + h], L);
      }
      fin[side * 8 * FD + e] = s;
      if (side == 0 && j == 0) { hM[h] = M; hL[h] = L; }
    }
    __syncthreads();
  }
  // ---- partial in original space: out = rot @ R + orig  (B[k=i][n] = R[i][j0+n] = R^T[j0+n][i])
  float* part = a.part + ((int64_t)row * a.nwg + c) * G * PS;
  {
    f4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      half8 ar;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int hh = r < G ? r : r - G;
        const float v = r < 2 * G ? fin[hh * FD + 32 * kb + 8 * q4 + i] : 0.f;
        const _Float16 hv = (_Float16)v;
        ar[i] = r < G ? hv : (_Float16)(v - (float)hv);
      }
      half8 bh, bl;
      split8(rt[2 * kb], rt[2 * kb + 1], bh, bl);
      d = mfma(ar, bh, d);
      d = mfma(ar, bl, d);
    }
    // row h (hi part) + row G + h (lo part): same lane for G < 4, lane + 16*(G/4) otherwise
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float lo;
      if (G >= 4) {
        lo = __shfl_down(d[i], 16 * (G / 4));
      } else {
        lo = (i + G < 4) ? d[(i + G) & 3] : 0.f;
      }
      const int h = 4 * q4 + i;
      if (h < G) {
        const float o = wg_has_fp16 ? fin[8 * FD + h * FD + j0 + r] : 0.f;
        store_coherent(part + h * PS + 2 + j0 + r, d[i] + lo + o);
      }
    }
    if (tid < G) {
      store_coherent(part + tid * PS + 0, hM[tid]);
      store_coherent(part + tid * PS + 1, hL[tid]);
    }
  }

  // ---- last workgroup of (b, g) merges all partials
  // Every thread waits until its device-coherent stores have completed
  // (s_waitcnt vmcnt(0): gfx9 counts stores in vmcnt) before the ticket; the
  // partials were written write-through (sc1), so no L2 writeback is needed.
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __syncthreads();
  if (tid == 0) {
    const int old = __hip_atomic_fetch_add(a.counter + row, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = (old == a.nwg - 1) ? 1 : 0;
  }
  __syncthreads();
  if (*flag == 0) return;
  const float* pall = a.part + (int64_t)row * a.nwg * G * PS;
  for (int e = tid; e < a.nwg * G; e += FT) {
    pm[e] = load_coherent(pall + e * PS);
    pl[e] = load_coherent(pall + e * PS + 1);
  }
  __syncthreads();
  if (tid < G) {
    float M = -INFINITY;
    for (int cc = 0; cc < a.nwg; ++cc) M = fmaxf(M, pm[cc * G + tid]);
    float L = 0.f;
    for (int cc = 0; cc < a.nwg; ++cc)
      if (pm[cc * G + tid] > -INFINITY) L += exp2f(pm[cc * G + tid] - M) * pl[cc * G + tid];
    hM[tid] = M;
    hL[tid] = L;
  }
  __syncthreads();
  for (int e = tid; e < a.nwg * G; e += FT) {
    const int h = e % G;
    pm[e] = pm[e] > -INFINITY ? exp2f(pm[e] - hM[h]) : 0.f;
  }
  __syncthreads();
  for (int e = tid; e < G * FD; e += FT) {
    const int h = e / FD, j = e % FD;
    float o = 0.f;
    int cc = 0;
    for (; cc + 16 <= a.nwg; cc += 16) {
      float v[16];
#pragma unroll
      for (int k = 0; k < 16; ++k) v[k] = load_coherent(pall + ((cc + k) * G + h) * PS + 2 + j);
#pragma unroll
      for (int k = 0; k < 16; ++k) o = fmaf(pm[(cc + k) * G + h], v[k], o);
    }
    for (; cc < a.nwg; ++cc) o = fmaf(pm[cc * G + h], load_coherent(pall + (cc * G + h) * PS + 2 + j), o);
    const float L = hL[h];
    a.out[((int64_t)b * a.hq + g * G + h) * FD + j] = L > 0.f ? o / L : 0.f;
  }
  if (tid == 0) __hip_atomic_store(a.counter + row, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

size_t fast_smem_bytes() { return Layout::total; }

int fast_max_wg() { return MAXWG; }

int launch_fast_decode(const FastArgs& a, int G, int batch, hipStream_t s) {
  dim3 grid(a.nwg, a.hkv, batch);
  const size_t smem = Layout::total;
  switch (G) {
    case 1: hipLaunchKernelGGL((fast_decode_kernel<1>), grid, dim3(FT), smem, s, a); break;
    case 2: hipLaunchKernelGGL((fast_decode_kernel<2>), grid, dim3(FT), smem, s, a); break;
    case 4: hipLaunchKernelGGL((fast_decode_kernel<4>), grid, dim3(FT), smem, s, a); break;
    default: hipLaunchKernelGGL((fast_decode_kernel<8>), grid, dim3(FT), smem, s, a); break;
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int fast_set_attributes() {
  static int done = 0;
  if (done) return 0;
  const int bytes = (int)Layout::total;
  hipError_t e = hipSuccess;
  e = hipFuncSetAttribute((const void*)fast_decode_kernel<1>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess) e = hipFuncSetAttribute((const void*)fast_decode_kernel<2>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess) e = hipFuncSetAttribute((const void*)fast_decode_kernel<4>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess) e = hipFuncSetAttribute((const void*)fast_decode_kernel<8>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e != hipSuccess) return -1;
  done = 1;
  return 0;
}

}  // namespace tq
