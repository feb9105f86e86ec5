// Single-launch fused decode attention for K4/V2 TurboQuant caches on gfx950.
//
// One workgroup (8 waves) per (token range, kv head g, sequence b). The token
// range is a run of 32-token blocks of the sequence's [compressed | sink |
// residual] block list; wave w takes every 8th block and keeps the loads of
// the next compressed block in flight while it computes one.
//
// Scores are computed transposed, S^T = K q^T (MFMA 16x16x32 f16):
//   A = 16 tokens x 32 k-slots of keys, B = 32 k-slots x 16 columns of queries.
// Column r of B holds query head (r % G) of kv group g, either its fp16 high
// part (even r / G) or the fp16 remainder (odd r / G), so a DPP row rotation
// by G adds the two halves and every column ends up with the full score of
// its head. In rotated space (compressed tokens, docs/FUSED_ATTENTION_DESIGN.md
// :62-67) each key code byte (two 4-bit codes) is looked up in an LDS table
// whose 8-byte entry is (c_hi[a], c_hi[b], c_lo[a], c_lo[b]); two lookups fill
// one A operand, and the matching B k-slots repeat the two query values, so
//   sum_k A B = sum_d (c_hi + c_lo)[idx_d] q_d   with c_lo = c - fp16(c).
// Scaled by the key norm and run through an online softmax in base 2.
// Output, transposed too: O^T += V^T P^T with A = 16 dims x 32 tokens of
// values decoded from an LDS table indexed by one 2-bit-code byte (4 dims of
// one token) and paired across tokens with v_perm, and B = p * n_v split into
// fp16 high part / remainder along the same columns as the scores.
// fp16 blocks (sink / residual ring, original space) use the same MFMAs with
// exact fp16 keys / values, accumulated separately.
//
// Lane (column r, group q4) of a score tile holds tokens 4*q4 + i of the
// tile, which is exactly the k-slot order (8*q4 + i) the P^T operand needs,
// so softmax weights never leave their lane. The accumulator of lane
// (column r, q4), MFMA nb, register i is rotated dim 32*q4 + 8*i + nb.
//
// The 8 waves of a workgroup are combined through LDS; each workgroup then
// writes (max, sum, rotated partial, original-space partial) per query head,
// and a second, small kernel on the same stream merges the partials of each
// (b, g) and applies the inverse rotation (docs/FULL_FUSED_ATTENTION_RESULTS.md
// :34-40). The kernel boundary orders the two; no device-scope handshake.

#include <math.h>

#include <type_traits>

#include "tq_common.h"
#include "tq_decode_fast.h"

namespace tq {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef __fp16 hx2 __attribute__((ext_vector_type(2)));

constexpr int FD = 128;
constexpr int FW = FAST_WAVES;        // waves per workgroup (FW * 16 == FD)
constexpr int FT = FW * 64;           // threads
constexpr int PS = FAST_PART_FLOATS;  // floats per (workgroup, head) partial
constexpr int P_ROT = 4;              // partial: [M, L, has_orig, pad, rot[128], orig[128]]
constexpr int P_ORIG = 4 + FD;
constexpr int MAXWG = 128;            // workgroups per (sequence, kv head)
constexpr float M_INIT = -1e30f;      // running max before the first block
constexpr int NCP = 16;               // table replicas per entry (lane % 16)

struct Layout {
  // tables: entry e of both tables in one 256-byte row, key copies in bytes
  // [0, 128), value copies in [128, 256), copy c at 8*c
  static constexpr uint32_t lut = 0;          // 256 rows x 256 B
  static constexpr uint32_t cmb = 65536;      // [8 waves][8 heads][2][128] f32 wave partials
  static constexpr uint32_t cml = cmb + 65536;  // [8 waves][8 heads][4] f32 max, sum, max of the orig part
  static constexpr uint32_t qop = cml + 1024; // [8 heads][2 parts][4][8][8] fp16 rotated-q B operands
  static constexpr uint32_t qfo = qop + 8192; // [8 heads][2 parts][4][4][8] fp16 original-space q B operands
  static constexpr uint32_t total = qfo + 4096;
};

__device__ inline half8 as_h8(u4 v) { return __builtin_bit_cast(half8, v); }

__device__ inline f4 mfma(half8 a, half8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ inline float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }

// value of lane (i - n) mod 16 of the same 16-lane row
template <int N>
__device__ inline float row_ror(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x120 + N, 0xF, 0xF, true));
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

__device__ inline uint32_t pk_rtz(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
}

__device__ inline uint32_t pack_h2(float lo, float hi) {
  const _Float16 a = (_Float16)lo, b = (_Float16)hi;
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// 8 floats -> fp16 high part and fp16 remainder
__device__ inline void split8(const float4& x0, const float4& x1, half8& hi, half8& lo) {
  const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const _Float16 h = (_Float16)v[i];
    hi[i] = h;
    lo[i] = (_Float16)(v[i] - (float)h);
  }
}

__device__ inline u2 lds_u2(const uint8_t* smem, uint32_t addr) {
  return *reinterpret_cast<const u2*>(smem + addr);
}

// loads of one compressed 32-token block (lane r, q4)
struct Blk {
  u4 k0, k1;            // key codes of tokens t0 + r and t0 + 16 + r, bytes 16*q4 ..
  uint32_t v[8];        // value code halfword r of tokens A0..A3, B0..B3 (zero-extended)
  float4 nkA, nkB;      // key norms of tokens t0 + 4q4 + i, t0 + 16 + 4q4 + i
  float4 nvA, nvB;      // value norms of the same tokens
};

template <int G>
__global__ __launch_bounds__(FT) void fast_decode_kernel(FastArgs a) {
  __shared__ __align__(16) uint8_t smem[Layout::total];

  const int c = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, q4 = lane >> 4;
  const int row = b * a.hkv + g;
  const int j0 = 16 * w;  // output-dim tile of this wave for the rotations
  const int hd = r % G;   // query head of column r
  const float partf = ((r / G) & 1) ? 1.f : 0.f;  // column holds the fp16 remainder

  // All kernel arguments the set-up needs are loaded in one batch of scalar
  // loads and waited for once (a branch on an argument would otherwise split
  // them into dependent round trips).
  {
    const void* p0 = a.comp_len_b; const void* p1 = a.sink_len_b;
    const void* p2 = a.res_len_b; const void* p3 = a.res_start_b;
    const void* p4 = a.kc; const void* p5 = a.kn; const void* p6 = a.vc; const void* p7 = a.vn;
    const void* p8 = a.q; const void* p9 = a.rot16; const void* p10 = a.kcen; const void* p11 = a.vcen;
    const int64_t s0 = a.k_hs, s1 = a.kn_hs, s2 = a.v_hs, s3 = a.vn_hs;
    const int i0 = a.max_comp, i1 = a.max_sink, i2 = a.max_res, i3 = a.res_start0, i4 = a.bpw, i5 = a.hkv,
              i6 = a.hq, i7 = a.q_dtype;
    asm volatile("" ::"s"(p0), "s"(p1), "s"(p2), "s"(p3), "s"(p4), "s"(p5), "s"(p6), "s"(p7), "s"(p8), "s"(p9),
                 "s"(p10), "s"(p11), "s"(s0), "s"(s1), "s"(s2), "s"(s3), "s"(i0), "s"(i1), "s"(i2), "s"(i3), "s"(i4),
                 "s"(i5), "s"(i6), "s"(i7));
  }
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

  const uint8_t* kcodes = a.kc + (int64_t)row * a.k_hs;
  const float* knorm = a.kn + (int64_t)row * a.kn_hs;
  const uint8_t* vcodes = a.vc + (int64_t)row * a.v_hs;
  const float* vnorm = a.vn + (int64_t)row * a.vn_hs;

  // ---- first loads: centroids, R rows and q (needed first), then two blocks
  // table centroids: waves 0-3 build the key table (two 4-bit codes per
  // entry), waves 4-7 the value table (four 2-bit codes per entry); each lane
  // loads one centroid, the entries gather theirs with lane shuffles
  const float cen_lane = (w < 4 ? a.kcen : a.vcen)[lane & (w < 4 ? 15 : 3)];
  // R rows j0 + n as MFMA B operands (k-slot (q4, i) of step kb = dim 32*kb + 8*q4 + i),
  // fp16 high part and remainder precomputed by the codec
  u4 rqh[4], rql[4];
  {
    const uint16_t* rh = a.rot16 + (j0 + r) * FD + 8 * q4;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      rqh[kb] = *reinterpret_cast<const u4*>(rh + 32 * kb);
      rql[kb] = *reinterpret_cast<const u4*>(rh + FD * FD + 32 * kb);
    }
  }
  // q rows (original space): raw 16-byte pieces now, converted after the block
  // loads; for 2-byte types the second piece repeats the first (stays in bounds)
  u4 qraw[8];
  {
    const int64_t qb = ((int64_t)b * a.hq + g * G + min(r, G - 1)) * FD + 8 * q4;
    const int esz = a.q_dtype == TQ_F32 ? 4 : 2;
    const uint8_t* p = static_cast<const uint8_t*>(a.q) + qb * esz;
    const int second = a.q_dtype == TQ_F32 ? 16 : 0;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      qraw[2 * kb] = *reinterpret_cast<const u4*>(p + 32 * kb * esz);
      qraw[2 * kb + 1] = *reinterpret_cast<const u4*>(p + 32 * kb * esz + second);
    }
  }
  // lane offsets (32-bit) from the uniform per-block bases
  const uint32_t koff = (uint32_t)(r * 64 + 16 * q4);        // key row t0 + r, bytes 16*q4 ..
  const uint32_t voff = (uint32_t)(4 * q4 * 32 + 2 * r);     // value row t0 + 4*q4, halfword r
  const uint32_t noff = (uint32_t)(4 * q4);                  // norm of token t0 + 4*q4
  // full compressed blocks of this wave come first; at most one partial block follows
  const int nfull = comp >> 5;
  const int npf = min(npk, nfull > blk0 + w ? (nfull - (blk0 + w) + FW - 1) / FW : 0);
  // Full block k of this wave. Loads are issued unconditionally so the wait
  // counts stay exact: k >= npf reads one line (zero lane offsets) of block 0,
  // or of the rotation matrix when the wave has no full block.
  const uint8_t* kbase = npf > 0 ? kcodes : reinterpret_cast<const uint8_t*>(a.rot);
  const uint8_t* vbase = npf > 0 ? vcodes : reinterpret_cast<const uint8_t*>(a.rot);
  const float* knbase = npf > 0 ? knorm : a.rot;
  const float* vnbase = npf > 0 ? vnorm : a.rot;
  auto load_blk = [&](int k) {
    Blk L;
    const bool valid = k < npf;
    const int t0 = valid ? (blk0 + w + k * FW) << 5 : (npf > 0 ? (blk0 + w) << 5 : 0);
    const uint32_t msk = valid ? 0xFFFFFFFFu : 0u;
    const uint8_t* kb = kbase + (int64_t)t0 * 64;
    const uint8_t* vb = vbase + (int64_t)t0 * 32;
    const float* nkb = knbase + t0;
    const float* nvb = vnbase + t0;
    const uint32_t ko = koff & msk, vo = voff & msk, no = noff & msk;
    L.k0 = *reinterpret_cast<const u4*>(kb + ko);
    L.k1 = *reinterpret_cast<const u4*>(kb + ko + 16 * 64);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      L.v[i] = *reinterpret_cast<const uint16_t*>(vb + vo + (uint32_t)(((i >> 2) * 16 + (i & 3)) * 32));
    L.nkA = *reinterpret_cast<const float4*>(nkb + no);
    L.nkB = *reinterpret_cast<const float4*>(nkb + no + 16);
    L.nvA = *reinterpret_cast<const float4*>(nvb + no);
    L.nvB = *reinterpret_cast<const float4*>(nvb + no + 16);
    return L;
  };
  // the sequence's last, partial block: every token clamped to the sequence
  auto load_tail = [&](int k) {
    Blk L;
    const int t0 = (blk0 + w + k * FW) << 5;
    const int lim = comp - 1;
    const int ta = t0 + 4 * q4, tb = t0 + 16 + 4 * q4;
    const uint8_t* vb = vcodes + 2 * r;
    L.k0 = *reinterpret_cast<const u4*>(kcodes + (int64_t)min(t0 + r, lim) * 64 + 16 * q4);
    L.k1 = *reinterpret_cast<const u4*>(kcodes + (int64_t)min(t0 + 16 + r, lim) * 64 + 16 * q4);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      L.v[i] = *reinterpret_cast<const uint16_t*>(vb + (int64_t)min((i < 4 ? ta : tb) + (i & 3), lim) * 32);
    float na[4], nb[4], va[4], vb4[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      na[i] = knorm[min(ta + i, lim)];
      nb[i] = knorm[min(tb + i, lim)];
      va[i] = vnorm[min(ta + i, lim)];
      vb4[i] = vnorm[min(tb + i, lim)];
    }
    L.nkA = make_float4(na[0], na[1], na[2], na[3]);
    L.nkB = make_float4(nb[0], nb[1], nb[2], nb[3]);
    L.nvA = make_float4(va[0], va[1], va[2], va[3]);
    L.nvB = make_float4(vb4[0], vb4[1], vb4[2], vb4[3]);
    return L;
  };
  // One block per wave goes out before the set-up work; one block in flight
  // per wave already covers HBM latency at full bandwidth, and deeper queues
  // stall the issuing wave.
  Blk b0 = load_blk(0);

  // fp16 (sink / residual ring, original space) blocks of this wave follow its
  // compressed ones in the block list but are processed first; the loads of
  // the first one go out now. Loads stay unconditional: a wave without fp16
  // blocks reads one line of the rotation operands instead.
  const int fblk = blk0 + w + npk * FW;
  const bool wave_has_fp16 = fblk < blk1;
  struct F16Blk {
    u4 kA[4], kB[4];  // keys: tokens ft0 + r / ft0 + 16 + r, dims 32*q4 + 8*kb ..
    u4 v[8];          // values: dims 8r .. 8r+7 of tokens A0..A3, B0..B3
  };
  auto load_f16 = [&](int blk, bool valid) {
    F16Blk L;
    const bool is_sink = blk < nbc + nbs;
    const int ft0 = (is_sink ? blk - nbc : blk - nbc - nbs) << 5;
    const int flen = max(is_sink ? sink : res, 1);
    const int64_t hs = is_sink ? a.sink_hs : a.res_hs;
    const uint16_t* fk = valid ? static_cast<const uint16_t*>(is_sink ? a.sink_k : a.res_k) + (int64_t)row * hs : a.rot16;
    const uint16_t* fv = valid ? static_cast<const uint16_t*>(is_sink ? a.sink_v : a.res_v) + (int64_t)row * hs : a.rot16;
    auto slot = [&](int t) {  // ring position of token t (rstart + t < 2 * res_cap)
      t = min(t, flen - 1);
      const int sl = rstart + t;
      return is_sink ? t : (sl >= a.res_cap ? sl - a.res_cap : sl);
    };
    const uint32_t msk = valid ? 0xFFFFFFFFu : 0u;
    const uint32_t oA = ((uint32_t)slot(ft0 + r) * FD + 32 * q4) & msk;
    const uint32_t oB = ((uint32_t)slot(ft0 + 16 + r) * FD + 32 * q4) & msk;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      L.kA[kb] = *reinterpret_cast<const u4*>(fk + oA + 8 * (kb & (int)msk));
      L.kB[kb] = *reinterpret_cast<const u4*>(fk + oB + 8 * (kb & (int)msk));
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int t = ft0 + (i < 4 ? 4 * q4 + i : 16 + 4 * q4 + i - 4);
      L.v[i] = *reinterpret_cast<const u4*>(fv + (((uint32_t)slot(t) * FD + 8 * r) & msk));
    }
    return L;
  };

  // ---- tables, 16 replicas (lane % 16) per entry, entry stride 256 bytes:
  // key byte e -> (c_hi[e&15], c_hi[e>>4], c_lo[e&15], c_lo[e>>4]) fp16
  // value byte e -> (c[e&3], c[(e>>2)&3], c[(e>>4)&3], c[(e>>6)&3]) fp16
  {
    const int e = tid & 255;
    float cen[4];
    const int sh = w < 4 ? 4 : 2, mk = w < 4 ? 15 : 3;
#pragma unroll
    for (int i = 0; i < 4; ++i) cen[i] = __shfl(cen_lane, (e >> (sh * i)) & mk);
    const float h0 = (float)(_Float16)cen[0], h1 = (float)(_Float16)cen[1];
    u4 ent;
    ent[0] = pack_h2(cen[0], cen[1]);
    ent[1] = w < 4 ? pack_h2(cen[0] - h0, cen[1] - h1) : pack_h2(cen[2], cen[3]);
    ent[2] = ent[0];
    ent[3] = ent[1];
    uint8_t* base = smem + Layout::lut + e * 256 + (w < 4 ? 0 : 128);
#pragma unroll
    for (int k = 0; k < NCP / 2; ++k)  // copies (2k', 2k'+1), rotated per entry against bank conflicts
      *reinterpret_cast<u4*>(base + 16 * ((k + e) & (NCP / 2 - 1))) = ent;
  }
  // q rows as MFMA A operands (row r = query head): fp16 high part and remainder
  half8 qo_hi[4], qo_lo[4];
  if (a.q_dtype == TQ_F16) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      qo_hi[kb] = as_h8(qraw[2 * kb]);
      qo_lo[kb] = half8{};
    }
  } else {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t hw = (qraw[2 * kb][i >> 1] >> (16 * (i & 1))) & 0xFFFF;
        const float x = a.q_dtype == TQ_F32 ? __uint_as_float(qraw[2 * kb + (i >> 2)][i & 3]) : __uint_as_float(hw << 16);
        const _Float16 hx = (_Float16)x;
        qo_hi[kb][i] = hx;
        qo_lo[kb][i] = (_Float16)(x - (float)hx);
      }
    }
  }
  // ---- q_rot tile: D[h][n] = sum_i q[h][i] R[j0+n][i]   (B[k=i][n] = R[j0+n][i]),
  // written (times qscale) as fp16 high part / remainder straight into the
  // score B-operand layout [head][part][q4][s][8 halves]: dim j = 32*q4 + 4*s + e
  // sits at halves (e & 1) + 4*(e >> 1) and + 2 (see the operand layout below)
  {
    f4 dq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      dq = mfma(qo_hi[kb], as_h8(rqh[kb]), dq);
      dq = mfma(qo_hi[kb], as_h8(rql[kb]), dq);
      dq = mfma(qo_lo[kb], as_h8(rqh[kb]), dq);
    }
    const int j = j0 + r, e = j & 3;
    const uint32_t off = ((uint32_t)(j >> 5) * 8 + ((j >> 2) & 7)) * 16 + 2 * ((e & 1) + 4 * (e >> 1));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * q4 + i;
      if (h < G) {
        const float v = dq[i] * a.qscale;
        const _Float16 hi = (_Float16)v, lo = (_Float16)(v - (float)hi);
        uint8_t* dh = smem + Layout::qop + (uint32_t)(h * 2) * 512 + off;
        *reinterpret_cast<_Float16*>(dh) = hi;
        *reinterpret_cast<_Float16*>(dh + 4) = hi;
        *reinterpret_cast<_Float16*>(dh + 512) = lo;
        *reinterpret_cast<_Float16*>(dh + 516) = lo;
      }
    }
  }
  // fp16 blocks use the (unscaled) q in original space as score B operands,
  // step kb k-slot (q4, i) = dim 32*q4 + 8*kb + i: fp16 high part / remainder
  // in [head][part][q4][kb][8 halves]; the lane holding dims 32*kb + 8*q4 ..
  // of head r copies its operand halves there (wave 0, workgroups with fp16 blocks)
  if (w == 0 && r < G && blk1 > nbc) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      uint8_t* d = smem + Layout::qfo + ((uint32_t)(r * 2 * 4 + kb) * 4 + q4) * 16;
      *reinterpret_cast<half8*>(d) = qo_hi[kb];
      *reinterpret_cast<half8*>(d + 4 * 4 * 16) = qo_lo[kb];
    }
  }
  // the first fp16 block's loads go out before the barrier (the rest of the
  // set-up has waited for its own loads already)
  F16Blk f0 = load_f16(fblk, wave_has_fp16);
  __syncthreads();

  // ---- per-lane online softmax state of column r (head hd)
  float m_run = M_INIT, l_run = 0.f;
  float m_orig = M_INIT;  // running max the stored original-space partial refers to
  half8 qop[8];           // rotated-space score B operands (set after the fp16 blocks)
  f4 acc_r[8];            // rotated-space output accumulators
  float* cm = reinterpret_cast<float*>(smem + Layout::cmb) + (w * 8) * 2 * FD;  // [head][side][128]
  float* cl = reinterpret_cast<float*>(smem + Layout::cml) + w * 32;             // [head][4]

  const uint32_t cpv = (uint32_t)(lane & (NCP - 1)) * 8;  // key replica offset within a row
  const uint32_t cpv_v = cpv + 128;                       // value replica offset
  auto kaddr = [&](uint32_t word, int byte) {      // (byte of word) << 8 | cpv
    return __builtin_amdgcn_perm(word, cpv, 0x0C0C0000u | ((4u + byte) << 8));
  };
  auto vaddr = [&](uint32_t word, int byte) {      // (byte of word) << 8 | cpv_v
    return __builtin_amdgcn_perm(word, cpv_v, 0x0C0C0000u | ((4u + byte) << 8));
  };

  // Online softmax of the 8 scores of this lane (tokens A0..A3, B0..B3 of
  // the block, column r), returns the P^T operand (p * nv, high part or
  // remainder by column) and rescales `acc` when the running max grows.
  auto softmax_pv = [&](float (&s)[8], const float (&nv)[8], f4 (&acc)[8]) {
    float bm = fmaxf(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])), fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7])));
    bm = rows_max(bm);
    if (__builtin_amdgcn_ballot_w64(bm > m_run) != 0) {
      const float mnew = fmaxf(m_run, bm);
      const float corr = fexp2(m_run - mnew);
      l_run *= corr;
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) acc[nb] *= corr;
      m_run = mnew;
    }
    float pv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float p = fexp2(s[i] - m_run);
      l_run += p;
      pv[i] = p * nv[i];
    }
    u4 pb;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const hx2 h = __builtin_amdgcn_cvt_pkrtz(pv[2 * j], pv[2 * j + 1]);
      const float t0 = fmaf(-partf, (float)h[0], pv[2 * j]);
      const float t1 = fmaf(-partf, (float)h[1], pv[2 * j + 1]);
      pb[j] = pk_rtz(t0, t1);
    }
    return as_h8(pb);
  };

  // ---- one compressed block (rotated space); `tail` masks tokens past the sequence
  auto packed_block = [&](const Blk& L, int k, auto tail) {
    const int t0 = (blk0 + w + k * FW) << 5;
    f4 sA = {0.f, 0.f, 0.f, 0.f}, sB = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const uint32_t wa = L.k0[s >> 1], wb = L.k1[s >> 1];
      const int by = 2 * (s & 1);
      const u2 ea0 = lds_u2(smem, kaddr(wa, by)), ea1 = lds_u2(smem, kaddr(wa, by + 1));
      const u2 eb0 = lds_u2(smem, kaddr(wb, by)), eb1 = lds_u2(smem, kaddr(wb, by + 1));
      sA = mfma(as_h8(u4{ea0[0], ea0[1], ea1[0], ea1[1]}), qop[s], sA);
      sB = mfma(as_h8(u4{eb0[0], eb0[1], eb1[0], eb1[1]}), qop[s], sB);
    }
    float sc[8];
    const float nk[8] = {L.nkA.x, L.nkA.y, L.nkA.z, L.nkA.w, L.nkB.x, L.nkB.y, L.nkB.z, L.nkB.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sc[i] = (sA[i] + row_ror<G>(sA[i])) * nk[i];
      sc[4 + i] = (sB[i] + row_ror<G>(sB[i])) * nk[4 + i];
    }
    if constexpr (decltype(tail)::value) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (t0 + 4 * q4 + i >= comp) sc[i] = -INFINITY;
        if (t0 + 16 + 4 * q4 + i >= comp) sc[4 + i] = -INFINITY;
      }
    }
    const float nv[8] = {L.nvA.x, L.nvA.y, L.nvA.z, L.nvA.w, L.nvB.x, L.nvB.y, L.nvB.z, L.nvB.w};
    const half8 pb = softmax_pv(sc, nv, acc_r);
    // V^T operands: row = dim 8r + nb, k-slot pairs = token pairs of the lane
    u4 va[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t px = L.v[2 * j], py = L.v[2 * j + 1];  // token pair j
      const u2 x0 = lds_u2(smem, vaddr(px, 0)), x1 = lds_u2(smem, vaddr(px, 1));
      const u2 y0 = lds_u2(smem, vaddr(py, 0)), y1 = lds_u2(smem, vaddr(py, 1));
      va[0][j] = __builtin_amdgcn_perm(y0[0], x0[0], 0x05040100u);
      va[1][j] = __builtin_amdgcn_perm(y0[0], x0[0], 0x07060302u);
      va[2][j] = __builtin_amdgcn_perm(y0[1], x0[1], 0x05040100u);
      va[3][j] = __builtin_amdgcn_perm(y0[1], x0[1], 0x07060302u);
      va[4][j] = __builtin_amdgcn_perm(y1[0], x1[0], 0x05040100u);
      va[5][j] = __builtin_amdgcn_perm(y1[0], x1[0], 0x07060302u);
      va[6][j] = __builtin_amdgcn_perm(y1[1], x1[1], 0x05040100u);
      va[7][j] = __builtin_amdgcn_perm(y1[1], x1[1], 0x07060302u);
    }
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) acc_r[nb] = mfma(as_h8(va[nb]), pb, acc_r[nb]);
  };

  // ---- fp16 blocks of the sink and the residual ring (original space), first
  if (wave_has_fp16) {
    half8 qf[4];
    {
      const uint8_t* src = smem + Layout::qfo + ((uint32_t)(hd * 2 + (partf != 0.f ? 1 : 0)) * 4 + q4) * 4 * 16;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) qf[kb] = *reinterpret_cast<const half8*>(src + 16 * kb);
    }
    f4 acc_o[8];
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) acc_o[nb] = f4{0.f, 0.f, 0.f, 0.f};
    for (int blk = fblk; blk < blk1; blk += FW) {
      const F16Blk L = blk == fblk ? f0 : load_f16(blk, true);
      const bool is_sink = blk < nbc + nbs;
      const int ft0 = (is_sink ? blk - nbc : blk - nbc - nbs) << 5;
      const int flen = is_sink ? sink : res;
      f4 sA = {0.f, 0.f, 0.f, 0.f}, sB = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        sA = mfma(as_h8(L.kA[kb]), qf[kb], sA);
        sB = mfma(as_h8(L.kB[kb]), qf[kb], sB);
      }
      float sc[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sc[i] = (sA[i] + row_ror<G>(sA[i])) * a.qscale;
        sc[4 + i] = (sB[i] + row_ror<G>(sB[i])) * a.qscale;
        if (ft0 + 4 * q4 + i >= flen) sc[i] = -INFINITY;
        if (ft0 + 16 + 4 * q4 + i >= flen) sc[4 + i] = -INFINITY;
      }
      const float ones[8] = {1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f};
      const half8 pb = softmax_pv(sc, ones, acc_o);
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) {
        const uint32_t sel = (nb & 1) ? 0x07060302u : 0x05040100u;
        u4 bv;
#pragma unroll
        for (int j = 0; j < 4; ++j) bv[j] = __builtin_amdgcn_perm(L.v[2 * j + 1][nb >> 1], L.v[2 * j][nb >> 1], sel);
        acc_o[nb] = mfma(as_h8(bv), pb, acc_o[nb]);
      }
    }
    // park the original-space partial (hi + lo columns summed) in LDS with the
    // running max it refers to; later blocks only rescale it at the combine
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float vo[8];
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) vo[nb] = acc_o[nb][i] + row_ror<G>(acc_o[nb][i]);
      if (r < G) {
        float* d = cm + r * 2 * FD + FD + 32 * q4 + 8 * i;
        *reinterpret_cast<float4*>(d) = make_float4(vo[0], vo[1], vo[2], vo[3]);
        *reinterpret_cast<float4*>(d + 4) = make_float4(vo[4], vo[5], vo[6], vo[7]);
      }
    }
    m_orig = m_run;
  }

  // B operands of the rotated-space scores, step s: k-slots (q4, i) hold
  // q[d], q[d+1], q[d], q[d+1], q[d+2], q[d+3], q[d+2], q[d+3], d = 32*q4 + 4*s,
  // matching the key table entry layout (hi pair, lo pair) of two code bytes;
  // column r reads the high part (even r / G) or the remainder of head r % G.
  {
    const uint8_t* src = smem + Layout::qop + (uint32_t)(hd * 2 + (partf != 0.f ? 1 : 0)) * 512 + (uint32_t)q4 * 128;
#pragma unroll
    for (int s = 0; s < 8; ++s) qop[s] = *reinterpret_cast<const half8*>(src + 16 * s);
  }

#pragma unroll
  for (int nb = 0; nb < 8; ++nb) acc_r[nb] = f4{0.f, 0.f, 0.f, 0.f};

  // ---- compressed blocks: two load slots, one block in flight
  {
    constexpr std::false_type full{};
    // loads stay unconditional (the wait counts need one issue order);
    // only the compute is skipped past the wave's last full block
    Blk b1 = load_blk(1);
    for (int k = 0; k < npf; k += 2) {
      packed_block(b0, k, full);
      b0 = load_blk(k + 2);
      if (k + 1 < npf) packed_block(b1, k + 1, full);
      b1 = load_blk(k + 3);
    }
    if (npf < npk) packed_block(load_tail(npf), npf, std::true_type{});
  }

  // ---- combine the 8 waves of this workgroup through LDS (own region, one barrier).
  // Columns r and r + G hold the fp16 high part / remainder products of head r:
  // one DPP row rotation by G adds them; lanes r < G then hold head r.
  l_run = rows_sum(l_run);
  const bool wg_has_fp16 = blk1 > nbc;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float vr[8];
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) vr[nb] = acc_r[nb][i] + row_ror<G>(acc_r[nb][i]);
    if (r < G) {
      float* d = cm + r * 2 * FD + 32 * q4 + 8 * i;
      *reinterpret_cast<float4*>(d) = make_float4(vr[0], vr[1], vr[2], vr[3]);
      *reinterpret_cast<float4*>(d + 4) = make_float4(vr[4], vr[5], vr[6], vr[7]);
    }
  }
  if (lane < G) *reinterpret_cast<float4*>(cl + 4 * lane) = make_float4(m_run, l_run, m_orig, 0.f);
  __syncthreads();
  // thread (head, dim): merge the 8 waves, write the workgroup partial
  float* part = a.part + ((int64_t)row * a.nwg + c) * G * PS;
  const float* cms = reinterpret_cast<const float*>(smem + Layout::cmb);
  const float* cls = reinterpret_cast<const float*>(smem + Layout::cml);
  for (int e = tid; e < G * FD; e += FT) {
    const int h = e / FD, j = e % FD;
    float M = M_INIT;
#pragma unroll
    for (int ww = 0; ww < FW; ++ww) M = fmaxf(M, cls[ww * 32 + 4 * h]);
    float sr = 0.f, so = 0.f, L = 0.f;
#pragma unroll
    for (int ww = 0; ww < FW; ++ww) {
      const float4 st = *reinterpret_cast<const float4*>(cls + ww * 32 + 4 * h);
      const float sc = fexp2(st.x - M);
      const float* src = cms + ((ww * 8 + h) * 2) * FD + j;
      sr = fmaf(sc, src[0], sr);
      // original-space part, parked at max st.z (absent: M_INIT, the LDS row is unwritten)
      if (wg_has_fp16 && st.z > M_INIT) so = fmaf(fexp2(st.z - M), src[FD], so);
      L = fmaf(sc, st.y, L);
    }
    part[h * PS + P_ROT + j] = sr;
    if (wg_has_fp16) part[h * PS + P_ORIG + j] = so;
    if (j == 0) *reinterpret_cast<float4*>(part + h * PS) = make_float4(M, L, wg_has_fp16 ? 1.f : 0.f, 0.f);
  }
}

// Merge of the per-workgroup partials of one query head of (kv head g, sequence b)
// and the inverse rotation, a second launch on the same stream (the kernel
// boundary makes the partials visible):
//   out = (sum_p w_p rot_p) R + sum_p w_p orig_p,  w_p = 2^(M_p - M) / L
// (docs/FULL_FUSED_ATTENTION_RESULTS.md:34-40). One workgroup (4 waves) per
// query head; reductions across lanes use permlane / DPP, not LDS loops.
constexpr int MT = 256;  // merge threads

__device__ inline float wave_max(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true)));  // quad_perm 1,0,3,2
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true)));  // quad_perm 2,3,0,1
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, true))); // row_half_mirror
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, true))); // row_mirror
  return rows_max(v);
}

__device__ inline float wave_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, true));
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, true));
  return rows_sum(v);
}

template <int G>
__global__ __launch_bounds__(MT) void fast_merge_kernel(FastArgs a) {
  constexpr int PPT = 4;                             // partials per thread per pass
  __shared__ __align__(16) float red[8][FD + 4];     // per-group sums of rot (then of the rotation)
  __shared__ __align__(16) float redo[8][FD + 4];    // per-group sums of orig
  __shared__ __align__(16) float fin[FD];
  const int h = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  {  // one batch of scalar loads for the arguments (see the decode kernel)
    const void* p0 = a.part; const void* p1 = a.rot; const void* p2 = a.out;
    const int i0 = a.nwg, i1 = a.hkv, i2 = a.hq;
    asm volatile("" ::"s"(p0), "s"(p1), "s"(p2), "s"(i0), "s"(i1), "s"(i2));
  }
  const int row = b * a.hkv + g;
  const int np = a.nwg;
  const float* pb = a.part + (int64_t)row * np * G * PS + h * PS;  // partial p at pb + p * G * PS
  const int jq = tid & 31, grp = tid >> 5;  // dims 4*jq .. 4*jq+3, partials grp, grp + 8, ...

  // rotation rows for the final product: thread (grp, jq) holds R[16*grp + i][4*jq .. +3]
  float4 rr[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) rr[i] = *reinterpret_cast<const float4*>(a.rot + (16 * grp + i) * FD + 4 * jq);

  // global max / sum: every wave reduces all partial headers itself (no barrier)
  float M = M_INIT;
  float mh[MAXWG / 64], lh[MAXWG / 64];
#pragma unroll
  for (int k = 0; k < MAXWG / 64; ++k) {
    const int p = lane + 64 * k;  // loads stay unconditional (exact wait counts), values masked
    const float4 x = *reinterpret_cast<const float4*>(pb + (int64_t)min(p, np - 1) * G * PS);
    mh[k] = p < np ? x.x : M_INIT;
    lh[k] = p < np ? x.y : 0.f;
    M = fmaxf(M, mh[k]);
  }
  M = wave_max(M);
  float L = 0.f;
#pragma unroll
  for (int k = 0; k < MAXWG / 64; ++k) L = fmaf(fexp2(mh[k] - M), lh[k], L);
  L = wave_sum(L);
  const float inv = L > 0.f ? 1.f / L : 0.f;

  // weighted sums of this thread's partials
  float4 sr = make_float4(0.f, 0.f, 0.f, 0.f), so = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int p0 = grp; p0 < np; p0 += 8 * PPT) {
    float4 hv[PPT], rv[PPT];
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
      const int p = min(p0 + 8 * k, np - 1);
      hv[k] = *reinterpret_cast<const float4*>(pb + (int64_t)p * G * PS);
      rv[k] = *reinterpret_cast<const float4*>(pb + (int64_t)p * G * PS + P_ROT + 4 * jq);
    }
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
      const float wp = p0 + 8 * k < np ? fexp2(hv[k].x - M) * inv : 0.f;
      sr.x = fmaf(wp, rv[k].x, sr.x);
      sr.y = fmaf(wp, rv[k].y, sr.y);
      sr.z = fmaf(wp, rv[k].z, sr.z);
      sr.w = fmaf(wp, rv[k].w, sr.w);
      if (p0 + 8 * k < np && hv[k].z != 0.f) {  // original-space part (sink / residual blocks)
        const float4 o = *reinterpret_cast<const float4*>(pb + (int64_t)(p0 + 8 * k) * G * PS + P_ORIG + 4 * jq);
        so.x = fmaf(wp, o.x, so.x);
        so.y = fmaf(wp, o.y, so.y);
        so.z = fmaf(wp, o.z, so.z);
        so.w = fmaf(wp, o.w, so.w);
      }
    }
  }
  *reinterpret_cast<float4*>(&red[grp][4 * jq]) = sr;
  *reinterpret_cast<float4*>(&redo[grp][4 * jq]) = so;
  __syncthreads();
  if (tid < FD) {
    float x = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) x += red[k][tid];
    fin[tid] = x;
  }
  __syncthreads();
  // out[j] = sum_i fin[i] R[i][j] + orig[j]: group grp covers rows i = 16*grp .. +15
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float f = fin[16 * grp + i];
    acc.x = fmaf(f, rr[i].x, acc.x);
    acc.y = fmaf(f, rr[i].y, acc.y);
    acc.z = fmaf(f, rr[i].z, acc.z);
    acc.w = fmaf(f, rr[i].w, acc.w);
  }
  *reinterpret_cast<float4*>(&red[grp][4 * jq]) = acc;
  __syncthreads();
  if (tid < FD) {
    float x = 0.f, y = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      x += red[k][tid];
      y += redo[k][tid];
    }
    a.out[((int64_t)b * a.hq + g * G + h) * FD + tid] = x + y;
  }
}

size_t fast_smem_bytes() { return Layout::total; }

int fast_max_wg() { return MAXWG; }

template <int G>
static void launch_pair(const FastArgs& a, int batch, bool merge, hipStream_t s) {
  hipLaunchKernelGGL((fast_decode_kernel<G>), dim3(a.nwg, a.hkv, batch), dim3(FT), 0, s, a);
  if (merge) hipLaunchKernelGGL((fast_merge_kernel<G>), dim3(G, a.hkv, batch), dim3(MT), 0, s, a);
}

int launch_fast_decode(const FastArgs& a, int G, int batch, bool merge, hipStream_t s) {
  switch (G) {
    case 1: launch_pair<1>(a, batch, merge, s); break;
    case 2: launch_pair<2>(a, batch, merge, s); break;
    case 4: launch_pair<4>(a, batch, merge, s); break;
    default: launch_pair<8>(a, batch, merge, s); break;
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// The kernel's LDS is static (Layout::total bytes); nothing to raise.
int fast_set_attributes() { return 0; }

}  // namespace tq
