// Fused decode attention for fractional-width TurboQuant caches (2.5 / 3.5
// bits: rotated dims [0, 64) quantised at the higher width KH / VH, dims
// [64, 128) at the lower width KL / VL, both codebooks built for d = 128;
// cache.py:63-84, 253-300) on gfx950, uniform batches, head_dim 128, fp16
// K/V, one query token. The partials + merge structure, the fp16 tile, the
// online softmax and the partial format are those of uniform_decode_kernel
// (tq_decode_uniform.h); what differs is the placement of the two code
// segments, so that every MFMA reads codes of one width:
//  - scores S^T = K q^T (MFMA 16x16x32 f16): k-steps 0-3 take the hi dims and
//    4-7 the lo dims; in step s lane (r, q4) holds dims d .. d + 3 of token r
//    (tile A) and 16 + r (tile B), d = 64 (s >> 2) + 16 q4 + 4 (s & 3), as
//    two entries of a pair table (2 dims per entry: fp16 high parts, then
//    remainders), and the query B operands repeat q[d], q[d + 1] as in the
//    integer kernels;
//  - output O^T += V^T P^T: PV MFMA nb produces rotated dims 64 (nb >> 2) +
//    4 r + (nb & 3) in row r, so MFMAs 0-3 read hi codes and 4-7 lo codes;
//    each takes two MFMAs (high parts, then remainders: centroids are not
//    fp16 numbers);
//  - a lane's key codes of a segment are 16 W contiguous bits (W the width)
//    of the token's row, loaded as two dwords; a block's value rows (32
//    tokens, hi and lo) arrive as one 16-byte load per lane per segment and
//    are staged in the wave's LDS area, from which each lane reads its 4 W
//    bits per token;
//  - the four pair tables (keys hi / lo, values hi / lo) hold 16 replicas
//    (128-byte rows; 80 KB at K3.5 / V3.5) and are built from the codecs'
//    float32 centroids in device memory (fp16 high part / remainder split in
//    the kernel, one lane per centroid, rows assembled with ds_bpermute).
// A side may also be integer (KI / VI: one codebook, the code row of 16 W
// bytes holds both segments, the lo one from byte 8 W), so that a
// fractional width on one side pairs with an integer width on the other.
// Partials are in the uniform kernel's format; uniform_merge_kernel merges
// them (value scale 1).
#pragma once

#include "tq_decode_uniform.h"

namespace tq {
namespace uk {

// LDS of the split kernel below the combine headers (Layout::cml): the pair
// tables (16 replicas of 8 bytes per row) and each wave's value-code staging
// (a block's hi rows, then its lo rows)
template <int KH, int KL, int VH, int VL, bool KI, bool VI>
struct SplitLds {
  static constexpr uint32_t RB = 128;  // bytes per table row
  static constexpr uint32_t vht = 0;
  static constexpr uint32_t vlt = VI ? vht : vht + (RB << (2 * VH));  // an integer side has one table
  static constexpr uint32_t kht = vlt + (VI ? (RB << (2 * VH)) : (RB << (2 * VL)));
  static constexpr uint32_t klt = KI ? kht : kht + (RB << (2 * KH));
  static constexpr uint32_t vst = klt + (RB << (2 * KL));
  // a block's value rows in the wave's staging area: hi rows (32 tokens x 8 VH
  // bytes) then lo rows, or (integer) the 32 rows of 16 VH bytes as they are
  static constexpr uint32_t VHB = VI ? 32 * 16 * VH : 32 * 8 * VH;
  static constexpr uint32_t VLB = VI ? 0 : 32 * 8 * VL;
  static constexpr uint32_t VSTW = VHB + VLB;   // per wave
  // staged row stride and the offset of the lo segment of token t's codes
  static constexpr uint32_t VRH = VI ? 16 * VH : 8 * VH, VRL = VI ? 16 * VH : 8 * VL;
  static constexpr uint32_t VLO = VI ? 8 * VH : VHB;
  static constexpr uint32_t end = vst + FW * VSTW;
  static_assert(end <= Layout::cml, "tables and staging below the combine headers");
  static_assert(FW * 8 * CMS * 4 <= Layout::cml, "combine buffers alias the table region");
};

// Pair table of B-bit codes, 16 replicas: row e = (c_hi[e & M], c_hi[e >> B],
// c_lo[e & M], c_lo[e >> B]) fp16, M = 2^B - 1, with c[i] (fp16 high part |
// remainder << 16) in lane cl0 + i of cw. Thread t stores replicas 2 (t & 7)
// and 2 (t & 7) + 1 of rows (t >> 3) + 64 k (one 16-byte store each).
template <int B>
__device__ inline void pair_table16(uint8_t* tab, int tid, uint32_t cw, int cl0) {
  constexpr int NR = 1 << (2 * B), M = (1 << B) - 1;
#pragma unroll
  for (int r0 = 0; r0 < NR; r0 += FT / 8) {
    const int row = r0 + (tid >> 3);
    const int rr = row < NR ? row : NR - 1;  // every lane takes part in the permutes
    const uint32_t ca = __builtin_amdgcn_ds_bpermute(4 * (cl0 + (rr & M)), (int)cw);
    const uint32_t cb = __builtin_amdgcn_ds_bpermute(4 * (cl0 + (rr >> B)), (int)cw);
    const uint32_t k0 = __builtin_amdgcn_perm(cb, ca, 0x05040100u);  // (c_hi[e & M], c_hi[e >> B])
    const uint32_t k1 = __builtin_amdgcn_perm(cb, ca, 0x07060302u);  // (c_lo[e & M], c_lo[e >> B])
    if (NR >= FT / 8 || row < NR) *reinterpret_cast<u4*>(tab + row * 128 + (tid & 7) * 16) = u4{k0, k1, k0, k1};
  }
}

// Bits [off, off + n) of the 64-bit value (x[1]:x[0]), off and n compile-time
template <int OFF, int N>
__device__ inline uint32_t bits64(const u2& x) {
  if constexpr (OFF + N <= 32) return (x[0] >> OFF) & ((1u << N) - 1u);
  else if constexpr (OFF >= 32) return (x[1] >> (OFF - 32)) & ((1u << N) - 1u);
  else return __builtin_amdgcn_alignbit(x[1], x[0], OFF) & ((1u << N) - 1u);
}

// The compressed blocks of one wave: loads issued ahead (lane r, q4)
struct SBlk {
  u2 kh[2], kl[2];  // key segments (hi, lo) of tokens t0 + r and t0 + 16 + r
  u4 vh, vl;        // 16 bytes of the block's hi / lo value rows (bytes 16 lane ..)
  float nk, nv;     // key / value norm of token t0 + (lane & 31)
};

template <int G, int NPW, int KH, int KL, int VH, int VL, bool KI, bool VI>
__global__ __launch_bounds__(FT) void split_decode_kernel(UniformArgs a) {
  static_assert(KH >= 2 && KH <= 4 && KL >= 2 && KL <= 4 && VH >= 2 && VH <= 4 && VL >= 2 && VL <= 4, "widths 2-4");
  static_assert((!KI || KH == KL) && (!VI || VH == VL), "an integer side has one width");
  using SL = SplitLds<KH, KL, VH, VL, KI, VI>;
  __shared__ __align__(16) uint8_t smem[Layout::total];

  const int c = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, q4 = lane >> 4;
  const int row = b * a.hkv + g;
  const int j0 = 16 * w;  // output-dim tile of this wave for the query rotation
  constexpr int TS = G <= 4 ? 2 : 1;
  constexpr int NS = 8 / TS;
  const int tile = TS == 2 ? r >> 3 : 0;
  const int c8 = r & 7;
  const int hd = TS == 2 ? (c8 < 4 ? c8 : 7 - c8) % G : c8;
  const bool lo_part = TS == 2 ? c8 >= 4 : r >= 8;
  const float partf = lo_part ? 1.f : 0.f;
  const bool writer = !lo_part && c8 < G;

  // the codebooks first, one centroid per lane (keys hi: lanes 0-15, keys lo:
  // 16-31, values hi: 32-47, values lo: 48-63; an integer side's lo codebook is
  // its hi one), so they are the first loads to return
  float cen;
  {
    const int i = lane & 15, grp = lane >> 4;
    const int n = grp == 0 ? (1 << KH) : grp == 1 ? (1 << KL) : grp == 2 ? (1 << VH) : (1 << VL);
    const float* src = grp == 0 ? a.kcen_hi : grp == 1 ? a.kcen_lo : grp == 2 ? a.vcen_hi : a.vcen_lo;
    cen = src[i < n ? i : n - 1];
  }
  const int comp = a.max_comp, sink = a.max_sink, res = a.max_res;
  int rs_raw;
  {
    typedef const __attribute__((address_space(4))) uint32_t* kptr;
    const auto* kargs = (const __attribute__((address_space(4))) uint8_t*)__builtin_amdgcn_kernarg_segment_ptr();
    const kptr rsp = a.res_start_b ? (kptr)(a.res_start_b + b) : (kptr)(kargs + offsetof(UniformArgs, res_start0));
    rs_raw = (int)*rsp;
  }
  const int rstart = min(max(rs_raw, 0), max(a.res_cap - 1, 0));
  const int nbc = (comp + 31) >> 5;
  const int blk0 = c * a.bpw, blk1 = min(blk0 + a.bpw, nbc);
  const int f0 = c * a.fpw, nf = max(0, min(a.fpw, sink + res - f0));

  // ---- set-up loads: R rows, q, the workgroup's fp16 tokens (as in the
  // uniform kernel)
  u4 rqh[4], rql[4];
  {
    const uint16_t* rh = a.rot16 + (j0 + r) * FD + 8 * q4;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      rqh[kb] = *reinterpret_cast<const u4*>(rh + 32 * kb);
      rql[kb] = *reinterpret_cast<const u4*>(rh + FD * FD + 32 * kb);
    }
  }
  const int esz = a.q_dtype == TQ_F32 ? 4 : 2;
  const int qchunks = G * FD * esz / 16;
  u4 qld;
  {
    const uint8_t* qp = static_cast<const uint8_t*>(a.q) + ((int64_t)b * a.hq + g * G) * FD * esz;
    const int e = tid < qchunks ? tid : 0;
    qld = *reinterpret_cast<const u4*>(qp + 16 * e);
  }
  u4 fst;
  {
    const int e = tid;
    const int u = f0 + min(e >> 5, max(nf - 1, 0));
    const bool is_v = (e >> 4) & 1;
    int sl = rstart + (u - sink);
    sl = sl >= a.res_cap ? sl - a.res_cap : sl;
    const uint16_t* ps = static_cast<const uint16_t*>(is_v ? a.sink_v : a.sink_k) + (int64_t)row * a.sink_hs + (int64_t)u * FD;
    const uint16_t* pr = static_cast<const uint16_t*>(is_v ? a.res_v : a.res_k) + (int64_t)row * a.res_hs + (int64_t)sl * FD;
    const uint16_t* src = nf == 0 ? a.rot16 : (u < sink ? ps : pr);
    fst = *reinterpret_cast<const u4*>(src + 8 * (e & 15));
  }
  // ---- block loads: buffers over the tokens [t0, comp) of the row (bytes
  // past the sequence read as zero; slots past the wave's blocks re-read
  // block 0 and are masked)
  // an integer side reads its lo segment from the same row, 8 W bytes in
  const uint8_t* kch = a.kc + (int64_t)row * a.k_hs;
  const uint8_t* kcl = KI ? kch + 8 * KH : a.kcl + (int64_t)row * a.kl_hs;
  const uint8_t* vch = a.vc + (int64_t)row * a.v_hs;
  const uint8_t* vcl = a.vcl + (int64_t)row * a.vl_hs;
  const float* knorm = a.kn + (int64_t)row * a.kn_hs;
  const float* vnorm = a.vn + (int64_t)row * a.vn_hs;
  auto slot_t0 = [&](int k) {
    const int blk = blk0 + w + FW * k;
    return blk < blk1 ? blk << 5 : 0;
  };
  // key segment of width W of token `tok`: 16 W bits at bit 16 W q4 of the
  // segment (rows of RK bytes), loaded as two dwords from a dword-aligned
  // offset (3 bits: the segment starts 16 bits into the first dword for odd q4)
  constexpr int RKH = KI ? 16 * KH : 8 * KH, RKL = KI ? 16 * KH : 8 * KL;
  auto koff = [&](int W, int RK, int tok) { return tok * RK + (W == 3 ? 4 * ((6 * q4) >> 2) : 2 * W * q4); };
  const int no = (lane & 31) * 4;
  SBlk B[NPW];
  auto kload = [&](__amdgpu_buffer_rsrc_t rk, int W, int RK, int tok) -> u2 {
    if (W == 2) return u2{__builtin_amdgcn_raw_buffer_load_b32(rk, koff(W, RK, tok), 0, 0), 0u};
    return __builtin_amdgcn_raw_buffer_load_b64(rk, koff(W, RK, tok), 0, 0);
  };
  auto load_slot = [&](int k) {
    const int t0 = slot_t0(k);
    const int n = comp - t0;
    const __amdgpu_buffer_rsrc_t rkh = rsrc(kch + (int64_t)t0 * RKH, n * RKH);
    const __amdgpu_buffer_rsrc_t rkl = rsrc(kcl + (int64_t)t0 * RKL, n * RKL);
    const __amdgpu_buffer_rsrc_t rvh = rsrc(vch + (int64_t)t0 * SL::VRH, n * SL::VRH);
    const __amdgpu_buffer_rsrc_t rvl = VI ? rvh : rsrc(vcl + (int64_t)t0 * (8 * VL), n * 8 * VL);
    const __amdgpu_buffer_rsrc_t rkn = rsrc(knorm + t0, n * 4);
    const __amdgpu_buffer_rsrc_t rvn = rsrc(vnorm + t0, n * 4);
    B[k].kh[0] = kload(rkh, KH, RKH, r);
    B[k].kh[1] = kload(rkh, KH, RKH, 16 + r);
    B[k].kl[0] = kload(rkl, KL, RKL, r);
    B[k].kl[1] = kload(rkl, KL, RKL, 16 + r);
    // the block's value bytes: [16 lane, + 16) of the hi rows and of the lo
    // rows, or (integer) [16 lane, + 16) and [1024 + 16 lane, + 16) of its rows
    B[k].vh = __builtin_amdgcn_raw_buffer_load_b128(rvh, 16 * lane, 0, 0);
    if constexpr (!VI || SL::VHB > 1024) B[k].vl = __builtin_amdgcn_raw_buffer_load_b128(rvl, (VI ? 1024 : 0) + 16 * lane, 0, 0);
    B[k].nk = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rkn, no, 0, 0));
    B[k].nv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rvn, no, 0, 0));
  };
  load_slot(0);

  // ---- tables: the centroids' fp16 high part / remainder per lane, then
  // the four pair tables
  {
    const _Float16 h = (_Float16)cen;
    const uint32_t cw = (uint32_t)__builtin_bit_cast(uint16_t, h) |
                        ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(cen - (float)h)) << 16);
    pair_table16<KH>(smem + SL::kht, tid, cw, 0);
    if constexpr (!KI) pair_table16<KL>(smem + SL::klt, tid, cw, 16);
    pair_table16<VH>(smem + SL::vht, tid, cw, 32);
    if constexpr (!VI) pair_table16<VL>(smem + SL::vlt, tid, cw, 48);
  }
  if (tid < qchunks) *reinterpret_cast<u4*>(smem + Layout::qst + 16 * tid) = qld;
  *reinterpret_cast<u4*>(smem + Layout::f16s + (tid >> 5) * (2 * FROW) + ((tid >> 4) & 1) * FROW + 16 * (tid & 15)) = fst;
  __syncthreads();

  load_slot(1);

  // q rows as MFMA A operands, scaled by 2^-qe per head (as in the uniform
  // kernel)
  half8 qo_hi[4], qo_lo[4];
  float qe_scale = 1.f;
  bool q_exact = false;
  {
    const uint8_t* qr = smem + Layout::qst + (uint32_t)min(r, G - 1) * FD * esz;
    if (a.q_dtype == TQ_F16) {
      u4 raw[4];
      float ss = 0.f;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        raw[kb] = *reinterpret_cast<const u4*>(qr + 2 * (32 * kb + 8 * q4));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const f16x2 h2 = __builtin_bit_cast(f16x2, raw[kb][j]);
          ss = __builtin_amdgcn_fdot2(h2, h2, ss, false);
        }
      }
      ss = rows_sum(ss);
      q_exact = __builtin_amdgcn_ballot_w64(__float_as_uint(sqrtf(ss) * a.qscale) - __float_as_uint(Q_LOW) >
                                            __float_as_uint(Q_LIMIT) - __float_as_uint(Q_LOW)) == 0;
      if (q_exact) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          qo_hi[kb] = as_h8(raw[kb]);
          qo_lo[kb] = as_h8(u4{0u, 0u, 0u, 0u});
        }
      }
    }
    if (!q_exact) {
      float x[4][8];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const int d = 32 * kb + 8 * q4;
        if (a.q_dtype == TQ_F32) {
          const float4 u0 = *reinterpret_cast<const float4*>(qr + 4 * d);
          const float4 u1 = *reinterpret_cast<const float4*>(qr + 4 * d + 16);
          x[kb][0] = u0.x; x[kb][1] = u0.y; x[kb][2] = u0.z; x[kb][3] = u0.w;
          x[kb][4] = u1.x; x[kb][5] = u1.y; x[kb][6] = u1.z; x[kb][7] = u1.w;
        } else {
          const u4 u = *reinterpret_cast<const u4*>(qr + 2 * d);
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const uint32_t hb = (u[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
            x[kb][i] = a.q_dtype == TQ_BF16 ? __uint_as_float(hb << 16) : (float)__builtin_bit_cast(_Float16, (uint16_t)hb);
          }
        }
      }
      float ss = 0.f;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 8; ++i) ss = fmaf(x[kb][i], x[kb][i], ss);
      ss = rows_sum(ss);
      const int qe = query_exponent(sqrtf(ss), a.qscale, Q_LIMIT, Q_LOW);
      const float qdown = __builtin_amdgcn_ldexpf(1.f, -qe);
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float xs = x[kb][i] * qdown;
          qo_hi[kb][i] = (_Float16)xs;
          qo_lo[kb][i] = (_Float16)(xs - (float)qo_hi[kb][i]);
        }
      int qeh = 0;
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const int xh = __builtin_amdgcn_readlane(qe, h);
        qeh = hd == h ? xh : qeh;
      }
      qe_scale = __builtin_amdgcn_ldexpf(1.f, qeh);
    }
  }
  // ---- q_rot tile D[h][n] = sum_i q[h][i] R[j0+n][i], written (times
  // qscale) as fp16 high part / remainder into the score B-operand layout
  // [head][part][q4][s][8 halves]: dim j of segment j >> 6 sits at lane q4 =
  // (j & 63) >> 4, step s = 4 (j >> 6) + ((j >> 2) & 3), halves (e & 1) +
  // 4 (e >> 1) and + 2, e = j & 3
  {
    f4 dq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      dq = mfma(qo_hi[kb], as_h8(rqh[kb]), dq);
      dq = mfma(qo_hi[kb], as_h8(rql[kb]), dq);
      if (!q_exact) dq = mfma(qo_lo[kb], as_h8(rqh[kb]), dq);
    }
    const int j = j0 + r, e = j & 3;
    const int sq4 = (j & 63) >> 4, ss = 4 * (j >> 6) + ((j >> 2) & 3);
    const uint32_t off = ((uint32_t)sq4 * 8 + ss) * 16 + 2 * ((e & 1) + 4 * (e >> 1));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * q4 + i;
      if (h < G) {
        const float v = dq[i] * a.qscale;
        const _Float16 hi = (_Float16)v, lo = (_Float16)(v - (float)hi);
        uint8_t* dh = smem + Layout::qop + (uint32_t)(h * 2) * QOPS + off;
        *reinterpret_cast<_Float16*>(dh) = hi;
        *reinterpret_cast<_Float16*>(dh + 4) = hi;
        *reinterpret_cast<_Float16*>(dh + QOPS) = lo;
        *reinterpret_cast<_Float16*>(dh + QOPS + 4) = lo;
      }
    }
  }
  if (w == 0 && r < G && nf > 0) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      uint8_t* d = smem + Layout::qfo + ((uint32_t)(r * 2 * 4 + kb) * 4 + q4) * 16;
      *reinterpret_cast<half8*>(d) = qo_hi[kb];
      *reinterpret_cast<half8*>(d + 4 * 4 * 16) = qo_lo[kb];
    }
  }
  __syncthreads();

  float m_run = M_INIT, l_run = 0.f;
  int vx = 0;
  bool vset = false;
  float m_orig = M_INIT;
  f4 acc_r[8];

  // online softmax of the lane's NS scores (as in the uniform kernel)
  auto softmax_pv = [&](float (&s)[NS], const float (&nv)[NS], f4 (&acc)[8], bool setx) {
    float bm = s[0];
#pragma unroll
    for (int i = 1; i < NS; ++i) bm = fmaxf(bm, s[i]);
    bm = rows_max(bm);
    if (__builtin_amdgcn_ballot_w64(bm > m_run) != 0) {
      const float mnew = bm > m_run ? bm + RESCALE_MARGIN : m_run;
      const float corr = fexp2(m_run - mnew);
      l_run *= corr;
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) acc[nb] *= corr;
      m_run = mnew;
    }
    float pv[NS];
    float pm = 0.f;
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const float p = fexp2(s[i] - m_run);
      l_run += p;
      pv[i] = p * nv[i];
      pm = fmaxf(pm, fabsf(pv[i]));
    }
    const float pmx = pm * __builtin_amdgcn_ldexpf(1.f, -vx);
    const bool first = setx && !vset;
    if (__builtin_amdgcn_ballot_w64(pmx > PV_LIMIT || (first && pmx > 0.f)) != 0) {
      const float cm = rows_max(pmx);
      int dx;
      if (first) {
        dx = cm > 0.f ? max((int)ceilf(log2f(cm / PV_SET)), -110) : 0;
        vset = true;
      } else {
        dx = cm > PV_LIMIT ? (int)ceilf(log2f(cm / PV_LIMIT)) : 0;
      }
      const float f = __builtin_amdgcn_ldexpf(1.f, -dx);
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) acc[nb] *= f;
      vx += dx;
    }
    const float down = __builtin_amdgcn_ldexpf(1.f, -vx);
    uint32_t d[NS / 2];
#pragma unroll
    for (int j = 0; j < NS / 2; ++j) {
      const float p0 = pv[2 * j] * down, p1 = pv[2 * j + 1] * down;
      const hx2 h = __builtin_amdgcn_cvt_pkrtz(p0, p1);
      const float t0 = fmaf(-partf, (float)h[0], p0);
      const float t1 = fmaf(-partf, (float)h[1], p1);
      d[j] = pk_rtz(t0, t1);
    }
    u4 pb;
    if constexpr (TS == 2) {
      pb[0] = tile ? 0u : d[0];
      pb[1] = tile ? 0u : d[1];
      pb[2] = tile ? d[0] : 0u;
      pb[3] = tile ? d[1] : 0u;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) pb[j] = d[j];
    }
    return as_h8(pb);
  };

  // ---- the staged fp16 tokens (original space): wave WF16, before its
  // compressed blocks (the uniform kernel's fp16 tile)
  if (w == WF16 && nf > 0) {
    half8 qf[4];
    {
      const uint8_t* src = smem + Layout::qfo + ((uint32_t)(hd * 2 + (partf != 0.f ? 1 : 0)) * 4 + q4) * 4 * 16;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) qf[kb] = *reinterpret_cast<const half8*>(src + 16 * kb);
    }
    f4 acc_o[8];
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) acc_o[nb] = f4{0.f, 0.f, 0.f, 0.f};
    const uint8_t* fs = smem + Layout::f16s;
    f4 sA = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const u4 kA = *reinterpret_cast<const u4*>(fs + r * (2 * FROW) + 64 * q4 + 16 * kb);
      sA = mfma(as_h8(kA), qf[kb], sA);
    }
    float sc[NS], ones[NS];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float full = (sA[i] + partner<G>(sA[i])) * (a.qscale * qe_scale);
      sc[i] = tile == 0 && 4 * q4 + i < nf ? full : -INFINITY;
      if constexpr (NS == 8) sc[4 + i] = -INFINITY;
    }
#pragma unroll
    for (int i = 0; i < NS; ++i) ones[i] = 1.f;
    const half8 pb = softmax_pv(sc, ones, acc_o, false);
    u4 vv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      vv[i] = i < 4 ? *reinterpret_cast<const u4*>(fs + (4 * q4 + i) * (2 * FROW) + FROW + 16 * r) : u4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
      const uint32_t sel = (nb & 1) ? 0x07060302u : 0x05040100u;
      u4 bv;
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[j] = __builtin_amdgcn_perm(vv[2 * j + 1][nb >> 1], vv[2 * j][nb >> 1], sel);
      acc_o[nb] = mfma(as_h8(bv), pb, acc_o[nb]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float vo[8];
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) vo[nb] = acc_o[nb][i] + partner<G>(acc_o[nb][i]);
      if (writer && tile == 0) {
        float* d = reinterpret_cast<float*>(smem + Layout::opk) + hd * FD + 32 * q4 + 8 * i;
        *reinterpret_cast<float4*>(d) = make_float4(vo[0], vo[1], vo[2], vo[3]);
        *reinterpret_cast<float4*>(d + 4) = make_float4(vo[4], vo[5], vo[6], vo[7]);
      }
    }
    m_orig = m_run;
  }

  half8 qop[8];
  {
    const uint8_t* src = smem + Layout::qop + (uint32_t)(hd * 2 + (partf != 0.f ? 1 : 0)) * QOPS + (uint32_t)q4 * 128;
#pragma unroll
    for (int s = 0; s < 8; ++s) qop[s] = *reinterpret_cast<const half8*>(src + 16 * s);
  }
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) acc_r[nb] = f4{0.f, 0.f, 0.f, 0.f};

  static_assert(NPW >= 2, "two blocks in flight");
  uint8_t* nst = smem + Layout::nst + w * 256;
  uint8_t* vst = smem + SL::vst + w * SL::VSTW;
  const uint32_t cp = (uint32_t)(lane & 15) * 8;  // replica offset within a table row
  // table address of a field value x (2 W bits) of table T
  auto taddr = [&](uint32_t T, uint32_t x) { return T + ((x << 7) | cp); };
  // the lane's 4 W value bits of token tt from the staged rows of width W
  // (row stride RV) at `base`: dims 4 r .. 4 r + 3 of the segment
  auto vcode = [&](const uint8_t* base, int W, int RV, int tt) -> uint32_t {
    const uint8_t* p = base + tt * RV;
    if (W == 4) return *reinterpret_cast<const uint16_t*>(p + 2 * r);
    if (W == 2) return p[r];
    const uint32_t* dw = reinterpret_cast<const uint32_t*>(p) + ((12 * r) >> 5);  // 3 bits: 12 r .. 12 r + 11
    return __builtin_amdgcn_alignbit(dw[1], dw[0], (12 * r) & 31) & 0xFFFu;
  };

#pragma unroll
  for (int k = 0; k < NPW; ++k) {
    if (k + 2 < NPW) load_slot(k + 2);
    const SBlk& L = B[k];
    const int t0 = slot_t0(k);
    const int tend = blk0 + w + FW * k < blk1 ? comp : 0;
    *reinterpret_cast<float*>(nst + 4 * lane) = lane < 32 ? L.nk : L.nv;
    // the block's value rows: hi rows then lo rows, or the integer rows (lanes
    // past each part store nothing)
    if constexpr (VI) {
      if (16 * lane < (int)SL::VHB) *reinterpret_cast<u4*>(vst + 16 * lane) = L.vh;
      if (1024 + 16 * lane < (int)SL::VHB) *reinterpret_cast<u4*>(vst + 1024 + 16 * lane) = L.vl;
    } else {
      if (16 * lane < (int)SL::VHB) *reinterpret_cast<u4*>(vst + 16 * lane) = L.vh;
      if (16 * lane < (int)SL::VLB) *reinterpret_cast<u4*>(vst + SL::VHB + 16 * lane) = L.vl;
    }
    float nk[NS], nv[NS];
#pragma unroll
    for (int t = 0; t < 2 / TS; ++t) {
      const float4 k4 = *reinterpret_cast<const float4*>(nst + 64 * (t + tile) + 16 * q4);
      const float4 v4 = *reinterpret_cast<const float4*>(nst + 128 + 64 * (t + tile) + 16 * q4);
      nk[4 * t] = k4.x; nk[4 * t + 1] = k4.y; nk[4 * t + 2] = k4.z; nk[4 * t + 3] = k4.w;
      nv[4 * t] = v4.x; nv[4 * t + 1] = v4.y; nv[4 * t + 2] = v4.z; nv[4 * t + 3] = v4.w;
    }
    // ---- scores: steps 0-3 over the hi dims, 4-7 over the lo dims
    f4 sA = {0.f, 0.f, 0.f, 0.f}, sB = {0.f, 0.f, 0.f, 0.f};
    u2 ka[2], kb2[2];  // the lane's segments of tokens r, 16 + r, as 64-bit values from bit 0
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      ka[t] = L.kh[t];
      kb2[t] = L.kl[t];
      if constexpr (KH == 3) {
        const uint32_t sh = 8 * ((6 * q4) & 3);
        ka[t] = u2{__builtin_amdgcn_alignbit(L.kh[t][1], L.kh[t][0], sh), L.kh[t][1] >> sh};
      }
      if constexpr (KL == 3) {
        const uint32_t sh = 8 * ((6 * q4) & 3);
        kb2[t] = u2{__builtin_amdgcn_alignbit(L.kl[t][1], L.kl[t][0], sh), L.kl[t][1] >> sh};
      }
    }
    auto kstep = [&](const u2& seg, uint32_t T, auto W_c, auto S_c) -> u4 {
      constexpr int W = decltype(W_c)::value, S = decltype(S_c)::value;
      const u2 e0 = lds_u2(smem, taddr(T, bits64<2 * W * (2 * S), 2 * W>(seg)));
      const u2 e1 = lds_u2(smem, taddr(T, bits64<2 * W * (2 * S + 1), 2 * W>(seg)));
      return u4{e0[0], e0[1], e1[0], e1[1]};
    };
#define TQ_SPLIT_STEP(S)                                                                                         \
    {                                                                                                             \
      const u4 aA = kstep(ka[0], SL::kht, std::integral_constant<int, KH>{}, std::integral_constant<int, S>{});  \
      const u4 aB = kstep(ka[1], SL::kht, std::integral_constant<int, KH>{}, std::integral_constant<int, S>{});  \
      sA = mfma(as_h8(aA), qop[S], sA);                                                                           \
      sB = mfma(as_h8(aB), qop[S], sB);                                                                           \
    }
#define TQ_SPLIT_STEP_LO(S)                                                                                      \
    {                                                                                                             \
      const u4 aA = kstep(kb2[0], SL::klt, std::integral_constant<int, KL>{}, std::integral_constant<int, S>{}); \
      const u4 aB = kstep(kb2[1], SL::klt, std::integral_constant<int, KL>{}, std::integral_constant<int, S>{}); \
      sA = mfma(as_h8(aA), qop[4 + S], sA);                                                                       \
      sB = mfma(as_h8(aB), qop[4 + S], sB);                                                                       \
    }
    TQ_SPLIT_STEP(0) TQ_SPLIT_STEP(1) TQ_SPLIT_STEP(2) TQ_SPLIT_STEP(3)
    TQ_SPLIT_STEP_LO(0) TQ_SPLIT_STEP_LO(1) TQ_SPLIT_STEP_LO(2) TQ_SPLIT_STEP_LO(3)
#undef TQ_SPLIT_STEP
#undef TQ_SPLIT_STEP_LO
    float sc[NS];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (TS == 2) {
        const float sv = tile ? sB[i] : sA[i];
        sc[i] = (sv + partner<G>(sv)) * (nk[i] * qe_scale);
      } else {
        sc[i] = (sA[i] + partner<G>(sA[i])) * (nk[i] * qe_scale);
        sc[4 + i] = (sB[i] + partner<G>(sB[i])) * (nk[4 + i] * qe_scale);
      }
    }
    if (t0 + 32 > tend) {
#pragma unroll
      for (int i = 0; i < NS; ++i)
        if (t0 + 16 * (tile + (i >> 2)) + 4 * q4 + (i & 3) >= tend) sc[i] = -INFINITY;
    }
    const half8 pb = softmax_pv(sc, nv, acc_r, true);
    // ---- V^T operands: token pair j = tokens (2 j, 2 j + 1) of the lane's
    // eight (A0..A3 = 4 q4 + i, B0..B3 = 16 + 4 q4 + i); MFMA nb reads
    // segment nb >> 2, dim nb & 3 of the lane's four (field (nb & 3) >> 1)
    u4 va[8], vl[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int tx = j < 2 ? 4 * q4 + 2 * j : 16 + 4 * q4 + 2 * (j - 2);
      const uint32_t hx = vcode(vst, VH, SL::VRH, tx), hy = vcode(vst, VH, SL::VRH, tx + 1);
      const uint32_t lx = vcode(vst + SL::VLO, VL, SL::VRL, tx), ly = vcode(vst + SL::VLO, VL, SL::VRL, tx + 1);
      u2 ex[4], ey[4];
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        ex[f] = lds_u2(smem, taddr(SL::vht, (hx >> (2 * VH * f)) & ((1u << (2 * VH)) - 1u)));
        ey[f] = lds_u2(smem, taddr(SL::vht, (hy >> (2 * VH * f)) & ((1u << (2 * VH)) - 1u)));
        ex[2 + f] = lds_u2(smem, taddr(SL::vlt, (lx >> (2 * VL * f)) & ((1u << (2 * VL)) - 1u)));
        ey[2 + f] = lds_u2(smem, taddr(SL::vlt, (ly >> (2 * VL * f)) & ((1u << (2 * VL)) - 1u)));
      }
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) {
        const int f = 2 * (nb >> 2) + ((nb & 3) >> 1);
        const uint32_t sel = (nb & 1) ? 0x07060302u : 0x05040100u;
        va[nb][j] = __builtin_amdgcn_perm(ey[f][0], ex[f][0], sel);
        vl[nb][j] = __builtin_amdgcn_perm(ey[f][1], ex[f][1], sel);
      }
    }
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
      acc_r[nb] = mfma(as_h8(va[nb]), pb, acc_r[nb]);
      acc_r[nb] = mfma(as_h8(vl[nb]), pb, acc_r[nb]);
    }
  }

  // ---- combine the 8 waves (as in the uniform kernel); the rotated dim of
  // accumulator (nb, i) of lane (column r, q4) is 64 (nb >> 2) + 16 q4 + 4 i
  // + (nb & 3)
  l_run = rows_sum(l_run);
  float tsc = __builtin_amdgcn_ldexpf(1.f, vx);
  if constexpr (TS == 2) {
    const float m2 = fmaxf(m_run, row_ror<8>(m_run));
    const float t = fexp2(m_run - m2);
    tsc *= t;
    l_run *= t;
    l_run += row_ror<8>(l_run);
    m_run = m2;
  }
  __syncthreads();
  float* cm = reinterpret_cast<float*>(smem + Layout::cmb) + (w * 8) * CMS;
  float* cl = reinterpret_cast<float*>(smem + Layout::cml) + w * 32;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float vr[8];
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
      float x = (acc_r[nb][i] + partner<G>(acc_r[nb][i])) * tsc;
      if constexpr (TS == 2) x += row_ror<8>(x);
      vr[nb] = x;
    }
    if (writer && tile == 0) {
      float* d = cm + hd * CMS + 16 * q4 + 4 * i;
      *reinterpret_cast<float4*>(d) = make_float4(vr[0], vr[1], vr[2], vr[3]);
      *reinterpret_cast<float4*>(d + 64) = make_float4(vr[4], vr[5], vr[6], vr[7]);
    }
  }
  if (q4 == 0 && writer && tile == 0) *reinterpret_cast<float4*>(cl + 4 * hd) = make_float4(m_run, l_run, m_orig, 0.f);
  __syncthreads();
  float* part = a.part + ((int64_t)row * a.nwg + c) * G * PPS;
  const bool wg_has_fp16 = nf > 0;
  {
    const float* cms = reinterpret_cast<const float*>(smem + Layout::cmb);
    const float* cls = reinterpret_cast<const float*>(smem + Layout::cml);
    const float* opk = reinterpret_cast<const float*>(smem + Layout::opk);
    for (int e = tid; e < G * FD; e += FT) {
      const int h = e / FD, j = e % FD;
      float M = M_INIT;
#pragma unroll
      for (int ww = 0; ww < FW; ++ww) M = fmaxf(M, cls[ww * 32 + 4 * h]);
      float sr = 0.f, L = 0.f;
#pragma unroll
      for (int ww = 0; ww < FW; ++ww) {
        const float4 st = *reinterpret_cast<const float4*>(cls + ww * 32 + 4 * h);
        const float sc = fexp2(st.x - M);
        sr = fmaf(sc, cms[(ww * 8 + h) * CMS + j], sr);
        L = fmaf(sc, st.y, L);
      }
      const float inv = L > 0.f ? 1.f / L : 0.f;
      part[h * PPS + P_OUT + j] = sr * inv * a.vscale;
      if (wg_has_fp16) {
        const float mo = cls[WF16 * 32 + 4 * h + 2];
        const float so = mo > M_INIT ? fexp2(mo - M) * opk[h * FD + j] : 0.f;
        part[h * PPS + P_OUT + FD + j] = so * inv;
      }
      if (j == 0) *reinterpret_cast<float4*>(part + h * PPS) = make_float4(M, L, wg_has_fp16 ? 1.f : 0.f, 0.f);
    }
  }
}

}  // namespace uk
}  // namespace tq

namespace tq {

// Host side: launch the split kernel (+ merge) for one (key, value) width
// pair; a side is (H, L, I): hi / lo bits and whether it is integer.
template <int G, int KH, int KL, bool KI, int VH, int VL, bool VI>
inline void launch_split_g(const UniformArgs& a, int merge, hipStream_t s) {
  if (a.bpw > FAST_WAVES * 4)
    hipLaunchKernelGGL((uk::split_decode_kernel<G, 8, KH, KL, VH, VL, KI, VI>), dim3(a.nwg, a.hkv, a.batch),
                       dim3(uk::FT), 0, s, a);
  else
    hipLaunchKernelGGL((uk::split_decode_kernel<G, 4, KH, KL, VH, VL, KI, VI>), dim3(a.nwg, a.hkv, a.batch),
                       dim3(uk::FT), 0, s, a);
  if (merge) hipLaunchKernelGGL((uk::uniform_merge_kernel<G>), dim3(a.hq, a.batch), dim3(uk::MT), 0, s, a);
}

template <int KH, int KL, bool KI, int VH, int VL, bool VI>
inline int launch_split_kv(const UniformArgs& a, int G, int merge, hipStream_t s) {
  switch (G) {
    case 1: launch_split_g<1, KH, KL, KI, VH, VL, VI>(a, merge, s); break;
    case 2: launch_split_g<2, KH, KL, KI, VH, VL, VI>(a, merge, s); break;
    case 4: launch_split_g<4, KH, KL, KI, VH, VL, VI>(a, merge, s); break;
    case 8: launch_split_g<8, KH, KL, KI, VH, VL, VI>(a, merge, s); break;
    default: return -1;
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// width kinds of one side: 7 = 3.5 bits (4 / 3), 5 = 2.5 (3 / 2), 2 / 3 / 4 integer
template <int KH, int KL, bool KI>
inline int launch_split_v(const UniformArgs& a, int G, int vkind, int merge, hipStream_t s) {
  switch (vkind) {
    case 7: return launch_split_kv<KH, KL, KI, 4, 3, false>(a, G, merge, s);
    case 5: return launch_split_kv<KH, KL, KI, 3, 2, false>(a, G, merge, s);
    default: break;
  }
  if constexpr (!KI) {  // integer values with fractional keys only
    switch (vkind) {
      case 2: return launch_split_kv<KH, KL, KI, 2, 2, true>(a, G, merge, s);
      case 3: return launch_split_kv<KH, KL, KI, 3, 3, true>(a, G, merge, s);
      case 4: return launch_split_kv<KH, KL, KI, 4, 4, true>(a, G, merge, s);
      default: break;
    }
  }
  return -1;
}

// one per key kind, each in its own translation unit (tq_decode_split*.hip)
int launch_split_k7(const UniformArgs& a, int G, int vkind, int merge, hipStream_t s);
int launch_split_k5(const UniformArgs& a, int G, int vkind, int merge, hipStream_t s);
int launch_split_ki(const UniformArgs& a, int G, int kkind, int vkind, int merge, hipStream_t s);

}  // namespace tq
