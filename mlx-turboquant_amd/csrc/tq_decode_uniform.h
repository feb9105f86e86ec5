// Fused decode attention for K4/V2 TurboQuant caches on gfx950, uniform
// batches (every sequence at the call's maximal lengths; a per-sequence ring
// start is allowed): a partials kernel over a fixed grid and a small merge
// kernel. Ragged batches take the persistent kernel of tq_decode_fast.hip.
//
// Grid (nwg, hkv, batch): workgroup c of (sequence b, kv head g) owns
//  - the compressed 32-token blocks [c*bpw, (c+1)*bpw) of the sequence (bpw <=
//    8 NPW, NPW = 4 or 8): wave w takes blocks c*bpw + w + 8k, k < NPW, with
//    two blocks' loads in flight while it computes;
//  - the fp16 tokens [c*fpw, (c+1)*fpw) (fpw <= 16) of the sequence's [sink |
//    residual ring] list, staged in LDS during set-up and scored by wave 0
//    (the first to be issued on its SIMD) before its compressed blocks.
//
// Scores are computed transposed, S^T = K q^T (MFMA 16x16x32 f16):
//   A = 16 tokens x 32 k-slots of keys, B = 32 k-slots x 16 columns of queries.
// A block of 32 tokens is two 16-token tiles. For G <= 4 the 16 columns are
// two groups of 8, group t serving tile t: column c8 of a group holds the
// fp16 high part of query head c8 % G (c8 < 4) or the remainder of head
// (7 - c8) % G, so a DPP row half-mirror (c8 <-> 7 - c8) adds the two parts,
// and each lane goes on with the 4 scores of its own tile only. For G = 8
// column r holds part r >> 3 of head r & 7 (a rotation by 8 pairs them) and
// every lane sees both tiles. In rotated space (compressed tokens,
// docs/FUSED_ATTENTION_DESIGN.md:62-67) each key code byte (two 4-bit codes)
// is looked up in an LDS table whose 8-byte entry is (c_hi[a], c_hi[b],
// c_lo[a], c_lo[b]); two lookups fill one A operand, and the matching B
// k-slots repeat the two query values, so
//   sum_k A B = sum_d (c_hi + c_lo)[idx_d] q_d   with c_lo = c - fp16(c).
// Scaled by the key norm and run through an online softmax in base 2.
// Output, transposed too: O^T += V^T P^T with A = 16 dims x 32 tokens of
// values decoded from an LDS table indexed by one 2-bit-code byte (4 dims of
// one token; the codec's exact fp16 value table, centroid = value_scale x
// entry) and paired across tokens with v_perm, and B = p * n_v split into
// fp16 high part / remainder along the same columns as the scores (zero in
// the k-slots of the other tile). Both tables come from the codecs' decode
// tables (tq_codec.decode_table), one 8-byte entry per code byte.
// fp16 tokens (original space) use the same MFMAs with exact fp16 keys /
// values, accumulated separately.
//
// Lane (column r, group q4) of a score tile holds tokens 4*q4 + i of the
// tile, which is exactly the k-slot order (8*q4 + i, tile 1 at + 4) the P^T
// operand needs, so softmax weights never leave their lane. The running max
// is raised with a margin, so most blocks need no rescale. The accumulator of
// lane (column r, q4), MFMA nb, register i is rotated dim 32*q4 + 8*i + nb.
//
// The 8 waves of a workgroup are combined through LDS into one partial per
// query head: (max, sum, rotated sum / sum, original-space sum / sum). The
// merge kernel combines the partials of each (b, g) with their softmax
// weights and applies the inverse rotation (the value codec's float32 R) once
// per query head.
//
// Other integer widths (KB, VB in 2..4, tq_decode_widths.hip) keep the
// structure: a key table entry holds 2 dims (fp16 high part / remainder pair)
// of a 2 KB-bit field, fields taken from the lane's 4 KB-byte segment with
// shifts (funnel shifts where a 3-bit field straddles a dword); 2-bit values
// keep the exact table; 3- and 4-bit values use a pair table with fp16 high
// part / remainder entries and two PV MFMAs per dim (value centroids are not
// fp16 numbers), their 8 VB bits per token loaded as one dword (two for 3 bits).

//
// This header holds the kernel templates (key width KB, value width VB);
// tq_decode_uniform.hip instantiates the K4/V2 kernels and
// tq_decode_widths.hip the other integer widths.
#pragma once

#include <math.h>
#include <stddef.h>

#include <type_traits>

#include "tq_common.h"
#include "tq_decode_fast.h"

namespace tq {
namespace uk {  // the uniform-batch kernels and their helpers

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef uint32_t u3 __attribute__((ext_vector_type(3)));
typedef __fp16 hx2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int FD = 128;
constexpr int FW = FAST_WAVES;            // waves per workgroup (FW * 16 == FD)
constexpr int FT = FW * 64;               // threads
constexpr int PPS = PACKED_PART_FLOATS;   // floats per (workgroup, head) partial
constexpr int P_OUT = 4;                  // partial: [M, L, has_orig, pad, rotated out[128], original out[128]]
constexpr int MAXWG = UNI_MAX_WG;         // workgroups per (sequence, kv head)
constexpr int FROW = 272;                 // LDS row of a staged fp16 token (256 + 16 against bank conflicts)
constexpr float M_INIT = -1e30f;          // running max before the first block
constexpr int WF16 = 0;                   // the wave that scores the staged fp16 tokens
constexpr int NCP = 32;                   // table replicas per entry (lane % 32: one per lane of an LDS pass)
// A block whose max exceeds the running max m raises m to that max + this
// margin (base-2 units), so later blocks rarely trigger a rescale; weights
// stay <= 1.
constexpr float RESCALE_MARGIN = 3.f;
// p * n_v above this is scaled down by a power of two (fp16 operand range);
// the column's exponent is applied at the combine.
constexpr float PV_LIMIT = 32768.f;
// the first non-empty compressed block of a column sets its exponent so that
// its largest p * n_v lands in (PV_SET / 2, PV_SET], up or down: small value
// norms keep fp16 remainders normal, and later blocks (p up to 8x the first
// block's, the rescale margin) stay below PV_LIMIT unless their norms grow
constexpr float PV_SET = 2048.f;
// |scale * (R q)_j| <= scale * ||q|| must stay below this for the fp16 query
// operands; larger queries are scaled by a power of two per head.
constexpr float Q_LIMIT = 16384.f;
// scale * ||q|| below this: the head is scaled up by a power of two (keeps
// the fp16 remainders of the rotated query normal)
constexpr float Q_LOW = 0.25f;

struct Layout {
  // Lookup tables: value entry e (four 2-bit codes) and key entry e (two
  // 4-bit codes) each in a 256-byte row of 32 replicas, replica c at 8*c, so
  // the LDS address of an entry is one byte permute of the code word. Once
  // every wave is past its blocks the table region holds the combine buffers.
  static constexpr uint32_t vlut = 0;            // 256 rows x 256 B
  static constexpr uint32_t klut = 65536;        // 256 rows x 256 B
  static constexpr uint32_t cmb = 0;             // [8 waves][8 heads][CMS] f32
  static constexpr uint32_t cml = 131072;        // [8 waves][8 heads][4] f32 max, sum, max of the orig part
  static constexpr uint32_t qop = cml + 1024;    // [8 heads][2 parts][QOPS bytes: 4][8][8] fp16 rotated-q B operands
  static constexpr uint32_t qfo = qop + 16 * 528; // [8 heads][2 parts][4][4][8] fp16 original-space q B operands
  static constexpr uint32_t opk = qfo + 4096;    // [8 heads][128] f32 parked original-space partial
  static constexpr uint32_t nst = opk + 4096;    // [8 waves][64] f32 norm staging
  static constexpr uint32_t qst = nst + 2048;    // [8 heads][128] q as given (up to 4 bytes per element)
  static constexpr uint32_t f16s = qst + 4096;   // [16 tokens][keys, values][FROW] staged fp16 tokens
  static constexpr uint32_t total = f16s + UNI_FP16_PER_WG * 2 * FROW;
};
// Row strides padded so that rows read by different lanes of one LDS
// instruction start in different banks: the rotated-q operand rows of the 8
// (head, part) columns, the combine rows of the G heads.
constexpr uint32_t QOPS = 528;  // bytes per (head, part) of qop (512 + 16)
constexpr int CMS = FD + 4;     // floats per (wave, head) of cmb
static_assert(FW * 8 * CMS * 4 <= Layout::cml, "combine buffers fit the table region");
static_assert(Layout::total <= 160 * 1024, "LDS of one workgroup");
static_assert(UNI_FP16_PER_WG == 16, "fp16 tokens: one 16-token score tile, one staging pass");

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

// the value of the column holding the other fp16 part of the same query head
// (and tile): row half-mirror for G <= 4, rotation by 8 for G = 8
template <int G>
__device__ inline float partner(float v) {
  if constexpr (G <= 4)
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, true));
  else
    return row_ror<8>(v);
}

__device__ inline uint32_t pk_rtz(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
}

__device__ inline u2 lds_u2(const uint8_t* smem, uint32_t addr) {
  return *reinterpret_cast<const u2*>(smem + addr);
}


// max / sum over the wave: DPP rotations within each 16-lane row, then the
// four rows
__device__ inline float wave_max(float v) {
  v = fmaxf(v, row_ror<8>(v));
  v = fmaxf(v, row_ror<4>(v));
  v = fmaxf(v, row_ror<2>(v));
  v = fmaxf(v, row_ror<1>(v));
  return rows_max(v);
}

__device__ inline float wave_sum(float v) {
  v += row_ror<8>(v);
  v += row_ror<4>(v);
  v += row_ror<2>(v);
  v += row_ror<1>(v);
  return rows_sum(v);
}

// The compressed blocks of one wave: loads issued at kernel start (lane r, q4)
template <int VB>
struct Blk {
  u4 k0, k1;      // key codes of tokens t0 + r and t0 + 16 + r: dims 32*q4 .. + 31 (4 KB bytes from byte 4 KB q4)
  uint32_t v[8];  // value codes of dims 8r .. 8r + 7 (8 VB bits) of tokens A0..A3 (t0 + 4q4 + i), B0..B3 (t0 + 16 + 4q4 + i)
  uint32_t vx[VB == 3 ? 8 : 1];  // VB = 3: the dword after v[i] (the 24 bits may straddle two)
  float nk, nv;   // key / value norm of token t0 + (lane & 31)
};

// max over the 64 lanes of a wave (unsigned), every lane gets it
__device__ inline uint32_t wave_max_u32(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x124, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x122, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x121, 0xF, 0xF, true));
  const auto x = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = max(x[0], x[1]);
  const auto y = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return max(y[0], y[1]);
}

// 8 bf16 values (bits) -> 8 fp16 values of x * s (s a power of two that keeps
// them in the fp16 range: exact for every scaled value in fp16's normal range)
__device__ inline u4 bf16_to_f16(u4 x, float s) {
  u4 o;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float lo = __uint_as_float(x[j] << 16) * s, hi = __uint_as_float(x[j] & 0xFFFF0000u) * s;
    o[j] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
  }
  return o;
}

// The 4-row stores of a pair table by wave w (B-bit codes: entry e of 2B bits
// -> (c_hi[e & M], c_hi[e >> B], c_lo[e & M], c_lo[e >> B]) fp16, M = 2^B - 1,
// c[i] = fp16 bits of c_hi[i] | c_lo[i] << 16, rows of 32 replicas): store sx
// fills rows 4 sx .. 4 sx + 3 with one 16-byte store (two replicas) per lane,
// lane l entry 4 sx + (l >> 4), replicas 2 (l & 15) and 2 (l & 15) + 1; of e
// only e & 3 varies over the lanes. sel4 picks x[l >> 4]; cb holds the second
// centroids of the wave's stores (c[2w], c[2w + 1] for B = 4, c[w] below).
template <int B, typename Sel>
__device__ inline void pair_table(uint8_t* tab, int w, int lane, const uint32_t (&c)[16], const uint32_t (&cb)[2],
                                  Sel sel4) {
  constexpr int NST = (1 << (2 * B)) / 4;       // stores: 64 / 16 / 4 for B = 4 / 3 / 2
  constexpr int SPW = NST >= 8 ? NST / 8 : 1;  // per wave (waves 0 .. 3 for B = 2)
  constexpr int MQ = ((1 << B) - 1) >> 2;      // e & M = 4 (k & MQ) + (l >> 4), e >> B = sx >> (B - 2)
  if (NST < 8 && w >= NST) return;
#pragma unroll
  for (int k = 0; k < SPW; ++k) {
    const int sx = NST >= 8 ? SPW * w + k : w;
    const int q = 4 * (k & MQ);
    const uint32_t ca = sel4(c[q], c[q + 1], c[q + 2], c[q + 3]);
    const uint32_t cbv = B == 4 ? cb[k >> 2] : cb[0];
    const uint32_t k0 = __builtin_amdgcn_perm(cbv, ca, 0x05040100u);  // (c_hi[e & M], c_hi[e >> B])
    const uint32_t k1 = __builtin_amdgcn_perm(cbv, ca, 0x07060302u);  // (c_lo[e & M], c_lo[e >> B])
    *reinterpret_cast<u4*>(tab + sx * 1024 + lane * 16) = u4{k0, k1, k0, k1};
  }
}

// Raw buffer over `bytes` bytes at p (stride 0): loads past the end read zero.
__device__ inline __amdgpu_buffer_rsrc_t rsrc(const void* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, bytes, 0x00020000);
}

// NPW: compressed blocks per wave (4, or 8 for long contexts and large
// batches, where fewer workgroups pay the set-up and combine)
template <int G, bool QB, int NPW, int KB = 4, int VB = 2, bool BF = false>
__global__ __launch_bounds__(FT) void uniform_decode_kernel(UniformArgs a) {
  static_assert(KB >= 2 && KB <= 4 && VB >= 2 && VB <= 4, "integer widths 2-4");
  static_assert(!QB || (KB == 4 && VB == 2), "the QJL key term runs with K4/V2");
  constexpr bool K4V2 = KB == 4 && VB == 2;
  constexpr int NKC = 1 << KB, NVC = VB == 2 ? 4 : 1 << VB;  // codebook words held (value: table or hi/lo pairs)
  __shared__ __align__(16) uint8_t smem[Layout::total];

  const int c = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, q4 = lane >> 4;
  const int row = b * a.hkv + g;
  const int j0 = 16 * w;  // output-dim tile of this wave for the query rotation
  constexpr int TS = G <= 4 ? 2 : 1;  // tiles sharing the columns
  constexpr int NS = 8 / TS;           // scores per lane per block
  const int tile = TS == 2 ? r >> 3 : 0;  // tile of column r (TS == 2)
  const int c8 = r & 7;
  const int hd = TS == 2 ? (c8 < 4 ? c8 : 7 - c8) % G : c8;  // query head of column r
  const bool lo_part = TS == 2 ? c8 >= 4 : r >= 8;          // column holds the fp16 remainder
  const float partf = lo_part ? 1.f : 0.f;
  const bool writer = !lo_part && c8 < G;  // one column per (tile, head) writes the combine rows

  // All kernel arguments the set-up needs are loaded in one batch of scalar
  // loads and waited for once; the set-up below has no branch on them, which
  // would split them into dependent round trips (the compiler reloads kernel
  // arguments inside branches).
  {
    const void* p4 = a.kc; const void* p5 = a.kn; const void* p6 = a.vc; const void* p7 = a.vn;
    const void* p8 = a.q; const void* p9 = a.rot16; const void* p10 = a.vrot; const void* p11 = a.part;
    const void* p12 = a.sink_k; const void* p13 = a.sink_v; const void* p14 = a.res_k; const void* p15 = a.res_v;
    const void* p3 = a.res_start_b;
    const int64_t s0 = a.k_hs, s1 = a.kn_hs, s2 = a.v_hs, s3 = a.vn_hs, s4 = a.sink_hs, s5 = a.res_hs;
    const int i0 = a.max_comp, i1 = a.max_sink, i2 = a.max_res, i3 = a.res_start0, i4 = a.bpw, i5 = a.hkv,
              i6 = a.hq, i7 = a.q_dtype, i8 = a.fpw, i9 = a.res_cap;
    asm volatile("" ::"s"(p3), "s"(p4), "s"(p5), "s"(p6), "s"(p7), "s"(p8), "s"(p9), "s"(p10), "s"(p11),
                 "s"(p12), "s"(p13), "s"(p14), "s"(p15), "s"(s0), "s"(s1), "s"(s2), "s"(s3), "s"(s4), "s"(s5),
                 "s"(i0), "s"(i1), "s"(i2), "s"(i3), "s"(i4), "s"(i5), "s"(i6), "s"(i7), "s"(i8), "s"(i9));
  }
  // the codebook entries this wave's table rows share (e >> 4 = 2w + k / 4,
  // (e >> 2) & 3 and e >> 6 of row e = 32w + 4k + lane / 16), at uniform
  // offsets of the kernel arguments, with the ones every lane selects from
  typedef const __attribute__((address_space(4))) uint32_t* kptr;
  const auto* kargs = (const __attribute__((address_space(4))) uint8_t*)__builtin_amdgcn_kernarg_segment_ptr();
  const kptr khu = (kptr)(kargs + offsetof(UniformArgs, khl));
  const kptr vtu = (kptr)(kargs + offsetof(UniformArgs, vtab));
  const kptr vhu = (kptr)(kargs + offsetof(UniformArgs, vhl));
  // the second centroid (e >> B) of this wave's pair-table stores: 2w + k / 4
  // for 4-bit codes, w for 2- and 3-bit codes
  const uint32_t cbw[2] = {khu[KB == 4 ? 2 * w : w], khu[KB == 4 ? 2 * w + 1 : w]};
  const uint32_t vtw[3] = {VB == 2 ? vtu[(2 * w) & 3] : vhu[VB == 4 ? 2 * w : w],
                           VB == 2 ? vtu[(2 * w + 1) & 3] : vhu[VB == 4 ? 2 * w + 1 : w], vtu[w >> 1]};
  // the ring start of the sequence: its res_start_b entry, or res_start0 (one
  // scalar load from either address, no branch); clamped to the ring, so
  // every read stays inside it
  const kptr rsp = a.res_start_b ? (kptr)(a.res_start_b + b) : (kptr)(kargs + offsetof(UniformArgs, res_start0));
  const int rs_raw = (int)*rsp;
  // the codebooks as opaque register values (the compiler would otherwise
  // reload them from the kernel arguments, one round trip per reload)
  uint32_t kh[16], vt[VB == 2 ? 4 : 16];
  if constexpr (K4V2) {
#pragma unroll
    for (int i = 0; i < 16; ++i) kh[i] = a.khl[i];
#pragma unroll
    for (int i = 0; i < 4; ++i) vt[i] = a.vtab[i];
    asm volatile("" : "+s"(kh[0]), "+s"(kh[1]), "+s"(kh[2]), "+s"(kh[3]), "+s"(kh[4]), "+s"(kh[5]), "+s"(kh[6]),
                 "+s"(kh[7]), "+s"(kh[8]), "+s"(kh[9]), "+s"(kh[10]), "+s"(kh[11]), "+s"(kh[12]), "+s"(kh[13]),
                 "+s"(kh[14]), "+s"(kh[15]), "+s"(vt[0]), "+s"(vt[1]), "+s"(vt[2]), "+s"(vt[3])
                 : "s"(cbw[0]), "s"(cbw[1]), "s"(vtw[0]), "s"(vtw[1]), "s"(vtw[2]), "s"(rs_raw));
  } else {
    // the codes' centroids (2^KB key pairs; the value table or 2^VB value pairs)
#pragma unroll
    for (int i = 0; i < 16; ++i) kh[i] = i < NKC ? a.khl[i] : 0u;
#pragma unroll
    for (int i = 0; i < (VB == 2 ? 4 : 16); ++i) vt[i] = VB == 2 ? a.vtab[i] : (i < NVC ? a.vhl[i] : 0u);
#pragma unroll
    for (int i = 0; i < 16; ++i) asm volatile("" : "+s"(kh[i]));
#pragma unroll
    for (int i = 0; i < (VB == 2 ? 4 : 16); ++i) asm volatile("" : "+s"(vt[i]));
    asm volatile("" ::"s"(cbw[0]), "s"(cbw[1]), "s"(vtw[0]), "s"(vtw[1]), "s"(vtw[2]), "s"(rs_raw));
  }
  // K4/V2: a uniform call, every sequence at the maximal lengths; the other
  // widths also serve ragged calls: the sequence's lengths (one scalar load
  // each, from its array entry or the maximum), clamped to the maxima
  auto seq_len = [&](const int32_t* arr, size_t max_off, int mx) {
    if constexpr (K4V2) {
      return mx;
    } else {
      const kptr p = arr ? (kptr)(arr + b) : (kptr)(kargs + max_off);
      return min(max((int)*p, 0), mx);
    }
  };
  const int comp = seq_len(a.comp_len_b, offsetof(UniformArgs, max_comp), a.max_comp);
  const int sink = seq_len(a.sink_len_b, offsetof(UniformArgs, max_sink), a.max_sink);
  const int res = seq_len(a.res_len_b, offsetof(UniformArgs, max_res), a.max_res);
  const int rstart = min(max(rs_raw, 0), max(a.res_cap - 1, 0));
  const int nbc = (comp + 31) >> 5;
  const int blk0 = c * a.bpw, blk1 = min(blk0 + a.bpw, nbc);
  const int f0 = c * a.fpw, nf = max(0, min(a.fpw, sink + res - f0));  // fp16 tokens [f0, f0 + nf)

  // ---- set-up loads: decode-table entries, R rows, q and the staged fp16 tokens, issued
  // before any compressed block so this small set-up data is not queued
  // behind a GPU-wide flood of block loads. All loads are issued
  // unconditionally (past the data, from valid addresses) so the compiler's
  // memory-counter waits stay exact.
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
  // the G query rows of this kv head, staged in LDS as given: 16-byte chunk e
  // (threads past the rows re-read chunk 0)
  const int esz = a.q_dtype == TQ_F32 ? 4 : 2;
  const int qchunks = G * FD * esz / 16;
  u4 qld;
  {
    const uint8_t* qp = static_cast<const uint8_t*>(a.q) + ((int64_t)b * a.hq + g * G) * FD * esz;
    const int e = tid < qchunks ? tid : 0;
    qld = *reinterpret_cast<const u4*>(qp + 16 * e);
  }
  // fp16 tokens of this workgroup: 512 chunks of 16 bytes, chunk e = tid =
  // token slot e >> 5, keys ((e >> 4) & 1 == 0) or values, bytes 16*(e & 15)
  // of the row
  u4 fst;
  {
    const int e = tid;
    const int u = f0 + min(e >> 5, max(nf - 1, 0));  // token of the [sink | residual] list
    const bool is_v = (e >> 4) & 1;
    int sl = rstart + (u - sink);  // ring slot (rstart + t < 2 * res_cap)
    sl = sl >= a.res_cap ? sl - a.res_cap : sl;
    // candidate rows, selected without a branch; nothing staged: a dummy read
    const uint16_t* ps = static_cast<const uint16_t*>(is_v ? a.sink_v : a.sink_k) + (int64_t)row * a.sink_hs + (int64_t)u * FD;
    const uint16_t* pr = static_cast<const uint16_t*>(is_v ? a.res_v : a.res_k) + (int64_t)row * a.res_hs + (int64_t)sl * FD;
    const uint16_t* src = nf == 0 ? a.rot16 : (u < sink ? ps : pr);
    fst = *reinterpret_cast<const u4*>(src + 8 * (e & 15));
  }
  // ---- loads of the compressed blocks of this wave: blocks blk0 + w + 8k.
  // Buffer loads over the tokens [t0, comp) of the row: bytes past the
  // sequence read as zero (those tokens are masked), slots past the wave's
  // blocks re-read block 0 and are masked.
  // (with no compressed token every buffer has zero bytes: its loads read zero
  // and touch no memory, whatever the base)
  const uint8_t* kcodes = a.kc + (int64_t)row * a.k_hs;
  const uint8_t* vcodes = a.vc + (int64_t)row * a.v_hs;
  const float* knorm = a.kn + (int64_t)row * a.kn_hs;
  const float* vnorm = a.vn + (int64_t)row * a.vn_hs;
  auto slot_t0 = [&](int k) {
    const int blk = blk0 + w + FW * k;
    return blk < blk1 ? blk << 5 : 0;
  };
  // lane byte offsets within a block (rows of RK = 16 KB and RV = 16 VB
  // bytes): key bytes 4 KB q4 .. of token r (token 16 + r at + 16 RK); value
  // bits 8 VB r .. of token 4*q4 (token 4*q4 + i at + i RV, token 16 + 4*q4 +
  // i at + (16 + i) RV; VB = 3: the dword holding bit 24 r and the next);
  // norm of token lane & 31
  constexpr int RK = 16 * KB, RV = 16 * VB;
  const int ko = r * RK + 4 * KB * q4;
  const int vo = q4 * 4 * RV + (VB == 3 ? 4 * ((3 * r) >> 2) : VB * r);
  const int no = (lane & 31) * 4;
  Blk<VB> B[NPW];
  auto load_slot = [&](int k) {
    const int t0 = slot_t0(k);
    const int n = comp - t0;  // tokens readable from t0 on (t0 = 0 when comp = 0)
    const __amdgpu_buffer_rsrc_t rk = rsrc(kcodes + (int64_t)t0 * RK, n * RK);
    const __amdgpu_buffer_rsrc_t rv = rsrc(vcodes + (int64_t)t0 * RV, n * RV);
    const __amdgpu_buffer_rsrc_t rkn = rsrc(knorm + t0, n * 4);
    const __amdgpu_buffer_rsrc_t rvn = rsrc(vnorm + t0, n * 4);
    if constexpr (KB == 4) {
      B[k].k0 = __builtin_amdgcn_raw_buffer_load_b128(rk, ko, 0, 0);
      B[k].k1 = __builtin_amdgcn_raw_buffer_load_b128(rk, ko + 16 * RK, 0, 0);
    } else if constexpr (KB == 3) {
      const u3 x0 = __builtin_amdgcn_raw_buffer_load_b96(rk, ko, 0, 0);
      const u3 x1 = __builtin_amdgcn_raw_buffer_load_b96(rk, ko + 16 * RK, 0, 0);
      B[k].k0 = u4{x0[0], x0[1], x0[2], 0u};
      B[k].k1 = u4{x1[0], x1[1], x1[2], 0u};
    } else {
      const u2 x0 = __builtin_amdgcn_raw_buffer_load_b64(rk, ko, 0, 0);
      const u2 x1 = __builtin_amdgcn_raw_buffer_load_b64(rk, ko + 16 * RK, 0, 0);
      B[k].k0 = u4{x0[0], x0[1], 0u, 0u};
      B[k].k1 = u4{x1[0], x1[1], 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int off = vo + (i < 4 ? RV * i : 16 * RV + RV * (i - 4));
      if constexpr (VB == 2) {
        B[k].v[i] = __builtin_amdgcn_raw_buffer_load_b16(rv, off, 0, 0);
      } else if constexpr (VB == 4) {
        B[k].v[i] = __builtin_amdgcn_raw_buffer_load_b32(rv, off, 0, 0);
      } else {
        const u2 x = __builtin_amdgcn_raw_buffer_load_b64(rv, off, 0, 0);
        B[k].v[i] = x[0];
        B[k].vx[i] = x[1];
      }
    }
    B[k].nk = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rkn, no, 0, 0));
    B[k].nv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rvn, no, 0, 0));
  };
  // block 0 is requested right behind the set-up loads: waiting for those
  // does not wait for it
  load_slot(0);
  // ---- tables, from the codebooks passed by value (no memory round trip):
  // key byte e -> (c_hi[e&15], c_hi[e>>4], c_lo[e&15], c_lo[e>>4]) fp16
  //   (c_hi = fp16(c), c_lo = fp16(c - c_hi), as in tq_codec.decode_table;
  //   khl[i] holds the pair of centroid i)
  // value byte e -> (t[e&3], t[(e>>2)&3], t[(e>>4)&3], t[(e>>6)&3]) fp16
  // Store k of wave w fills rows 4s .. 4s + 3 (s = 8w + k) of a table with one
  // 16-byte store (two replicas) per lane, lane-linear and so conflict-free:
  // lane l writes entry e = 4s + (l >> 4), replicas 2(l & 15) and 2(l & 15) + 1.
  // Of e, only e & 3 = l >> 4 varies over the lanes.
  {
    // x[lane >> 4], by bit masks (a conditional form becomes divergent branches)
    const uint32_t m1 = 0u - ((uint32_t)lane >> 4 & 1u), m2 = 0u - ((uint32_t)lane >> 5 & 1u);
    auto sel4 = [&](uint32_t x0, uint32_t x1, uint32_t x2, uint32_t x3) {
      const uint32_t lo = (m1 & x1) | (~m1 & x0), hi = (m1 & x3) | (~m1 & x2);
      return (m2 & hi) | (~m2 & lo);
    };
    if constexpr (K4V2) {
      const uint32_t vq = sel4(vt[0], vt[1], vt[2], vt[3]);  // t[e & 3]
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int sx = 8 * w + k;  // uniform
        const uint32_t ka = sel4(kh[4 * (k & 3)], kh[4 * (k & 3) + 1], kh[4 * (k & 3) + 2],
                                 kh[4 * (k & 3) + 3]);  // centroid e & 15
        const uint32_t kb = cbw[k >> 2];                   // centroid e >> 4
        const uint32_t k0 = __builtin_amdgcn_perm(kb, ka, 0x05040100u);  // (c_hi[e&15], c_hi[e>>4])
        const uint32_t k1 = __builtin_amdgcn_perm(kb, ka, 0x07060302u);  // (c_lo[e&15], c_lo[e>>4])
        *reinterpret_cast<u4*>(smem + Layout::klut + sx * 1024 + lane * 16) = u4{k0, k1, k0, k1};
        const uint32_t v0 = vq | (vt[k & 3] << 16);
        const uint32_t v1 = vtw[k >> 2] | (vtw[2] << 16);  // t[(e >> 4) & 3], t[e >> 6]
        *reinterpret_cast<u4*>(smem + Layout::vlut + sx * 1024 + lane * 16) = u4{v0, v1, v0, v1};
      }
    } else {
      // other widths: a pair table of the key codes (2 dims per entry); the
      // 2-bit value table as above, or a pair table of the value codes
      // (fp16 high part / remainder, 2 dims per entry)
      const uint32_t cbk[2] = {cbw[0], cbw[1]};
      pair_table<KB>(smem + Layout::klut, w, lane, kh, cbk, sel4);
      if constexpr (VB == 2) {
        const uint32_t vq = sel4(vt[0], vt[1], vt[2], vt[3]);  // t[e & 3]
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const int sx = 8 * w + k;
          const uint32_t v0 = vq | (vt[k & 3] << 16);
          const uint32_t v1 = vtw[k >> 2] | (vtw[2] << 16);  // t[(e >> 4) & 3], t[e >> 6]
          *reinterpret_cast<u4*>(smem + Layout::vlut + sx * 1024 + lane * 16) = u4{v0, v1, v0, v1};
        }
      } else {
        const uint32_t cbv[2] = {vtw[0], vtw[1]};
        uint32_t vc16[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) vc16[i] = vt[i % (sizeof(vt) / sizeof(vt[0]))];
        pair_table<VB>(smem + Layout::vlut, w, lane, vc16, cbv, sel4);
      }
    }
  }
  if constexpr (BF) {
    // bf16 sink / ring tokens: the largest |x| of the staged keys and of the
    // staged values (bf16 bits, sign cleared), per wave into the combine
    // header region (free until the combine), for the fp16 scale of the tile
    uint32_t mx = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t x = fst[j] & 0x7FFF7FFFu;
      mx = max(mx, max(x & 0xFFFFu, x >> 16));
    }
    const bool isv = (tid >> 4) & 1;
    const uint32_t mk = wave_max_u32(isv ? 0u : mx), mv = wave_max_u32(isv ? mx : 0u);
    if (lane == 0) {
      uint32_t* bm = reinterpret_cast<uint32_t*>(smem + Layout::cml);
      bm[2 * w] = mk;
      bm[2 * w + 1] = mv;
    }
  }
  if (tid < qchunks) *reinterpret_cast<u4*>(smem + Layout::qst + 16 * tid) = qld;
  // staged fp16 tokens: [slot][keys | values][272-byte row]
  *reinterpret_cast<u4*>(smem + Layout::f16s + (tid >> 5) * (2 * FROW) + ((tid >> 4) & 1) * FROW + 16 * (tid & 15)) = fst;
  __syncthreads();

  // block 1 once the tables are built; block k + 2 as slot k starts
  load_slot(1);


  // q rows as MFMA A operands (row r = query head min(r, G-1), k-slots = dims
  // 32*kb + 8*q4 ..): fp16 high part and remainder of q 2^-qe, the power of
  // two 2^qe of the head keeping scale * |R q| <= scale * ||q|| below Q_LIMIT
  // and, for small queries, the rotated remainders normal
  half8 qo_hi[4], qo_lo[4];
  float qe_scale = 1.f;  // 2^qe of this lane's column head: multiplies its scores
  bool q_exact = false;  // the remainders qo_lo are zero
  {
    const uint8_t* qr = smem + Layout::qst + (uint32_t)min(r, G - 1) * FD * esz;
    if (a.q_dtype == TQ_F16) {
      // fp16 queries: the operands are the inputs themselves (remainder zero)
      // unless a head of the wave needs scaling down
      u4 raw[4];
      float ss = 0.f;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        raw[kb] = *reinterpret_cast<const u4*>(qr + 2 * (32 * kb + 8 * q4));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const f16x2 h = __builtin_bit_cast(f16x2, raw[kb][j]);
          ss = __builtin_amdgcn_fdot2(h, h, ss, false);
        }
      }
      ss = rows_sum(ss);
      // scale * ||q|| in [Q_LOW, Q_LIMIT] (query_exponent 0) for every head:
      // one unsigned range test of the float bits
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
      // the fp16 high part / remainder of q 2^-qe
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
      ss = rows_sum(ss);  // the 4 lanes of row r hold the 128 dims of its head
      const int qe = query_exponent(sqrtf(ss), a.qscale, Q_LIMIT, Q_LOW);  // lanes r: head min(r, G - 1)
      const float qdown = __builtin_amdgcn_ldexpf(1.f, -qe);
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float xs = x[kb][i] * qdown;
          qo_hi[kb][i] = (_Float16)xs;
          qo_lo[kb][i] = (_Float16)(xs - (float)qo_hi[kb][i]);
        }
      // lane h (column h, group 0) holds the exponent of head h
      int qeh = 0;
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const int xh = __builtin_amdgcn_readlane(qe, h);
        qeh = hd == h ? xh : qeh;
      }
      qe_scale = __builtin_amdgcn_ldexpf(1.f, qeh);
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
      if (!q_exact) dq = mfma(qo_lo[kb], as_h8(rqh[kb]), dq);
    }
    const int j = j0 + r, e = j & 3;
    const uint32_t off = ((uint32_t)(j >> 5) * 8 + ((j >> 2) & 7)) * 16 + 2 * ((e & 1) + 4 * (e >> 1));
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
  // fp16 tokens use the (unscaled, 2^-qe) q in original space as score B operands,
  // step kb k-slot (q4, i) = dim 32*q4 + 8*kb + i: fp16 high part / remainder
  // in [head][part][q4][kb][8 halves]; the lane holding dims 32*kb + 8*q4 ..
  // of head r copies its operand halves there
  if (w == 0 && r < G && nf > 0) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      uint8_t* d = smem + Layout::qfo + ((uint32_t)(r * 2 * 4 + kb) * 4 + q4) * 16;
      *reinterpret_cast<half8*>(d) = qo_hi[kb];
      *reinterpret_cast<half8*>(d + 4 * 4 * 16) = qo_lo[kb];
    }
  }
  __syncthreads();

  // ---- per-lane online softmax state of column r (head hd)
  float m_run = M_INIT, l_run = 0.f;
  int vx = 0;             // exponent of the column: acc_r holds the sums times 2^-vx
  bool vset = false;      // vx set by the wave's first non-empty compressed block (wave-uniform)
  float m_orig = M_INIT;  // running max the parked original-space partial refers to
  f4 acc_r[8];            // rotated-space output accumulators

  const uint32_t cp = (uint32_t)(lane & (NCP - 1)) * 8;  // replica offset within a table row
  static_assert(Layout::klut == 0x10000 && Layout::vlut == 0, "table addresses are byte permutes");
  const uint32_t cpk = cp | Layout::klut;
  auto kaddr = [&](uint32_t word, int byte) {      // klut + (byte of word) * 256 + cp: bytes (cp, code byte, 1, 0)
    return __builtin_amdgcn_perm(word, cpk, 0x0C020000u | ((4u + byte) << 8));
  };
  auto vaddr = [&](uint32_t word, int byte) {      // vlut + (byte of word) * 256 + cp
    return Layout::vlut + __builtin_amdgcn_perm(word, cp, 0x0C0C0000u | ((4u + byte) << 8));
  };

  // Online softmax of the NS scores of this lane (tokens A0..A3 and / or
  // B0..B3 of the block, column r), returns the P^T operand (p * nv 2^-vx,
  // high part or remainder by column, zero in the k-slots of the other tile)
  // and rescales `acc` when a block's max exceeds the running max, or when
  // p * nv would leave the fp16 range (the column exponent vx then grows);
  // with `setx` (compressed blocks) the first non-empty block sets vx.
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
    const bool first = setx && !vset;  // wave-uniform
    if (__builtin_amdgcn_ballot_w64(pmx > PV_LIMIT || (first && pmx > 0.f)) != 0) {
      const float cm = rows_max(pmx);  // max of the column
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

  // ---- the staged fp16 tokens (sink / residual ring, original space): wave
  // WF16, before its compressed blocks
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
    // bf16 tokens: keys and values scaled by powers of two 2^-ek, 2^-ev that
    // bring the tile's largest |x| into [2^14, 2^15): exact in fp16 down to
    // 2^-38 of it (fp16 subnormals below); the scores and the parked sums are
    // scaled back
    float ks = 1.f, vs = 1.f, kback = 1.f, vback = 1.f;
    if constexpr (BF) {
      const uint32_t* bm = reinterpret_cast<const uint32_t*>(smem + Layout::cml);
      uint32_t mk = 0, mv = 0;
#pragma unroll
      for (int ww = 0; ww < FW; ++ww) {
        mk = max(mk, bm[2 * ww]);
        mv = max(mv, bm[2 * ww + 1]);
      }
      // bf16 exponent field (bits 14..7) of the tile maxima; zero tiles keep 1
      const int ek = mk == 0u ? 0 : max(-100, (int)(mk >> 7) - 127 - 14);
      const int ev = mv == 0u ? 0 : max(-100, (int)(mv >> 7) - 127 - 14);
      ks = __builtin_amdgcn_ldexpf(1.f, -ek);
      vs = __builtin_amdgcn_ldexpf(1.f, -ev);
      kback = __builtin_amdgcn_ldexpf(1.f, ek);
      vback = __builtin_amdgcn_ldexpf(1.f, ev);
    }
    // one 16-token score tile (tokens r); the k-slots of tokens 16.. of the
    // P^T operand stay empty
    f4 sA = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      u4 kA = *reinterpret_cast<const u4*>(fs + r * (2 * FROW) + 64 * q4 + 16 * kb);
      if constexpr (BF) kA = bf16_to_f16(kA, ks);
      sA = mfma(as_h8(kA), qf[kb], sA);
    }
    float sc[NS], ones[NS];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float full = (sA[i] + partner<G>(sA[i])) * (a.qscale * qe_scale * kback);
      sc[i] = tile == 0 && 4 * q4 + i < nf ? full : -INFINITY;  // the tile-1 columns see no fp16 token
      if constexpr (NS == 8) sc[4 + i] = -INFINITY;
    }
#pragma unroll
    for (int i = 0; i < NS; ++i) ones[i] = 1.f;
    const half8 pb = softmax_pv(sc, ones, acc_o, false);
    u4 vv[8];  // values: dims 8r .. 8r+7 of tokens A0..A3 (k-slots of B0..B3 zero)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      vv[i] = i < 4 ? *reinterpret_cast<const u4*>(fs + (4 * q4 + i) * (2 * FROW) + FROW + 16 * r) : u4{0u, 0u, 0u, 0u};
      if constexpr (BF) vv[i] = bf16_to_f16(vv[i], vs);
    }
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
      const uint32_t sel = (nb & 1) ? 0x07060302u : 0x05040100u;
      u4 bv;
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[j] = __builtin_amdgcn_perm(vv[2 * j + 1][nb >> 1], vv[2 * j][nb >> 1], sel);
      acc_o[nb] = mfma(as_h8(bv), pb, acc_o[nb]);
    }
    // park the original-space partial (hi + lo columns summed) in LDS with the
    // running max it refers to; later blocks only rescale it at the combine
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float vo[8];
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) vo[nb] = (acc_o[nb][i] + partner<G>(acc_o[nb][i])) * vback;
      if (writer && tile == 0) {
        float* d = reinterpret_cast<float*>(smem + Layout::opk) + hd * FD + 32 * q4 + 8 * i;
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
  half8 qop[8];
  {
    const uint8_t* src = smem + Layout::qop + (uint32_t)(hd * 2 + (partf != 0.f ? 1 : 0)) * QOPS + (uint32_t)q4 * 128;
#pragma unroll
    for (int s = 0; s < 8; ++s) qop[s] = *reinterpret_cast<const half8*>(src + 16 * s);
  }
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) acc_r[nb] = f4{0.f, 0.f, 0.f, 0.f};

  static_assert(NPW >= 2, "two blocks in flight");

  // ---- the compressed blocks of this wave (rotated space)
  uint8_t* nst = smem + Layout::nst + w * 256;  // this wave's norm staging: [key norms 32][value norms 32]
#pragma unroll
  for (int k = 0; k < NPW; ++k) {
    // every slot is computed (no branch between them, so the scheduler can
    // overlap one block's lookups with the previous block's softmax); a slot
    // past the wave's blocks masks all its tokens. Block k + 2 is requested
    // as slot k starts, so two blocks stay in flight while slot k computes.
    if (k + 2 < NPW) load_slot(k + 2);
    const Blk<VB>& L = B[k];
    const int t0 = slot_t0(k);
    const int tend = blk0 + w + FW * k < blk1 ? comp : 0;
    *reinterpret_cast<float*>(nst + 4 * lane) = lane < 32 ? L.nk : L.nv;
    // key / value norms of the lane's tokens: tile `tile` (TS == 2) or both
    float nk[NS], nv[NS];
#pragma unroll
    for (int t = 0; t < 2 / TS; ++t) {
      const float4 k4 = *reinterpret_cast<const float4*>(nst + 64 * (t + tile) + 16 * q4);
      const float4 v4 = *reinterpret_cast<const float4*>(nst + 128 + 64 * (t + tile) + 16 * q4);
      nk[4 * t] = k4.x; nk[4 * t + 1] = k4.y; nk[4 * t + 2] = k4.z; nk[4 * t + 3] = k4.w;
      nv[4 * t] = v4.x; nv[4 * t + 1] = v4.y; nv[4 * t + 2] = v4.z; nv[4 * t + 3] = v4.w;
    }
    // V^T operands (row = dim 8r + nb, k-slot pairs = token pairs of the
    // lane), looked up first: they depend only on the codes, and their LDS
    // latency then overlaps the scores and the softmax
    u4 va[8];
#pragma unroll
    for (int j = 0; j < 4 && VB == 2; ++j) {
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
    f4 sA = {0.f, 0.f, 0.f, 0.f}, sB = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      u2 ea0, ea1, eb0, eb1;
      if constexpr (KB == 4) {
        const uint32_t wa = L.k0[s >> 1], wb = L.k1[s >> 1];
        const int by = 2 * (s & 1);
        ea0 = lds_u2(smem, kaddr(wa, by)), ea1 = lds_u2(smem, kaddr(wa, by + 1));
        eb0 = lds_u2(smem, kaddr(wb, by)), eb1 = lds_u2(smem, kaddr(wb, by + 1));
      } else {
        // fields 2s, 2s + 1 (2 KB bits each, dims 4s .. 4s + 3 of the segment)
        auto kfield = [&](const u4& seg, int f) {
          const int off = 2 * KB * f, wd = off >> 5, sh = off & 31;
          const uint32_t x =
              sh + 2 * KB <= 32 ? seg[wd] >> sh : __builtin_amdgcn_alignbit(seg[wd < 3 ? wd + 1 : 3], seg[wd], sh);
          return cpk | ((x & ((1u << (2 * KB)) - 1u)) << 8);
        };
        ea0 = lds_u2(smem, kfield(L.k0, 2 * s)), ea1 = lds_u2(smem, kfield(L.k0, 2 * s + 1));
        eb0 = lds_u2(smem, kfield(L.k1, 2 * s)), eb1 = lds_u2(smem, kfield(L.k1, 2 * s + 1));
      }
      sA = mfma(as_h8(u4{ea0[0], ea0[1], ea1[0], ea1[1]}), qop[s], sA);
      sB = mfma(as_h8(u4{eb0[0], eb0[1], eb1[0], eb1[1]}), qop[s], sB);
    }
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
    if constexpr (QB) {
      // QJL key term of the lane's tokens (tile `tile`, or both for TS == 1)
      const float* qb = a.qjl_bias + ((int64_t)row * G + hd) * a.qb_hs + t0 + 4 * q4;
#pragma unroll
      for (int t = 0; t < 2 / TS; ++t) {
        const float4 bb = *reinterpret_cast<const float4*>(qb + 16 * (t + tile));
        sc[4 * t] += bb.x; sc[4 * t + 1] += bb.y; sc[4 * t + 2] += bb.z; sc[4 * t + 3] += bb.w;
      }
    }
    if (t0 + 32 > tend) {  // uniform: only the last block of a sequence and empty slots mask
#pragma unroll
      for (int i = 0; i < NS; ++i)
        if (t0 + 16 * (tile + (i >> 2)) + 4 * q4 + (i & 3) >= tend) sc[i] = -INFINITY;
    }
    if constexpr (QB) {
      // the final scores of the compressed tokens, for the QJL value term
      if (tend > 0 && !lo_part && c8 < G) {
        float* so = a.scores + ((int64_t)row * G + hd) * a.qb_hs + t0 + 4 * q4;
#pragma unroll
        for (int t = 0; t < 2 / TS; ++t)
          *reinterpret_cast<float4*>(so + 16 * (t + tile)) = make_float4(sc[4 * t], sc[4 * t + 1], sc[4 * t + 2], sc[4 * t + 3]);
      }
    }
    const half8 pb = softmax_pv(sc, nv, acc_r, true);
    u4 vl[8];  // the remainders (value pair tables)
    if constexpr (VB != 2) {
      // built after the scores: fewer registers live across the score MFMAs
      // 2 dims per table entry (fp16 high part, remainder): field f of a
      // token's 8 VB bits holds dims 8r + 2f, 8r + 2f + 1
      auto vfield = [&](uint32_t x, int f) {
        if constexpr (VB == 4) return vaddr(x, f);
        else return Layout::vlut + ((((x >> (6 * f)) & 63u) << 8) | cp);
      };
      const uint32_t sh3 = (24u * (uint32_t)r) & 31u;  // VB = 3: bit of 24 r in its dword
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t px = L.v[2 * j], py = L.v[2 * j + 1];
        if constexpr (VB == 3) {
          px = __builtin_amdgcn_alignbit(L.vx[2 * j], px, sh3);
          py = __builtin_amdgcn_alignbit(L.vx[2 * j + 1], py, sh3);
        }
        u2 ex[4], ey[4];
#pragma unroll
        for (int f = 0; f < 4; ++f) {
          ex[f] = lds_u2(smem, vfield(px, f));
          ey[f] = lds_u2(smem, vfield(py, f));
        }
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) {
          const uint32_t sel = (nb & 1) ? 0x07060302u : 0x05040100u;
          va[nb][j] = __builtin_amdgcn_perm(ey[nb >> 1][0], ex[nb >> 1][0], sel);
          vl[nb][j] = __builtin_amdgcn_perm(ey[nb >> 1][1], ex[nb >> 1][1], sel);
        }
      }
    }
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
      acc_r[nb] = mfma(as_h8(va[nb]), pb, acc_r[nb]);
      if constexpr (VB != 2) acc_r[nb] = mfma(as_h8(vl[nb]), pb, acc_r[nb]);
    }
  }

  // ---- combine the 8 waves of this workgroup through LDS (the table region,
  // free once every wave is past its blocks). The two fp16 parts of a (tile,
  // head) meet through `partner`; for TS == 2 the two tiles of a head (columns
  // r and r ^ 8) are then merged at their common max by a rotation by 8, and
  // the high-part column of tile 0 writes the head's row.
  l_run = rows_sum(l_run);
  float tsc = __builtin_amdgcn_ldexpf(1.f, vx);  // scale of this lane's sums to the merged max
  if constexpr (TS == 2) {
    const float m2 = fmaxf(m_run, row_ror<8>(m_run));
    const float t = fexp2(m_run - m2);
    tsc *= t;
    l_run *= t;
    l_run += row_ror<8>(l_run);
    m_run = m2;
  }
  __syncthreads();
  float* cm = reinterpret_cast<float*>(smem + Layout::cmb) + (w * 8) * CMS;  // [wave][head][CMS]
  float* cl = reinterpret_cast<float*>(smem + Layout::cml) + w * 32;        // [wave][head][4]
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
      float* d = cm + hd * CMS + 32 * q4 + 8 * i;
      *reinterpret_cast<float4*>(d) = make_float4(vr[0], vr[1], vr[2], vr[3]);
      *reinterpret_cast<float4*>(d + 4) = make_float4(vr[4], vr[5], vr[6], vr[7]);
    }
  }
  if (q4 == 0 && writer && tile == 0) *reinterpret_cast<float4*>(cl + 4 * hd) = make_float4(m_run, l_run, m_orig, 0.f);
  __syncthreads();
  // thread (head, dim): merge the 8 waves into the workgroup's rotated sum
  // (times the value scale) and original-space sum at the workgroup max M,
  // both divided by the workgroup sum L, straight into the partial; the
  // merge kernel applies the inverse rotation once per query head
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
        // original-space part of wave WF16, parked at its max then
        const float mo = cls[WF16 * 32 + 4 * h + 2];
        const float so = mo > M_INIT ? fexp2(mo - M) * opk[h * FD + j] : 0.f;
        part[h * PPS + P_OUT + FD + j] = so * inv;
      }
      if (j == 0) *reinterpret_cast<float4*>(part + h * PPS) = make_float4(M, L, wg_has_fp16 ? 1.f : 0.f, 0.f);
    }
  }
}

// Merge of the partials of (sequence b, kv head g), a second launch on the
// same stream (the kernel boundary makes the partials visible), in float32
// (docs/FULL_FUSED_ATTENTION_RESULTS.md:34-40). Partial p holds its max M_p,
// its sum L_p, its rotated output y_p and (flag f_p) its original-space
// output x_p, both normalised by L_p:
//   out = (sum_p w_p y_p) @ R + sum_p w_p f_p x_p,  w_p = 2^(M_p - M) L_p / L,
//   M = max_p M_p,  L = sum_p 2^(M_p - M) L_p,
// with R the value codec's float32 rotation (x = R^T y). One workgroup of 256
// threads per (query head, b): thread t sums dim t & 127 of the partials of
// parity t >> 7, and for the rotation takes output dims 4 (t & 31) .. + 3
// over rows 16 (t >> 5) .. + 15 of R. Headers, the first MB partials of each
// parity and the R block are requested together, headers first.
constexpr int MB = 16;     // partials per parity per batch of loads
constexpr int MT = 256;    // threads of the merge

template <int G>
__global__ __launch_bounds__(MT) void uniform_merge_kernel(UniformArgs a) {
  __shared__ __align__(16) float wsh[MT / 64][MAXWG];  // per wave: w_p (0 past nwg and for empty partials)
  __shared__ __align__(16) float hsh[MT / 64][MAXWG];  // per wave: f_p
  __shared__ __align__(16) float ys[2][FD];   // the two parities' weighted sums, rotated
  __shared__ __align__(16) float xs[2][FD];   // and original-space
  __shared__ __align__(16) float red[8][FD];  // rotation: sums over the 8 row blocks
  const int hqi = blockIdx.x, b = blockIdx.y;
  const int g = hqi / G, h = hqi % G;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int d = tid & (FD - 1), par = tid >> 7;
  const int np = a.nwg;

  const int64_t pst = (int64_t)G * PPS;
  const float* pp = a.part + (int64_t)(b * a.hkv + g) * np * pst + h * PPS;  // partial p at pp + p * pst
  const int last = np - 1;
  // every wave reads all headers (lane + 64k), so the weights need no barrier
  static_assert(MAXWG == 256, "four headers per lane");
  float4 hd[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) hd[k] = *reinterpret_cast<const float4*>(pp + min(lane + 64 * k, last) * pst);
  float x[MB], xo[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) {
    const float* pr = pp + min(2 * i + par, last) * pst + P_OUT + d;
    x[i] = pr[0];
    xo[i] = pr[FD];
  }
  const int j4 = 4 * (tid & 31), ib = tid >> 5;
  float4 rr[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) rr[k] = *reinterpret_cast<const float4*>(a.vrot + (16 * ib + k) * FD + j4);

  // the global max over the partials with a sum, then the weights
  float m = M_INIT;
#pragma unroll
  for (int k = 0; k < 4; ++k) m = lane + 64 * k < np && hd[k].y > 0.f ? fmaxf(m, hd[k].x) : m;
  const float M = wave_max(m);
  float ls = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const bool ok = lane + 64 * k < np && hd[k].y > 0.f;
    const float wp = ok ? fexp2(hd[k].x - M) * hd[k].y : 0.f;
    wsh[wv][lane + 64 * k] = wp;  // zero past np
    hsh[wv][lane + 64 * k] = ok ? hd[k].z : 0.f;
    ls += wp;
  }
  const float Ls = wave_sum(ls);
  const float inv = Ls > 0.f ? 1.f / Ls : 0.f;
  float acc = 0.f, acco = 0.f;
  for (int p0 = 0;; p0 += 2 * MB) {
    // branch-free: values of empty partials (weight 0) and of partials
    // without an original-space part are replaced by 0 (they may hold
    // anything, NaN included); partials past np have weight 0
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      const float w = wsh[wv][p0 + 2 * i + par], f = hsh[wv][p0 + 2 * i + par];
      acc = fmaf(w, w != 0.f ? x[i] : 0.f, acc);
      acco = fmaf(w, f != 0.f ? xo[i] : 0.f, acco);
    }
    if (p0 + 2 * MB >= np) break;
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      const float* pr = pp + min(p0 + 2 * MB + 2 * i + par, last) * pst + P_OUT + d;
      x[i] = pr[0];
      xo[i] = pr[FD];
    }
  }
  ys[par][d] = acc;
  xs[par][d] = acco;
  __syncthreads();
  // rotation: rows 16 ib .. + 15 of R times the merged rotated sum
  float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int i = 16 * ib + k;
    const float y = ys[0][i] + ys[1][i];  // one address per wave: a broadcast
    o.x = fmaf(y, rr[k].x, o.x);
    o.y = fmaf(y, rr[k].y, o.y);
    o.z = fmaf(y, rr[k].z, o.z);
    o.w = fmaf(y, rr[k].w, o.w);
  }
  *reinterpret_cast<float4*>(&red[ib][j4]) = o;
  __syncthreads();
  if (tid < FD) {
    float r = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) r += red[k][tid];
    a.out[((int64_t)b * a.hq + hqi) * FD + tid] = (r + (xs[0][tid] + xs[1][tid])) * inv;
  }
  if (a.ml && tid == 0) {
    a.ml[((int64_t)b * a.hq + hqi) * 2] = M;
    a.ml[((int64_t)b * a.hq + hqi) * 2 + 1] = Ls;
  }
}

}  // namespace uk

}  // namespace tq
