// Fused decode attention for K4/V2 TurboQuant caches on gfx950: a persistent
// partials kernel over the compressed and fp16 tokens, and a merge kernel that
// combines the partials and applies the inverse rotation once per query head.
//
// Work (plan in tq_decode_fast.h): the tokens of (sequence b, kv head g) are
// weighted units, its fp16 blocks (32 tokens of the [sink | residual ring]
// list) first, then its packed 32-token blocks. The units of (b, g) are cut
// into chunks; workgroup p (one per CU, 8 waves) takes a contiguous run of
// chunks. A run of chunks of one (b, g) is a segment: the waves take its fp16
// blocks, then its packed blocks, round robin, and the workgroup writes one
// partial per segment (max, sum, rotated-space output / sum per query head)
// and empty partials (sum 0) for the other chunks of the run. The lookup tables
// are built once per workgroup; the query is rotated once per segment.
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
// one token) and paired across tokens with v_perm, and B = p * n_v split into
// fp16 high part / remainder along the same columns as the scores (zero in
// the k-slots of the other tile). The value table holds an exact fp16 copy of
// the codebook scaled by 1 / vscale (chosen on the host so that both
// magnitudes of the 2-bit codebook are fp16 numbers to within 5e-8), and
// vscale is folded into n_v.
// fp16 tokens (original space) use the same MFMAs with exact fp16 keys /
// values and the query in original space; their normalised sum is rotated
// into the segment's partial (MFMA, R high part / remainder) at the end of
// their phase.
//
// The merge kernel (one workgroup per query head and 32-dim output slice)
// combines the partials of (b, g) with their softmax weights
// (docs/FULL_FUSED_ATTENTION_RESULTS.md:34-40) and applies out = sum @ R in
// float32 (rotation.py:68-78).

#include <math.h>

#include "tq_common.h"
#include "tq_decode_fast.h"

namespace tq {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef __fp16 hx2 __attribute__((ext_vector_type(2)));

constexpr int FD = 128;
constexpr int FW = FAST_WAVES;       // waves per workgroup (FW * 16 == FD)
constexpr int FT = FW * 64;          // threads
constexpr int PS = FAST_PART_FLOATS; // floats per (slot, head) partial
constexpr int P_OUT = 4;             // partial: [M, L, pad, pad, out[128]]
constexpr int PPS = PACKED_PART_FLOATS;  // floats per (slot, head) K4/V2 partial
constexpr float M_INIT = -1e30f;     // running max before the first block
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

// LDS layout. Lookup tables: key entry of code byte e (two 4-bit codes) and
// value entry of byte e (four 2-bit codes), NCP replicas of 8 bytes each in
// rows of 256 bytes, so the LDS address of an entry is one byte permute of
// the code word (code byte as address bits 8-15). NCP = 32: two tables of
// 64 KB; NCP = 16: one table whose row e holds the 16 key replicas, then the
// 16 value replicas.
//
// With the QJL key term (QB = 1 for sketches of at most 128 projections, 2
// for at most 256), the combine region holds, while the blocks run, the table
// of the 16 patterns of 4 sign bits (row n: the halves (bit j of n ? 1 : -1),
// j < 4, in 32 replicas: its address is a byte permute too), the S q B
// operands of the segment's heads (zero past the sketch's projections) and
// their key-term factors, and, at the query rotation, S (scale q) in float32
// (computed there on MFMA from S); the norm staging also holds the key
// residual norms.
template <int G, int QB = 0>
struct Lay {
  static constexpr int NCP = G <= 4 ? 32 : 16;
  static constexpr uint32_t tabs = NCP == 32 ? 0x20000u : 0x10000u;  // bytes of the tables
  static constexpr int CMS = FD + 4;                                  // floats per combine row: 128 sums, m, l
  static constexpr uint32_t cmb = tabs;                               // [FW][G][CMS] f32
  static constexpr uint32_t slut = cmb;                               // QB: 16 rows x 256 B sign patterns
  static constexpr uint32_t SQS = 256 * (QB > 1 ? 2 : 1) + 16;       // QB: bytes per (head, part) of sqo
  static constexpr uint32_t sqo = slut + 4096;                        // QB: [G][2 parts][SQS] S q B operands
  static constexpr uint32_t kfx = sqo + G * 2 * SQS;                  // QB: [G] f32 key-term factors
  static constexpr int SQM = 128 * (QB > 1 ? 2 : 1);                   // QB: projections per head of sqf
  static constexpr uint32_t sqf = kfx + 64;                           // QB: [G][SQM] f32 S (scale q)
  static constexpr uint32_t QBEND = sqf + G * SQM * 4;
  static constexpr uint32_t CMB_BYTES = !QB || FW * G * CMS * 4 >= QBEND - cmb ? FW * G * CMS * 4 : QBEND - cmb;
  static constexpr uint32_t QOPS = 528;                               // bytes per (head, part) of qop (512 + 16)
  static constexpr uint32_t qop = cmb + CMB_BYTES;                    // [G][2 parts][QOPS] rotated-q B operands
  static constexpr uint32_t qfo = qop + G * 2 * QOPS;                 // [G][2 parts][4 q4][4 kb][16 B] original-space q
  static constexpr uint32_t NSTW = QB ? 384 : 256;                    // norm staging bytes per wave
  static constexpr uint32_t nst = qfo + G * 2 * 256;                  // [FW][NSTW / 4] f32 norm staging
  static constexpr uint32_t pre = nst + FW * NSTW;                    // [G][CMS] parked fp16 tiles: sums, m, l
  static constexpr uint32_t total = pre + G * CMS * 4;
  static constexpr uint32_t qstage = G * FD * 4;                      // bytes of the query rows as given (own array)
};
static_assert(Lay<4>::total + Lay<4>::qstage <= 160 * 1024 && Lay<8>::total + Lay<8>::qstage <= 160 * 1024 &&
              Lay<4, 2>::total + Lay<4, 2>::qstage <= 160 * 1024 &&
              Lay<8, 2>::total + Lay<8, 2>::qstage <= 160 * 1024, "LDS of one workgroup");
static_assert((Lay<1, 1>::slut & 0xFFFFu) == 0 && (Lay<8, 1>::slut & 0xFFFFu) == 0,
              "sign-pattern addresses are byte permutes");

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

__device__ inline uint32_t h16(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }

// A value at a uniform address, read through the scalar cache (constant
// address space: the value is not written during the kernel).
template <typename T>
__device__ inline T ld_uniform(const T* p, int i) {
  return ((const __attribute__((address_space(4))) T*)(p))[i];
}

// Global -> LDS copy of 16 bytes per lane (the active lanes of the wave fill
// consecutive 16-byte pieces from `lds`). The builtin exists in the device
// pass only; the host pass of this file only needs the kernel's declaration.
__device__ inline void load_lds16(const void* g, uint8_t* lds) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_global_load_lds(g, lds, 16, 0, 0);
#endif
}

__device__ inline u2 lds_u2(const uint8_t* smem, uint32_t addr) {
  return *reinterpret_cast<const u2*>(smem + addr);
}

__device__ inline int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

// ---------------------------------------------------------------- work plan
struct SeqLen {
  int comp, sink, res, rstart;
};

// lengths of sequence b clamped to the bounds the host checked, so every read
// stays inside the stores, the sink and the ring; the four loads are issued
// together (an absent array is read through another valid pointer and its
// value replaced)
__device__ inline SeqLen seq_len(const FastArgs& a, int b) {
  const int32_t* any = a.comp_len_b ? a.comp_len_b : a.sink_len_b ? a.sink_len_b : a.res_len_b ? a.res_len_b : a.res_start_b;
  SeqLen s;
  if (!any) {
    s.comp = a.max_comp; s.sink = a.max_sink; s.res = a.max_res; s.rstart = a.res_start0;
    return s;
  }
  const int c = (a.comp_len_b ? a.comp_len_b : any)[b];
  const int k = (a.sink_len_b ? a.sink_len_b : any)[b];
  const int e = (a.res_len_b ? a.res_len_b : any)[b];
  const int t = (a.res_start_b ? a.res_start_b : any)[b];
  s.comp = a.comp_len_b ? min(max(c, 0), a.max_comp) : a.max_comp;
  s.sink = a.sink_len_b ? min(max(k, 0), a.max_sink) : a.max_sink;
  s.res = a.res_len_b ? min(max(e, 0), a.max_res) : a.max_res;
  s.rstart = a.res_start_b ? min(max(t, 0), max(a.res_cap - 1, 0)) : a.res_start0;
  return s;
}

__device__ inline int cdiv(int a, int b) { return (a + b - 1) / b; }

// work units of one (sequence, kv head): its packed blocks, at least one when
// it has fp16 tokens only
__device__ inline int units_of(int comp, int nf) { return max((comp + 31) >> 5, nf > 0 ? 1 : 0); }

struct Plan {
  int T;        // units per chunk (a multiple of FW)
  int V;        // chunks of the call
  bool uni;     // every sequence has the maximal lengths
  int Wu, nu;   // uniform: units and chunks per (b, g)
};

__device__ inline int round8(int64_t t) { return (int)((max<int64_t>(t, 1) + FW - 1) / FW * FW); }

// inclusive prefix sum over the 64 lanes of the wave
__device__ inline int wave_prefix(int x) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o);
    x += lane >= o ? y : 0;
  }
  return x;
}

// Identical in every wave of both kernels (wave-uniform results). Lane
// b - base holds sequence b of each 64-sequence batch: one division per lane
// and wave sums (no per-sequence loop of divisions).
__device__ Plan make_plan(const FastArgs& a) {
  Plan p{};
  const int lane = threadIdx.x & 63;
  p.uni = a.uni != 0;
  if (p.uni) {  // computed on the host (fast_uniform_plan)
    p.Wu = units_of(a.max_comp, a.max_sink + a.max_res);
    p.T = a.plan_T;
    p.nu = a.plan_nu;
    p.V = a.plan_V;
    return p;
  }
  const int64_t div = (int64_t)a.chunks * a.nwg;
  int64_t U = 0;
  int w0 = 0;  // lane b's units of the first 64 sequences
  for (int base = 0; base < a.batch; base += 64) {
    const int b = base + lane;
    SeqLen s{};
    if (b < a.batch) s = seq_len(a, b);
    const int w = b < a.batch ? units_of(s.comp, s.sink + s.res) : 0;
    if (base == 0) w0 = w;
    U += __builtin_amdgcn_readlane(wave_prefix(w), 63);
  }
  U *= a.hkv;
  p.T = round8((U + div - 1) / div);
  int V = 0;
  for (int base = 0; base < a.batch; base += 64) {
    int w = w0;
    if (base > 0) {
      const int b = base + lane;
      SeqLen s{};
      if (b < a.batch) s = seq_len(a, b);
      w = b < a.batch ? units_of(s.comp, s.sink + s.res) : 0;
    }
    V += __builtin_amdgcn_readlane(wave_prefix(cdiv(w, p.T)), 63);
  }
  p.V = V * a.hkv;
  return p;
}

// Sequence of chunk `key` (or sequence `key` when by_seq): its first chunk
// N_b, chunks per kv head n_b, units W_b and lengths.
struct Loc {
  int b, Nb, nb, W;
  SeqLen s;
};

__device__ Loc locate(const FastArgs& a, const Plan& p, int key, bool by_seq) {
  Loc L{};
  if (p.uni) {
    const int per = a.hkv * p.nu;
    L.b = by_seq ? key : key / per;
    L.Nb = L.b * per;
    L.nb = p.nu;
    L.W = p.Wu;
    L.s = seq_len(a, L.b);
    return L;
  }
  // lane b - base: its sequence's chunks hkv n_b and their end (inclusive
  // prefix) after the chunks of the sequences before the batch (carry)
  const int lane = threadIdx.x & 63;
  int carry = 0;
  for (int base = 0; base < a.batch; base += 64) {
    const int b = base + lane;
    SeqLen s{};
    if (b < a.batch) s = seq_len(a, b);
    const int w = b < a.batch ? units_of(s.comp, s.sink + s.res) : 0;
    const int n = a.hkv * cdiv(w, p.T);
    const int end = carry + wave_prefix(n);
    int k = -1;
    if (by_seq) {
      if (key >= base && key < base + 64) k = key - base;
    } else {
      // the first sequence whose chunks end past the key (sequences past the
      // batch end at the total and are never the first)
      const uint64_t past = __builtin_amdgcn_ballot_w64(b < a.batch && end > key);
      if (past != 0) k = (int)__builtin_ctzll(past);
    }
    if (k >= 0) {
      L.b = base + k;
      L.nb = __builtin_amdgcn_readlane(n, k) / a.hkv;
      L.Nb = __builtin_amdgcn_readlane(end, k) - __builtin_amdgcn_readlane(n, k);
      L.W = __builtin_amdgcn_readlane(w, k);
      L.s.comp = __builtin_amdgcn_readlane(s.comp, k);
      L.s.sink = __builtin_amdgcn_readlane(s.sink, k);
      L.s.res = __builtin_amdgcn_readlane(s.res, k);
      L.s.rstart = __builtin_amdgcn_readlane(s.rstart, k);
      break;
    }
    carry = __builtin_amdgcn_readlane(end, 63);
  }
  return L;
}

// One segment of a workgroup: chunks [v, vend) of (b, g), their packed blocks
// [k0, k1) and fp16 tiles [t0, t1).
struct Seg {
  int b, g, row, vend;
  int k0, k1, t0, t1;
  int comp, sink, nf, rstart;
};

// Per sequence b: (N_b, n_b) of the plan into tab[2b], tab[2b + 1], for the
// merge kernel (one wave; the lanes take 64 sequences at a time).
__device__ void write_plan_table(const FastArgs& a, const Plan& p, int32_t* tab) {
  const int lane = threadIdx.x & 63;
  int carry = 0;
  for (int base = 0; base < a.batch; base += 64) {
    const int b = base + lane;
    SeqLen s{};
    if (b < a.batch) s = seq_len(a, b);
    const int w = b < a.batch ? units_of(s.comp, s.sink + s.res) : 0;
    const int n = a.hkv * cdiv(w, p.T);
    const int end = carry + wave_prefix(n);
    if (b < a.batch) {
      tab[2 * b] = end - n;
      tab[2 * b + 1] = n / a.hkv;
    }
    carry = __builtin_amdgcn_readlane(end, 63);
  }
}

__device__ inline Seg segment(const FastArgs& a, const Plan& P, int v, int v1) {
  const Loc L = locate(a, P, v, false);
  Seg S;
  const int rel = v - L.Nb;
  S.b = L.b;
  S.g = uni(rel / L.nb);
  const int jc = uni(rel % L.nb);
  S.vend = uni(min(v1, L.Nb + (S.g + 1) * L.nb));
  const int cnt = S.vend - v;
  S.row = S.b * a.hkv + S.g;
  S.comp = L.s.comp;
  S.sink = L.s.sink;
  S.nf = L.s.sink + L.s.res;
  S.rstart = L.s.rstart;
  const int Pb = (S.comp + 31) >> 5;
  S.k0 = min(Pb, jc * P.T);
  S.k1 = min(Pb, (jc + cnt) * P.T);
  const int ntl = (S.nf + 15) >> 4;
  const int tpc = cdiv(ntl, L.nb);
  S.t0 = min(ntl, jc * tpc);
  S.t1 = min(ntl, (jc + cnt) * tpc);
  return S;
}

// max / sum over the 64 lanes of a wave (every lane gets the result)
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

// ------------------------------------------------------------ partials kernel
// One packed block of a wave, loaded from HBM (lane r, q4)
struct Blk {
  u4 k0, k1;      // key codes of tokens t0 + r and t0 + 16 + r, bytes 16*q4 ..
  uint32_t v[8];  // value code halfword r of tokens A0..A3 (t0 + 4q4 + i), B0..B3 (t0 + 16 + 4q4 + i)
  float nk, nv;   // key / value norm of token t0 + (lane & 31)
  // QJL key term (QB): key sign dwords 4 c + q4 (c < QB) of tokens t0 + r
  // and t0 + 16 + r, key residual norm of token t0 + (lane & 31)
  uint32_t ks0[2], ks1[2];
  float gk;
};

// One fp16 tile (16 tokens of the [sink | ring] list) of wave FW - 1 (lane r, q4)
struct Tile16 {
  u4 k[4];  // key row of token r, dims 32 q4 + 8 kb .. + 8
  u4 v[4];  // value rows of tokens 4 q4 + i, dims 8 r .. 8 r + 7
};

// Raw buffer over `bytes` bytes at p (stride 0): loads past the end read zero.
__device__ inline __amdgpu_buffer_rsrc_t rsrc(const void* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, bytes, 0x00020000);
}

constexpr int WF16 = FW - 1;  // the wave that takes the fp16 tiles (it has the fewest packed blocks)

template <int G, int QB>
__global__ __launch_bounds__(FT) void decode_partials_kernel(FastArgs a) {
  using LY = Lay<G, QB>;
  __shared__ __align__(16) uint8_t smem[LY::total];
  // the G query rows of the segment as given, written by direct global->LDS
  // loads (an array of its own, so those loads are not ordered with smem)
  __shared__ __align__(16) uint8_t qst[LY::qstage];

  constexpr int TS = G <= 4 ? 2 : 1;  // tiles sharing the columns
  constexpr int NS = 8 / TS;           // scores per lane per block
  const int w = uni(threadIdx.x >> 6);
  const int j0 = 16 * w;  // rotated dims of this wave in the query rotation
  const int esz = a.q_dtype == TQ_F32 ? 4 : 2;
  // Lane-derived values, recomputed at the start of every phase from an opaque
  // copy of the thread id: otherwise the compiler computes them once and keeps
  // them live through the block loop, where they do not fit beside its
  // registers.
  int tid, lane, r, q4, tile, c8, hd, ko, vo, no;
  bool lo_part, writer;
  float partf;
  auto rederive = [&]() {
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    tid = t;
    lane = t & 63;
    r = lane & 15;
    q4 = lane >> 4;
    tile = TS == 2 ? r >> 3 : 0;  // tile of column r (TS == 2)
    c8 = r & 7;
    hd = TS == 2 ? (c8 < 4 ? c8 : 7 - c8) % G : c8;  // query head of column r
    lo_part = TS == 2 ? c8 >= 4 : r >= 8;          // column holds the fp16 remainder
    partf = lo_part ? 1.f : 0.f;
    writer = !lo_part && c8 < G;  // one column per (tile, head) writes the combine rows
    // lane byte offsets within a block: key bytes 16*q4 .. of token r (token
    // 16 + r at +1024); value halfword r of token 4*q4 (token 4*q4 + i at
    // +32 i, token 16 + 4*q4 + i at +512 + 32 i); norm of token lane & 31
    ko = r * 64 + 16 * q4;
    vo = q4 * 128 + 2 * r;
    no = (lane & 31) * 4;
  };
  rederive();

  // Every kernel argument the set-up needs, loaded in one batch of scalar
  // loads and waited for once (first uses spread over the set-up would
  // otherwise wait one by one).
  asm volatile("" ::"s"(a.kc), "s"(a.kn), "s"(a.vc), "s"(a.vn), "s"(a.q), "s"(a.rot16), "s"(a.sink_k),
               "s"(a.sink_v), "s"(a.res_k), "s"(a.res_v), "s"(a.k_hs), "s"(a.kn_hs), "s"(a.v_hs), "s"(a.vn_hs),
               "s"(a.sink_hs), "s"(a.res_hs), "s"(a.max_comp), "s"(a.max_sink), "s"(a.max_res), "s"(a.res_start0),
               "s"(a.res_cap), "s"(a.hq), "s"(a.hkv), "s"(a.q_dtype), "s"(a.uni), "s"(a.plan_T), "s"(a.plan_nu),
               "s"(a.plan_V), "s"(a.nwg), "s"(a.batch));
  asm volatile("" ::"s"(a.klut), "s"(a.vlut), "s"(a.qscale), "s"(a.vscale), "s"(a.comp_len_b), "s"(a.sink_len_b),
               "s"(a.res_len_b), "s"(a.res_start_b), "s"(a.part));
  // the decode-table entries of this lane's rows of the LDS tables (row e =
  // 32 w + 4 k + lane / 16, k < 8), requested before anything else
  uint64_t ke[8], ve[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int e = 32 * w + 4 * k + (lane >> 4);
    ke[k] = a.klut[e];
    ve[k] = a.vlut[e];
  }
  const Plan P = make_plan(a);
  if (!P.uni && blockIdx.x == 0 && w == 0) write_plan_table(a, P, a.plan_tab);
  const int v0 = (int)((int64_t)blockIdx.x * P.V / a.nwg);
  const int v1 = (int)((int64_t)(blockIdx.x + 1) * P.V / a.nwg);

  // ---- per-segment loads, issued at the end of the previous segment (for
  // the first segment before the lookup tables are built): the query rows,
  // the R rows j0 + n of this wave as MFMA B operands (fp16 high part and
  // remainder; k-slot (q4, i) of step kb = dim 32 kb + 8 q4 + i; QB: at the
  // segment's start instead, with the S rows), then the first two packed
  // blocks of the wave.
  Seg S{};
  const int qchunks = G * FD * esz / 16;  // 16-byte chunks of the G query rows
  u4 rqh[4], rql[4];
  Tile16 T16;
  Blk B0, B1, B2;
  int nkw = 0;
  const uint8_t *kcodes = nullptr, *vcodes = nullptr, *ksgn = nullptr;
  const float *knorm = nullptr, *vnorm = nullptr, *kgam = nullptr;
  auto slot_t0 = [&](int m) { return (S.k0 + w + FW * m) << 5; };
  auto load_slot = [&](Blk& B, int m) {
    const bool live = m < nkw;
    const int t0 = live ? slot_t0(m) : 0;
    const int n = live ? S.comp - t0 : 0;  // tokens readable from t0 on
    const __amdgpu_buffer_rsrc_t rk = rsrc(kcodes + (int64_t)t0 * 64, n * 64);
    const __amdgpu_buffer_rsrc_t rv = rsrc(vcodes + (int64_t)t0 * 32, n * 32);
    const __amdgpu_buffer_rsrc_t rkn = rsrc(knorm + t0, n * 4);
    const __amdgpu_buffer_rsrc_t rvn = rsrc(vnorm + t0, n * 4);
    // constant offsets as the scalar offset operand (no per-offset VGPRs)
    B.k0 = __builtin_amdgcn_raw_buffer_load_b128(rk, ko, 0, 0);
    B.k1 = __builtin_amdgcn_raw_buffer_load_b128(rk, ko, 1024, 0);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      B.v[i] = __builtin_amdgcn_raw_buffer_load_b16(rv, vo, i < 4 ? 32 * i : 512 + 32 * (i - 4), 0);
    B.nk = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rkn, no, 0, 0));
    B.nv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rvn, no, 0, 0));
    if constexpr (QB) {
      // dword q4 + 4 c of the sign rows of a.qm / 8 bytes; dwords past a row
      // read the next token's (or zero past the block): their projections
      // have zero S q operands
      const int rb = a.qm >> 3;
      const __amdgpu_buffer_rsrc_t rks = rsrc(ksgn + (int64_t)t0 * rb, n * rb);
      const __amdgpu_buffer_rsrc_t rkg = rsrc(kgam + t0, n * 4);
#pragma unroll
      for (int c = 0; c < QB; ++c) {
        B.ks0[c] = __builtin_amdgcn_raw_buffer_load_b32(rks, r * rb + 4 * q4 + 16 * c, 0, 0);
        B.ks1[c] = __builtin_amdgcn_raw_buffer_load_b32(rks, (16 + r) * rb + 4 * q4 + 16 * c, 0, 0);
      }
      B.gk = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rkg, no, 0, 0));
    }
  };
  // row of token u of the [sink | ring] list (u clamped into the list)
  auto tok = [&](const uint16_t* s_base, const uint16_t* r_base, int u) {
    u = min(u, S.nf - 1);
    if (u < S.sink) return s_base + (int64_t)u * FD;
    int sl = S.rstart + (u - S.sink);
    sl = sl >= a.res_cap ? sl - a.res_cap : sl;
    return r_base + (int64_t)sl * FD;
  };
  auto load_tile = [&](int t) {
    const uint16_t* sk = a.sink_k + (int64_t)S.row * a.sink_hs;
    const uint16_t* sv = a.sink_v + (int64_t)S.row * a.sink_hs;
    const uint16_t* rk = a.res_k + (int64_t)S.row * a.res_hs;
    const uint16_t* rv = a.res_v + (int64_t)S.row * a.res_hs;
    const uint16_t* pk = tok(sk, rk, 16 * t + r) + 32 * q4;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) T16.k[kb] = *reinterpret_cast<const u4*>(pk + 8 * kb);
#pragma unroll
    for (int i = 0; i < 4; ++i) T16.v[i] = *reinterpret_cast<const u4*>(tok(sv, rv, 16 * t + 4 * q4 + i) + 8 * r);
  };
  // the R rows j0 + n of this wave (QB: loaded at each segment's rotation
  // from an opaque address, so that they are neither hoisted nor held across
  // the block loop, where the sketch's operands need the registers)
  auto load_rrows = [&]() {
    const uint16_t* rh = a.rot16 + (j0 + r) * FD + 8 * q4;
    if constexpr (QB) asm volatile("" : "+v"(rh));
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      rqh[kb] = *reinterpret_cast<const u4*>(rh + 32 * kb);
      rql[kb] = *reinterpret_cast<const u4*>(rh + FD * FD + 32 * kb);
    }
  };
  auto issue = [&](int v) {
    S = segment(a, P, v, v1);
    {
      // the G query rows of (b, g), 16-byte chunk e by thread e, straight into
      // LDS (wave w fills bytes [1024 w, 1024 w + 1024))
      const uint8_t* qp = static_cast<const uint8_t*>(a.q) + ((int64_t)S.b * a.hq + S.g * G) * FD * esz;
      if (tid < qchunks)
        load_lds16(qp + 16 * tid, qst + 1024 * w);
    }
    if constexpr (!QB) load_rrows();
    nkw = S.k1 - S.k0 > w ? (S.k1 - S.k0 - w + FW - 1) / FW : 0;
    kcodes = a.kc + (int64_t)S.row * a.k_hs;
    vcodes = a.vc + (int64_t)S.row * a.v_hs;
    knorm = a.kn + (int64_t)S.row * a.kn_hs;
    vnorm = a.vn + (int64_t)S.row * a.vn_hs;
    if constexpr (QB) {
      ksgn = a.ksg + (int64_t)S.row * a.ksg_hs;
      kgam = a.kgam + (int64_t)S.row * a.kgam_hs;
    }
    // wave WF16 requests its packed blocks after its fp16 tiles (their
    // registers do not overlap)
    if (!(w == WF16 && S.t1 > S.t0)) {
      load_slot(B0, 0);
      load_slot(B1, 1);
    }
  };
  if (v0 < v1) issue(v0);

  // ---- lookup tables (once per workgroup): each lane stores two replicas of
  // its rows' entries per 16-byte store, lane-linear (a wave's store fills 4
  // consecutive rows)
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const uint32_t off = (uint32_t)(32 * w + 4 * k + (lane >> 4)) * 256 + 16 * (lane & 15);
    const u4 kv = u4{(uint32_t)ke[k], (uint32_t)(ke[k] >> 32), (uint32_t)ke[k], (uint32_t)(ke[k] >> 32)};
    const u4 vv = u4{(uint32_t)ve[k], (uint32_t)(ve[k] >> 32), (uint32_t)ve[k], (uint32_t)(ve[k] >> 32)};
    if constexpr (LY::NCP == 32) {
      *reinterpret_cast<u4*>(smem + 0x10000u + off) = kv;
      *reinterpret_cast<u4*>(smem + off) = vv;
    } else {
      *reinterpret_cast<u4*>(smem + off) = (lane & 15) >= 8 ? vv : kv;
    }
  }
  // per-lane table address constants: byte 0 the replica offset, byte 2 the
  // key table's base bit (NCP = 32)
  uint32_t ck, cv;
  constexpr uint32_t selk = LY::NCP == 32 ? 0x0C020000u : 0x0C0C0000u;
  auto table_consts = [&]() {
    if constexpr (LY::NCP == 32) {
      ck = (uint32_t)(lane & 31) * 8 | 0x10000u;
      cv = (uint32_t)(lane & 31) * 8;
    } else {
      ck = (uint32_t)(lane & 15) * 8;
      cv = (uint32_t)(lane & 15) * 8 + 128;
    }
  };
  auto kaddr = [&](uint32_t word, int byte) { return __builtin_amdgcn_perm(word, ck, selk | ((4u + byte) << 8)); };
  auto vaddr = [&](uint32_t word, int byte) { return __builtin_amdgcn_perm(word, cv, 0x0C0C0000u | ((4u + byte) << 8)); };

  // Online softmax of the NS scores of this lane (tokens A0..A3 and / or
  // B0..B3 of the block, column r); returns the P^T operand (p * nv, high
  // part or remainder by column, zero in the k-slots of the other tile) and
  // rescales `acc` when a block's max exceeds the running max, or when p *
  // nv would leave the fp16 range (the column exponent vx then grows); with
  // `setx` (compressed blocks) the first non-empty block sets vx (`vset`).
  auto softmax_pv = [&](float (&s)[NS], const float (&nv)[NS], f4 (&acc)[8], float& m_run, float& l_run,
                        int& vx, bool& vset, bool setx) {
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
      pm = fmaxf(pm, pv[i]);
    }
    const float pmx = pm * __builtin_amdgcn_ldexpf(1.f, -vx);
    const bool first = setx && !vset;  // wave-uniform
    if (__builtin_amdgcn_ballot_w64(pmx > PV_LIMIT || (first && pmx > 0.f)) != 0) {
      const float cm = rows_max(pmx);
      int d;
      if (first) {
        d = cm > 0.f ? max((int)ceilf(log2f(cm / PV_SET)), -110) : 0;
        vset = true;
      } else {
        d = cm > PV_LIMIT ? (int)ceilf(log2f(cm / PV_LIMIT)) : 0;
      }
      const float f = __builtin_amdgcn_ldexpf(1.f, -d);
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) acc[nb] *= f;
      vx += d;
    }
    const float down = __builtin_amdgcn_ldexpf(1.f, -vx);
    uint32_t dd[NS / 2];
#pragma unroll
    for (int j = 0; j < NS / 2; ++j) {
      const float p0 = pv[2 * j] * down, p1 = pv[2 * j + 1] * down;
      const hx2 h = __builtin_amdgcn_cvt_pkrtz(p0, p1);
      const float e0 = fmaf(-partf, (float)h[0], p0);
      const float e1 = fmaf(-partf, (float)h[1], p1);
      dd[j] = pk_rtz(e0, e1);
    }
    u4 pb;
    if constexpr (TS == 2) {
      pb[0] = tile ? 0u : dd[0];
      pb[1] = tile ? 0u : dd[1];
      pb[2] = tile ? dd[0] : 0u;
      pb[3] = tile ? dd[1] : 0u;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) pb[j] = dd[j];
    }
    return as_h8(pb);
  };

  // A wave's state -> one LDS row per head [sums 128 | m | l]: the two fp16
  // parts of a (tile, head) meet through `partner`; for TS == 2 the two tiles
  // of a head (columns r and r ^ 8) are merged at their common max by a
  // rotation by 8, and the high-part column of tile 0 writes the row.
  auto to_rows = [&](f4 (&acc)[8], float m_run, float l_run, int vx, float* rows) {
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
    float* cm = rows + hd * LY::CMS;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float vr[8];
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) {
        float x = (acc[nb][i] + partner<G>(acc[nb][i])) * tsc;
        if constexpr (TS == 2) x += row_ror<8>(x);
        vr[nb] = x;
      }
      if (writer && tile == 0) {
        float* d = cm + 32 * q4 + 8 * i;
        *reinterpret_cast<float4*>(d) = make_float4(vr[0], vr[1], vr[2], vr[3]);
        *reinterpret_cast<float4*>(d + 4) = make_float4(vr[4], vr[5], vr[6], vr[7]);
      }
    }
    if (q4 == 0 && writer && tile == 0) *reinterpret_cast<float2*>(cm + FD) = make_float2(m_run, l_run);
  };

  const float vsc = a.vscale;
  // this wave's norm staging: [key norms 32][value norms 32] (QB: [key residual norms 32] after them)
  uint8_t* nst = smem + LY::nst + w * LY::NSTW;

  for (int v = v0; v < v1;) {
    rederive();
    const bool has16 = S.t1 > S.t0;
    // QB: the R rows and rows 16 (w + FW c) + r of S, dims 32 kb + 8 q4 .. + 8
    // at [c][2 kb], [c][2 kb + 1] (opaque addresses: loaded per segment, not
    // held across the block loop), requested before the barrier; tiles past
    // the sketch's projections read row r
    [[maybe_unused]] float4 srow[QB > 1 ? 2 : 1][8];
    if constexpr (QB) {
      load_rrows();
#pragma unroll
      for (int c = 0; c < QB; ++c) {
        const int p0 = 16 * (w + FW * c);
        const float* sp = a.sproj + (int64_t)((p0 < a.qm ? p0 : 0) + r) * FD + 8 * q4;
        asm volatile("" : "+v"(sp));
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          srow[c][2 * kb] = *reinterpret_cast<const float4*>(sp + 32 * kb);
          srow[c][2 * kb + 1] = *reinterpret_cast<const float4*>(sp + 32 * kb + 4);
        }
      }
    }
    __syncthreads();

    // ---- query rotation: D[h][n] = sum_i q[h][i] R[j0 + n][i] on MFMA (q
    // high part x R high part + q high x R remainder + q remainder x R high),
    // written (times qscale, and 2^-qe per head for very large queries) as
    // fp16 high part / remainder straight into the score B-operand layout
    // [head][part][q4][s][8 halves]: dim j = 32*q4 + 4*s + e sits at halves
    // (e & 1) + 4*(e >> 1) and + 2
    float qe_scale;  // 2^qe of this lane's column head: multiplies its scores
    {
      // dims 32 kb + 8 q4 .. + 8 of query head min(r, G - 1) (the A operand
      // rows), as float
      float x[4][8];
      {
        const uint8_t* qr = qst + (uint32_t)min(r, G - 1) * FD * esz;
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
      }
      float ss = 0.f;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 8; ++i) ss = fmaf(x[kb][i], x[kb][i], ss);
      // the query norm of head r (4 lanes hold its 128 dims) bounds every
      // rotated coordinate: the power of two that keeps the operands in fp16
      // range
      ss = rows_sum(ss);
      const int qe = query_exponent(sqrtf(ss), a.qscale, Q_LIMIT, Q_LOW);  // lanes r: head r
      const float qdown = __builtin_amdgcn_ldexpf(1.f, -qe);
      half8 qo_hi[4], qo_lo[4];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float xs = x[kb][i] * qdown;
          qo_hi[kb][i] = (_Float16)xs;
          qo_lo[kb][i] = (_Float16)(xs - (float)qo_hi[kb][i]);
        }
      f4 dq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        dq = mfma(qo_hi[kb], as_h8(rqh[kb]), dq);
        dq = mfma(qo_hi[kb], as_h8(rql[kb]), dq);
        dq = mfma(qo_lo[kb], as_h8(rqh[kb]), dq);
      }
      if constexpr (QB) {
        // S (scale q) of the segment's heads on MFMA: the rotation's A
        // operands against S rows as B operands (fp16 high part / remainder);
        // lane (r, q4) ends with projection 16 (w + FW c) + r of heads
        // 4 q4 + i, times scale 2^qe_h (undoing the query's 2^-qe_h), into sqf
        float sfac[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          int e = 0;
#pragma unroll
          for (int h = 0; h < G; ++h) {
            const int xh = __builtin_amdgcn_readlane(qe, h);
            e = 4 * q4 + i == h ? xh : e;
          }
          sfac[i] = __builtin_amdgcn_ldexpf(a.sscale, e);
        }
#pragma unroll
        for (int c = 0; c < QB; ++c) {
          const int p0 = 16 * (w + FW * c);
          if (p0 >= a.qm) break;  // wave-uniform
          f4 ds = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kb = 0; kb < 4; ++kb) {
            half8 sh, sl;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const float4 v4 = srow[c][2 * kb + (e >> 2)];
              const float v = (e & 3) == 0 ? v4.x : (e & 3) == 1 ? v4.y : (e & 3) == 2 ? v4.z : v4.w;
              sh[e] = (_Float16)v;
              sl[e] = (_Float16)(v - (float)sh[e]);
            }
            ds = mfma(qo_hi[kb], sh, ds);
            ds = mfma(qo_hi[kb], sl, ds);
            ds = mfma(qo_lo[kb], sh, ds);
          }
          float* sf = reinterpret_cast<float*>(smem + LY::sqf);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int h = 4 * q4 + i;
            if (h < G) sf[h * LY::SQM + p0 + r] = ds[i] * sfac[i];
          }
        }
      }
      // the first fp16 tile of wave WF16, requested once the rotation's
      // registers are free (its latency overlaps the barrier)
      if (has16 && w == WF16) load_tile(S.t0);
      const int j = j0 + r, e = j & 3;
      const uint32_t off = ((uint32_t)(j >> 5) * 8 + ((j >> 2) & 7)) * 16 + 2 * ((e & 1) + 4 * (e >> 1));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int h = 4 * q4 + i;
        if (h < G) {
          const float vq = dq[i] * a.qscale;
          const _Float16 hi = (_Float16)vq, lo = (_Float16)(vq - (float)hi);
          uint8_t* dh = smem + LY::qop + (uint32_t)(h * 2) * LY::QOPS + off;
          *reinterpret_cast<_Float16*>(dh) = hi;
          *reinterpret_cast<_Float16*>(dh + 4) = hi;
          *reinterpret_cast<_Float16*>(dh + LY::QOPS) = lo;
          *reinterpret_cast<_Float16*>(dh + LY::QOPS + 4) = lo;
        }
      }
      // fp16 tokens: the (unscaled, 2^-qe) query in original space, step kb
      // k-slot (q4, i) = dim 32*q4 + 8*kb + i, high part / remainder in
      // [head][part][q4][kb][8 halves]; the lane holding dims 32*kb + 8*q4 ..
      // of head r copies its operand halves there
      if (has16 && w == 0 && r < G) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          uint8_t* dd = smem + LY::qfo + ((uint32_t)(r * 2 * 4 + kb) * 4 + q4) * 16;
          *reinterpret_cast<half8*>(dd) = qo_hi[kb];
          *reinterpret_cast<half8*>(dd + 4 * 4 * 16) = qo_lo[kb];
        }
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
    if constexpr (QB) {
      // the sign-pattern table (thread t: replica t & 31 of row t >> 5) and
      // the S q B operands of head w: (S q) 2^-e (its largest |(S q)_j| into
      // [2^13, 2^14)) as fp16 high part / remainder at [head][part][j], and
      // the head's factor log2(e) sqrt(pi / 2) / 128 2^e
      {
        const uint32_t n = (uint32_t)tid >> 5;
        auto hv = [&](int j) { return ((n >> j) & 1u) ? 0x3C00u : 0xBC00u; };
        *reinterpret_cast<u2*>(smem + LY::slut + n * 256 + 8 * (tid & 31)) = u2{hv(0) | hv(1) << 16, hv(2) | hv(3) << 16};
      }
      __syncthreads();  // every wave's S q is in sqf
      if (w < G) {
        constexpr int NQ = QB > 1 ? 4 : 2;
        float sqv[NQ];
        {
          const float* sf = reinterpret_cast<const float*>(smem + LY::sqf) + w * LY::SQM;
#pragma unroll
          for (int i = 0; i < NQ; ++i) sqv[i] = NQ * lane + i < a.qm ? sf[NQ * lane + i] : 0.f;
        }
        float mx = 0.f;
#pragma unroll
        for (int i = 0; i < NQ; ++i) mx = fmaxf(mx, fabsf(sqv[i]));
        mx = wave_max(mx);
        const int eh = mx > 0.f ? max((int)((__float_as_uint(mx) >> 23) & 0xFFu) - 140, -100) : 0;
        const float sc = __builtin_amdgcn_ldexpf(1.f, -eh);
        uint32_t hw[NQ / 2], lw[NQ / 2];
#pragma unroll
        for (int i = 0; i < NQ / 2; ++i) {
          const float y0 = sqv[2 * i] * sc, y1 = sqv[2 * i + 1] * sc;
          const _Float16 h0 = (_Float16)y0, h1 = (_Float16)y1;
          const _Float16 l0 = (_Float16)(y0 - (float)h0), l1 = (_Float16)(y1 - (float)h1);
          hw[i] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | (uint32_t)__builtin_bit_cast(uint16_t, h1) << 16;
          lw[i] = (uint32_t)__builtin_bit_cast(uint16_t, l0) | (uint32_t)__builtin_bit_cast(uint16_t, l1) << 16;
        }
        uint8_t* d = smem + LY::sqo + (uint32_t)(w * 2) * LY::SQS + 2 * NQ * lane;
#pragma unroll
        for (int i = 0; i < NQ / 2; ++i) {
          *reinterpret_cast<uint32_t*>(d + 4 * i) = hw[i];
          *reinterpret_cast<uint32_t*>(d + LY::SQS + 4 * i) = lw[i];
        }
        if (lane == 0)
          reinterpret_cast<float*>(smem + LY::kfx)[w] =
              __builtin_amdgcn_ldexpf(1.4426950408889634f * 1.2533141373155003f / 128.f, eh);
      }
    }
    __syncthreads();

    // ---- fp16 tiles (wave WF16, original space): parked in LDS (`pre`) as
    // [sums | m | l] per head
    rederive();
    if (has16 && w == WF16) {
      half8 qf[4];
      {
        const uint8_t* src = smem + LY::qfo + ((uint32_t)(hd * 2 + (lo_part ? 1 : 0)) * 4 + q4) * 4 * 16;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) qf[kb] = *reinterpret_cast<const half8*>(src + 16 * kb);
      }
      f4 acc_o[8];
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) acc_o[nb] = f4{0.f, 0.f, 0.f, 0.f};
      float m_o = M_INIT, l_o = 0.f;
      int vx_o = 0;
      bool vset_o = true;  // p * 1 <= 1: the fp16 tiles keep vx_o = 0
      const float sf = a.qscale * qe_scale;
      for (int t = S.t0; t < S.t1; ++t) {
        if (t != S.t0) load_tile(t);
        // one 16-token score tile (tokens r); the k-slots of tokens 16.. of
        // the P^T operand stay empty
        f4 sA = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) sA = mfma(as_h8(T16.k[kb]), qf[kb], sA);
        float sc[NS], ones[NS];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float full = (sA[i] + partner<G>(sA[i])) * sf;
          sc[i] = tile == 0 && 16 * t + 4 * q4 + i < S.nf ? full : -INFINITY;  // the tile-1 columns see no fp16 token
          if constexpr (NS == 8) sc[4 + i] = -INFINITY;
        }
#pragma unroll
        for (int i = 0; i < NS; ++i) ones[i] = 1.f;
        const half8 pb = softmax_pv(sc, ones, acc_o, m_o, l_o, vx_o, vset_o, false);
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) {
          const uint32_t sel = (nb & 1) ? 0x07060302u : 0x05040100u;
          u4 bv;
          bv[0] = __builtin_amdgcn_perm(T16.v[1][nb >> 1], T16.v[0][nb >> 1], sel);
          bv[1] = __builtin_amdgcn_perm(T16.v[3][nb >> 1], T16.v[2][nb >> 1], sel);
          bv[2] = 0u;
          bv[3] = 0u;
          acc_o[nb] = mfma(as_h8(bv), pb, acc_o[nb]);
        }
      }
      to_rows(acc_o, m_o, l_o, vx_o, reinterpret_cast<float*>(smem + LY::pre));
      load_slot(B0, 0);
      load_slot(B1, 1);
    }
    // QB: the tile registers carry nothing into the next segment (which
    // loads its own), so they are not held across the block loop
    if constexpr (QB) T16 = Tile16{};

    // ---- packed blocks (rotated space)
    rederive();
    table_consts();
    half8 qop[8];
    {
      const uint8_t* src = smem + LY::qop + (uint32_t)(hd * 2 + (lo_part ? 1 : 0)) * LY::QOPS + (uint32_t)q4 * 128;
#pragma unroll
      for (int s = 0; s < 8; ++s) qop[s] = *reinterpret_cast<const half8*>(src + 16 * s);
    }
    f4 acc[8];
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) acc[nb] = f4{0.f, 0.f, 0.f, 0.f};
    float m_run = M_INIT, l_run = 0.f;
    int vx = 0;
    bool vset = false;

    // The norms go to the wave's staging row first, for every slot (also the
    // skipped ones): the wait for a slot's loads then sits before the branch
    // on both paths, and the counts of loads in flight stay exact.
    auto stage = [&](const Blk& Bk) {
      *reinterpret_cast<float*>(nst + 4 * lane) = lane < 32 ? Bk.nk : Bk.nv * vsc;
      if constexpr (QB) {
        if (lane < 32) *reinterpret_cast<float*>(nst + 256 + 4 * lane) = Bk.gk;
      }
    };
    // QB: sign-pattern addresses (byte `byte` of a word of nibbles, one per
    // byte), the S q operands and the key-term factor of this lane's column
    [[maybe_unused]] const uint32_t cs = (uint32_t)(lane & 31) * 8 | LY::slut;
    [[maybe_unused]] const uint32_t ssrc =
        LY::sqo + (uint32_t)(hd * 2 + (lo_part ? 1 : 0)) * LY::SQS + (uint32_t)q4 * 64;
    [[maybe_unused]] const float kfac = QB ? reinterpret_cast<const float*>(smem + LY::kfx)[hd] : 0.f;
    auto saddr = [&](uint32_t word, int byte) { return __builtin_amdgcn_perm(word, cs, 0x0C020000u | ((4u + byte) << 8)); };
    auto compute = [&](const Blk& Bk, int m) {
      const int t0 = slot_t0(m);
      const int tend = m < nkw ? S.comp : 0;
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
      for (int j = 0; j < 4; ++j) {
        const uint32_t px = Bk.v[2 * j], py = Bk.v[2 * j + 1];  // token pair j
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
        const uint32_t wa = Bk.k0[s >> 1], wb = Bk.k1[s >> 1];
        const int by = 2 * (s & 1);
        const u2 ea0 = lds_u2(smem, kaddr(wa, by)), ea1 = lds_u2(smem, kaddr(wa, by + 1));
        const u2 eb0 = lds_u2(smem, kaddr(wb, by)), eb1 = lds_u2(smem, kaddr(wb, by + 1));
        sA = mfma(as_h8(u4{ea0[0], ea0[1], ea1[0], ea1[1]}), qop[s], sA);
        sB = mfma(as_h8(u4{eb0[0], eb0[1], eb1[0], eb1[1]}), qop[s], sB);
      }
      // QJL key term (QB), transposed like the scores: A = 16 tokens x 32
      // projections of +-1 (sign patterns of 4 bits, two lookups per
      // operand), B = (S q) 2^-e high part / remainder along the columns;
      // lane (r, q4) holds sign dwords 4 c + q4 of token r, so step (c, kb)
      // covers projections 128 c + 32 q4 + 8 kb .. + 7. Scaled by the key
      // residual norm and the head's factor, added to the lane's scores.
      f4 zA = {0.f, 0.f, 0.f, 0.f}, zB = {0.f, 0.f, 0.f, 0.f};
      if constexpr (QB) {
#pragma unroll
        for (int c = 0; c < QB; ++c) {
          const uint32_t la = Bk.ks0[c] & 0x0F0F0F0Fu, ha = (Bk.ks0[c] >> 4) & 0x0F0F0F0Fu;
          const uint32_t lb = Bk.ks1[c] & 0x0F0F0F0Fu, hb = (Bk.ks1[c] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
          for (int kb = 0; kb < 4; ++kb) {
            const u2 a0 = lds_u2(smem, saddr(la, kb)), a1 = lds_u2(smem, saddr(ha, kb));
            const u2 b0 = lds_u2(smem, saddr(lb, kb)), b1 = lds_u2(smem, saddr(hb, kb));
            const half8 so = *reinterpret_cast<const half8*>(smem + ssrc + 256 * c + 16 * kb);
            zA = mfma(as_h8(u4{a0[0], a0[1], a1[0], a1[1]}), so, zA);
            zB = mfma(as_h8(u4{b0[0], b0[1], b1[0], b1[1]}), so, zB);
          }
        }
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
        // the key term times the key residual norm and the head's factor
#pragma unroll
        for (int t = 0; t < 2 / TS; ++t) {
          const float4 g4 = *reinterpret_cast<const float4*>(nst + 256 + 64 * (t + tile) + 16 * q4);
          const float gk[4] = {g4.x, g4.y, g4.z, g4.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float zv = TS == 2 ? (tile ? zB[i] : zA[i]) : (t ? zB[i] : zA[i]);
            sc[4 * t + i] = fmaf((zv + partner<G>(zv)) * kfac, gk[i], sc[4 * t + i]);
          }
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
          float* so = a.scores + ((int64_t)S.row * G + hd) * a.qb_hs + t0 + 4 * q4;
#pragma unroll
          for (int t = 0; t < 2 / TS; ++t)
            *reinterpret_cast<float4*>(so + 16 * (t + tile)) =
                make_float4(sc[4 * t], sc[4 * t + 1], sc[4 * t + 2], sc[4 * t + 3]);
        }
      }
      const half8 pb = softmax_pv(sc, nv, acc, m_run, l_run, vx, vset, true);
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) acc[nb] = mfma(as_h8(va[nb]), pb, acc[nb]);
    };

    // three blocks in registers: block m + 2 is requested as block m starts;
    // slots past the wave's blocks read nothing (empty buffer ranges) and are
    // skipped
    for (int m = 0; m < nkw; m += 3) {
      load_slot(B2, m + 2);
      stage(B0);
      compute(B0, m);
      load_slot(B0, m + 3);
      stage(B1);
      if (m + 1 < nkw) compute(B1, m + 1);
      load_slot(B1, m + 4);
      stage(B2);
      if (m + 2 < nkw) compute(B2, m + 2);
    }

    // ---- combine the waves (and the parked fp16 tiles) into the segment's
    // partial: [M, L, has_orig, 0, rotated sum / L, original-space sum / L]
    rederive();
    if constexpr (QB) __syncthreads();  // every wave is past its blocks: the sign table and S q operands are read
    to_rows(acc, m_run, l_run, vx, reinterpret_cast<float*>(smem + LY::cmb) + w * G * LY::CMS);
    __syncthreads();
    {
      const float* cms = reinterpret_cast<const float*>(smem + LY::cmb);
      const float* pr = reinterpret_cast<const float*>(smem + LY::pre);
      float* part = a.part + (int64_t)v * G * PPS;
      for (int e = tid; e < G * FD; e += FT) {
        const int h = e / FD, jj = e % FD;
        float M = has16 ? pr[h * LY::CMS + FD] : M_INIT;
#pragma unroll
        for (int ww = 0; ww < FW; ++ww) M = fmaxf(M, cms[(ww * G + h) * LY::CMS + FD]);
        float O = 0.f, Lt = 0.f;
#pragma unroll
        for (int ww = 0; ww < FW; ++ww) {
          const float* rw = cms + (ww * G + h) * LY::CMS;
          const float sc = fexp2(rw[FD] - M);
          O = fmaf(sc, rw[jj], O);
          Lt = fmaf(sc, rw[FD + 1], Lt);
        }
        float Oo = 0.f;
        if (has16) {
          const float so = fexp2(pr[h * LY::CMS + FD] - M);
          Oo = so * pr[h * LY::CMS + jj];
          Lt = fmaf(so, pr[h * LY::CMS + FD + 1], Lt);
        }
        const float inv = Lt > 0.f ? 1.f / Lt : 0.f;
        part[h * PPS + P_OUT + jj] = O * inv;
        if (has16) part[h * PPS + P_OUT + FD + jj] = Oo * inv;
        if (jj == 0) *reinterpret_cast<float4*>(part + h * PPS) = make_float4(M, Lt, has16 ? 1.f : 0.f, 0.f);
      }
      // the other chunks of the run: empty partials (sum 0, skipped by the merge)
      for (int e = tid; e < (S.vend - v - 1) * G; e += FT)
        *reinterpret_cast<float4*>(a.part + ((int64_t)(v + 1) * G + e) * PPS) = make_float4(M_INIT, 0.f, 0.f, 0.f);
    }
    // the next segment's loads (its query rotation waits for them)
    const int vn = S.vend;
    rederive();
    if (vn < v1) issue(vn);
    v = vn;
  }
}

// ---------------------------------------------------------------- merge kernel

// Query head hqi of sequence b: the partials of (b, g) combined with w_p =
// 2^(M_p - M) L_p / L (M = max_p M_p, L = sum_p 2^(M_p - M) L_p), then out =
// (sum_p w_p rot_p) @ R + sum_p w_p f_p orig_p (float32, R the value codec's
// rotation). One workgroup of 256 threads per (query head, sequence): every
// wave reads all headers for M and L (no barrier), thread t sums dim t & 127
// of the partials of parity t >> 7 with the weights recomputed from the
// headers (uniform over the wave: scalar loads), and for the rotation takes
// output dims 4 (t & 31) .. + 3 over rows 16 (t >> 5) .. + 15 of R. The first
// MB partials of each parity and the R block are requested with the headers.
constexpr int MB = 32;   // partials per batch of loads (orig_merge_kernel)
constexpr int RMB = 16;  // partials per parity per batch of loads (decode_merge_kernel)
constexpr int RMT = 256; // threads of decode_merge_kernel

template <int G, int QV = 0>
__global__ __launch_bounds__(RMT) void decode_merge_kernel(FastArgs a) {
  __shared__ __align__(16) float ys[2][FD];   // the two parities' weighted sums, rotated
  __shared__ __align__(16) float xs[2][FD];   // and original-space
  __shared__ __align__(16) float red[8][FD];  // rotation: sums over the 8 row blocks
  __shared__ __align__(16) float us[QV ? 2 : 1][QV ? 128 * QV : 1];  // QV: the parities' weighted value partials
  const int hqi = blockIdx.x, b = blockIdx.y;
  const int g = hqi / G, h = hqi % G;
  const int tid = threadIdx.x, lane = tid & 63;
  const int d = tid & (FD - 1), par = tid >> 7;

  // R[16 ib + k][j4 .. j4 + 3]: independent of the plan, requested first
  const int j4 = 4 * (tid & 31), ib = tid >> 5;
  float4 rr[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) rr[k] = *reinterpret_cast<const float4*>(a.vrot + (16 * ib + k) * FD + j4);

  // the partials of (b, g): slots N_b + g n_b .. + n_b - 1 (the uniform plan
  // from the host's figures, else the partials kernel's table)
  int Nb, nb;
  if (a.uni) {
    nb = a.plan_nu;
    Nb = b * a.hkv * nb;
  } else {
    const int2 e = *reinterpret_cast<const int2*>(a.plan_tab + 2 * b);
    Nb = e.x;
    nb = e.y;
  }
  const int s0 = Nb + g * nb, cnt = nb;
  const int64_t pst = (int64_t)G * PPS;
  const float* pp = a.part + ((int64_t)s0 * G + h) * PPS;  // partial p at pp + p * pst
  const int last = max(cnt - 1, 0);
  const int upar = __builtin_amdgcn_readfirstlane(par);  // wave-uniform
  // one round of loads: the first RMB partials of the parity (values and,
  // uniform over the wave, headers) and the headers lane + 64 k
  float x[RMB], xo[RMB];
  float4 hu[RMB];
#pragma unroll
  for (int i = 0; i < RMB; ++i) {
    const float* pr = pp + min(2 * i + upar, last) * pst;
    hu[i] = *reinterpret_cast<const float4*>(pr);
    x[i] = pr[P_OUT + d];
    xo[i] = pr[P_OUT + FD + d];
  }
  constexpr int HK = 4;  // headers per lane held in registers (cnt <= 256)
  float2 hl[HK];
#pragma unroll
  for (int k = 0; k < HK; ++k) hl[k] = *reinterpret_cast<const float2*>(pp + min(lane + 64 * k, last) * pst);
  // the global max and sum, every wave over all headers
  float m = M_INIT;
#pragma unroll
  for (int k = 0; k < HK; ++k)
    if (lane + 64 * k < cnt && hl[k].y > 0.f) m = fmaxf(m, hl[k].x);
  for (int p = lane + 64 * HK; p < cnt; p += 64) {
    const float2 hh = *reinterpret_cast<const float2*>(pp + p * pst);
    if (hh.y > 0.f) m = fmaxf(m, hh.x);
  }
  const float M = wave_max(m);
  float ls = 0.f;
#pragma unroll
  for (int k = 0; k < HK; ++k) ls += lane + 64 * k < cnt && hl[k].y > 0.f ? fexp2(hl[k].x - M) * hl[k].y : 0.f;
  for (int p = lane + 64 * HK; p < cnt; p += 64) {
    const float2 hh = *reinterpret_cast<const float2*>(pp + p * pst);
    ls += hh.y > 0.f ? fexp2(hh.x - M) * hh.y : 0.f;
  }
  const float Ls = wave_sum(ls);
  const float inv = Ls > 0.f ? 1.f / Ls : 0.f;
  float acc = 0.f, acco = 0.f;
  for (int p0 = 0;; p0 += 2 * RMB) {
    // branch-free: values of empty partials (weight 0) and of partials
    // without an original-space part are replaced by 0 (they may hold
    // anything, NaN included); partials past cnt have weight 0
#pragma unroll
    for (int i = 0; i < RMB; ++i) {
      const int p = p0 + 2 * i + upar;
      const float w = p < cnt && hu[i].y > 0.f ? fexp2(hu[i].x - M) * hu[i].y : 0.f;
      acc = fmaf(w, w != 0.f ? x[i] : 0.f, acc);
      acco = fmaf(w, w != 0.f && hu[i].z != 0.f ? xo[i] : 0.f, acco);
    }
    if (p0 + 2 * RMB >= cnt) break;
#pragma unroll
    for (int i = 0; i < RMB; ++i) {
      const float* pr = pp + min(p0 + 2 * RMB + 2 * i + upar, last) * pst;
      hu[i] = *reinterpret_cast<const float4*>(pr);
      x[i] = pr[P_OUT + d];
      xo[i] = pr[P_OUT + FD + d];
    }
  }
  ys[par][d] = acc;
  xs[par][d] = acco;
  // QV: S[16 ib + k + 128 c][j4 .. j4 + 3] (rows past the sketch's
  // projections clamped: their weights are zero), requested with the value
  // partials
  [[maybe_unused]] float4 sr[QV ? QV : 1][16];
  if constexpr (QV) {
#pragma unroll
    for (int c = 0; c < QV; ++c)
#pragma unroll
      for (int k = 0; k < 16; ++k)
        sr[c][k] = *reinterpret_cast<const float4*>(a.sproj + min(16 * ib + k + 128 * c, a.qm - 1) * FD + j4);
    // value partials of the query head weighted by 2^(umax - M) (the value
    // kernel's workgroups holding tokens of the sequence; uniform over the
    // wave), projection d (+ 128) of parity par; zero past the sketch
    const int comp = a.comp_len_b ? a.comp_len_b[b] : a.max_comp;
    const int nvb = min(a.qnvc, (comp + a.qtok - 1) / a.qtok);
    const int64_t hb = (int64_t)b * a.hq + hqi;
    const float* up = a.qjl_up + hb * a.qnvc * a.qm;
    const float* um = a.qjl_umax + hb * a.qnvc;
#pragma unroll
    for (int c = 0; c < QV; ++c) {
      const int i = d + 128 * c;
      const int il = i < a.qm ? i : 0;  // projections past the sketch read projection 0 and store 0
      float v[4] = {0.f, 0.f, 0.f, 0.f};
      int q = upar;
      for (; q + 6 < nvb; q += 8) {
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = fmaf(fexp2(um[q + 2 * k] - M), up[(int64_t)(q + 2 * k) * a.qm + il], v[k]);
      }
      for (; q < nvb; q += 2) v[0] = fmaf(fexp2(um[q] - M), up[(int64_t)q * a.qm + il], v[0]);
      us[par][i] = i < a.qm ? (v[0] + v[1]) + (v[2] + v[3]) : 0.f;
    }
  }
  __syncthreads();
  // rotation: rows 16 ib .. + 15 of R times the merged rotated sum (QV: and
  // the value term, sqrt(pi / 2) / 128 S^T u)
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
  if constexpr (QV) {
    constexpr float QJL_C = 1.2533141373155003f / 128.f;  // sqrt(pi / 2) / d
#pragma unroll
    for (int c = 0; c < QV; ++c)
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const int i = 16 * ib + k + 128 * c;
        const float u = QJL_C * (us[0][i] + us[1][i]);
        o.x = fmaf(u, sr[c][k].x, o.x);
        o.y = fmaf(u, sr[c][k].y, o.y);
        o.z = fmaf(u, sr[c][k].z, o.z);
        o.w = fmaf(u, sr[c][k].w, o.w);
      }
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

// ------------------------------------------------ merge of original-space partials
// (the dense kernel's): one wave per (query head, half of the dims); lane p +
// 64k holds the header of partial p + 64k, lane j sums dim 64 * half + j.
struct OrigMergeArgs {
  const float* part;
  float* out;
  int nwg, hq, hkv;
};

template <int G>
__global__ __launch_bounds__(64) void orig_merge_kernel(OrigMergeArgs a) {
  __shared__ __align__(16) float wsh[FAST_MAX_WG];  // w_p, written and read back by the one wave
  const int half = blockIdx.x, hqi = blockIdx.y, b = blockIdx.z;
  const int g = hqi / G, h = hqi % G;
  const int lane = threadIdx.x;
  const int np = a.nwg;
  const int64_t pstride = (int64_t)G * PS;
  const float* pall = a.part + (int64_t)(b * a.hkv + g) * np * pstride + h * PS;  // partial p at pall + p*pstride
  const int dim = 64 * half + lane;

  static_assert(FAST_MAX_WG == 256 && MB == 32, "merge register layout");
  float2 hd[FAST_MAX_WG / 64];
#pragma unroll
  for (int k = 0; k < FAST_MAX_WG / 64; ++k)
    hd[k] = *reinterpret_cast<const float2*>(pall + min(lane + 64 * k, np - 1) * pstride);
  float x[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) x[i] = pall[min(i, np - 1) * pstride + P_OUT + dim];

  float m = M_INIT;
#pragma unroll
  for (int k = 0; k < FAST_MAX_WG / 64; ++k)
    if (lane + 64 * k < np) m = fmaxf(m, hd[k].x);
  m = wave_max(m);
  float wgt[FAST_MAX_WG / 64];
  float l = 0.f;
#pragma unroll
  for (int k = 0; k < FAST_MAX_WG / 64; ++k) {
    wgt[k] = lane + 64 * k < np ? fexp2(hd[k].x - m) * hd[k].y : 0.f;
    l += wgt[k];
  }
  l = wave_sum(l);
  const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
  for (int k = 0; k < FAST_MAX_WG / 64; ++k) wsh[lane + 64 * k] = wgt[k];  // zero past np

  float acc = 0.f;
  for (int p0 = 0;; p0 += MB) {
#pragma unroll
    for (int i = 0; i < MB; i += 4) {
      const float4 wp = *reinterpret_cast<const float4*>(wsh + p0 + i);  // one address: a broadcast
      acc = fmaf(wp.x, x[i], acc);
      acc = fmaf(wp.y, x[i + 1], acc);
      acc = fmaf(wp.z, x[i + 2], acc);
      acc = fmaf(wp.w, x[i + 3], acc);
    }
    if (p0 + MB >= np) break;
#pragma unroll
    for (int i = 0; i < MB; ++i) x[i] = pall[min(p0 + MB + i, np - 1) * pstride + P_OUT + dim];
  }
  a.out[((int64_t)b * a.hq + hqi) * FD + dim] = acc * inv;
}

// ---------------------------------------------------------------- host side
void fast_plan_host(int batch, int hkv, int max_comp, int max_sink, int max_res, bool uniform, int cus, int& nwg,
                    int& chunks, int& vmax) {
  const int64_t pb = (max_comp + 31) / 32;
  const int64_t W = pb > 0 ? pb : (max_sink + max_res > 0 ? 1 : 0);
  const int64_t U = (int64_t)batch * hkv * W;
  int64_t n = (U + 7) / 8;  // at least one unit per wave
  if (n < 1) n = 1;
  if (n > cus) n = cus;
  nwg = (int)n;
  chunks = uniform ? 1 : 16;
  vmax = chunks * nwg + batch * hkv;
}

void fast_uniform_plan(int batch, int hkv, int max_comp, int max_sink, int max_res, int nwg, int chunks, int& T,
                       int& nu, int& V) {
  const int64_t pb = (max_comp + 31) / 32;
  const int64_t W = pb > 0 ? pb : (max_sink + max_res > 0 ? 1 : 0);
  const int64_t U = (int64_t)batch * hkv * W;
  const int64_t div = (int64_t)chunks * nwg;
  int64_t t = (U + div - 1) / div;
  if (t < 1) t = 1;
  T = (int)((t + FW - 1) / FW * FW);
  nu = (int)((W + T - 1) / T);
  V = batch * hkv * nu;
}

template <int G, int QB>
static void launch_g(const FastArgs& a, int merge, hipStream_t s) {
  hipLaunchKernelGGL((decode_partials_kernel<G, QB>), dim3(a.nwg), dim3(FT), 0, s, a);
  if (merge) hipLaunchKernelGGL((decode_merge_kernel<G>), dim3(a.hq, a.batch), dim3(RMT), 0, s, a);
}

int launch_fast_decode(const FastArgs& a, int G, int qb, int merge, hipStream_t s) {
  switch (G * 4 + qb) {
    case 4: launch_g<1, 0>(a, merge, s); break;
    case 5: launch_g<1, 1>(a, merge, s); break;
    case 6: launch_g<1, 2>(a, merge, s); break;
    case 8: launch_g<2, 0>(a, merge, s); break;
    case 9: launch_g<2, 1>(a, merge, s); break;
    case 10: launch_g<2, 2>(a, merge, s); break;
    case 16: launch_g<4, 0>(a, merge, s); break;
    case 17: launch_g<4, 1>(a, merge, s); break;
    case 18: launch_g<4, 2>(a, merge, s); break;
    case 32: launch_g<8, 0>(a, merge, s); break;
    case 33: launch_g<8, 1>(a, merge, s); break;
    case 34: launch_g<8, 2>(a, merge, s); break;
    default: return -1;
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_fast_merge_qjl(const FastArgs& a, int G, int qv, hipStream_t s) {
  const dim3 grid(a.hq, a.batch);
  switch (G * 4 + qv) {
    case 5: hipLaunchKernelGGL((decode_merge_kernel<1, 1>), grid, dim3(RMT), 0, s, a); break;
    case 6: hipLaunchKernelGGL((decode_merge_kernel<1, 2>), grid, dim3(RMT), 0, s, a); break;
    case 9: hipLaunchKernelGGL((decode_merge_kernel<2, 1>), grid, dim3(RMT), 0, s, a); break;
    case 10: hipLaunchKernelGGL((decode_merge_kernel<2, 2>), grid, dim3(RMT), 0, s, a); break;
    case 17: hipLaunchKernelGGL((decode_merge_kernel<4, 1>), grid, dim3(RMT), 0, s, a); break;
    case 18: hipLaunchKernelGGL((decode_merge_kernel<4, 2>), grid, dim3(RMT), 0, s, a); break;
    case 33: hipLaunchKernelGGL((decode_merge_kernel<8, 1>), grid, dim3(RMT), 0, s, a); break;
    case 34: hipLaunchKernelGGL((decode_merge_kernel<8, 2>), grid, dim3(RMT), 0, s, a); break;
    default: return -1;
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_partial_merge(float* part, int nwg, int G, int hq, int hkv, int batch, float* out, hipStream_t s) {
  OrigMergeArgs a{part, out, nwg, hq, hkv};
  const dim3 grid(2, hq, batch);
  switch (G) {
    case 1: hipLaunchKernelGGL((orig_merge_kernel<1>), grid, dim3(64), 0, s, a); break;
    case 2: hipLaunchKernelGGL((orig_merge_kernel<2>), grid, dim3(64), 0, s, a); break;
    case 4: hipLaunchKernelGGL((orig_merge_kernel<4>), grid, dim3(64), 0, s, a); break;
    default: hipLaunchKernelGGL((orig_merge_kernel<8>), grid, dim3(64), 0, s, a); break;
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace tq
