// Decode attention over a TurboQuant cache on gfx950 (split-T flash decoding).
//
// For sequence b, kv head g and its G = hq/hkv query heads the cache holds
// [sink fp16 | compressed | residual fp16] tokens. Compressed tokens are scored
// without dequantising (docs/FUSED_ATTENTION_DESIGN.md:62-67):
//     q . k_hat = n_k * (q @ R^T) . c[idx_k]
// and values are accumulated in rotated space with one inverse rotation at the
// end (docs/FULL_FUSED_ATTENTION_RESULTS.md:34-40):
//     sum_t p_t v_hat_t = (sum_t p_t n_t c[idx_t]) @ R.
// With the QJL sketch (qjl.py:70-94) the corrections are
//     q . dk = sqrt(pi/2)/D * gamma * (S q) . z,
//     sum_t p_t dv_t = sqrt(pi/2)/D * (sum_t p_t gamma_t z_t) @ S.
//
// Launches: (1) rotate / scale the queries, (2) one workgroup per (token
// chunk, kv head, sequence) writes a partial (max, sum, acc) per query head,
// (3) one workgroup per (query head, sequence) merges the partials, applies
// R once, adds the fp16-segment and QJL terms and normalises.

#include <math.h>

#include <mutex>

#include "tq_common.h"
#include "tq_decode_fast.h"

namespace tq {

constexpr int CHUNK = 256;   // tokens per partial
constexpr int NT = 256;      // threads per workgroup
constexpr float SQRT_HALF_PI = 1.2533141373155003f;

// Per-sequence lengths read from device arrays are clamped to the bounds the
// host checked (tq_abi.h: 0 <= len_b <= max_*, 0 <= res_start_b < res_cap), so
// an inconsistent array cannot send a kernel past the stores, sink or ring.
__device__ inline int clamp_len(int v, int mx) { return min(max(v, 0), mx); }
__device__ inline int seq_comp(const tq_attn_desc& d, int b) {
  return d.comp_len ? clamp_len(d.comp_len[b], d.max_comp) : d.max_comp;
}
__device__ inline int seq_ring_start(const tq_attn_desc& d, int b) {
  return d.res_start ? clamp_len(d.res_start[b], max(d.res_cap - 1, 0)) : d.res_start0;
}

struct AttnArgs {
  tq_attn_desc d;
  int D;
  const float* rot;   // key codec R: query rotation
  const float* vrot;  // value codec R: inverse rotation of the output
  const float* kc_hi;
  const float* kc_lo;
  const float* vc_hi;
  const float* vc_lo;
  const float* proj;
  int m;  // qjl projections (0 = off)
  int kb_hi, kb_lo, ks, vb_hi, vb_lo, vs;
  int k_row_hi, k_row_lo, v_row_hi, v_row_lo, row_sign;
  float* qr;    // (B, Hq, D)  scale * q @ R^T
  float* qs;    // (B, Hq, D)  scale * q
  float* sq;    // (B, Hq, m)  S @ (scale * q)
  float* part;  // (B, Hq, nch, PS)
  int nc, ns, nr, nch, ps;
  int c0;    // first chunk of a chunk_kernel launch
  int gsub;  // launch groups per kv head: a chunk_kernel<D, G> group holds G = (hq / hkv) / gsub query heads
};

// Column of the low-width segment in a staged code row: the hi bytes rounded
// up to a dword, so dot_codes reads both segments as aligned dwords (head_dim
// 96 at 2.5 bits has an 18-byte hi segment).
__host__ __device__ inline int lo_col(int row_hi) { return (row_hi + 3) & ~3; }

// Bytes dot_codes reads for a segment of n codes: whole 32-code groups of
// 4 * bits bytes (a trailing 16-code half group reads a full group).
__host__ __device__ inline int seg_span(int n, int bits) { return n > 0 ? (n + 31) / 32 * 4 * bits : 0; }

// LDS row stride of chunk_kernel's staged code rows: the longer of a key and a
// value row (hi bytes, then lo bytes at lo_col), covering every dword the key
// dot products read, in dwords rounded up to an odd count so that the rows of
// neighbouring tokens start in different banks.
__host__ __device__ inline int tile_stride(const AttnArgs& a) {
  const int kspan = max(seg_span(a.ks, a.kb_hi), a.k_row_lo ? lo_col(a.k_row_hi) + seg_span(a.D - a.ks, a.kb_lo) : 0);
  const int vspan = a.v_row_lo ? lo_col(a.v_row_hi) + a.v_row_lo : a.v_row_hi;
  const int b = max(max(kspan, a.k_row_hi), vspan);
  return 4 * (((b + 3) / 4) | 1);
}

__host__ __device__ inline int part_stride(int D, int m) { return ((2 + D + m) + 3) & ~3; }

// Query row (b, h, query token qi) of the call: q is (batch, hq, n_q, d).
// The general path treats query token qi of sequence b as its own row vb =
// b n_q + qi of the workspace (qr / qs / sq / partials are (batch n_q, hq, .)).
__device__ inline int nq_of(const tq_attn_desc& d) { return d.n_q > 1 ? d.n_q : 1; }

__global__ void prologue_kernel(AttnArgs a) {
  extern __shared__ float sm[];
  const int h = blockIdx.x, vb = blockIdx.y, D = a.D;
  const int nq = nq_of(a.d), b = vb / nq, qi = vb % nq;
  const int64_t qin = (((int64_t)b * a.d.hq + h) * nq + qi) * D;
  const int64_t qo = ((int64_t)vb * a.d.hq + h) * D;
  float* qsm = sm;
  for (int i = threadIdx.x; i < D; i += blockDim.x) {
    const float v = a.d.scale * load_elem(a.d.q, qin + i, a.d.q_dtype);
    qsm[i] = v;
    a.qs[qo + i] = v;
  }
  __syncthreads();
  for (int j = threadIdx.x; j < D; j += blockDim.x) {
    const float* rj = a.rot + (int64_t)j * D;
    float acc = 0.f;
    for (int i = 0; i < D; ++i) acc = fmaf(qsm[i], rj[i], acc);
    a.qr[qo + j] = acc;
  }
  if (a.m > 0) {
    const int64_t so = ((int64_t)vb * a.d.hq + h) * a.m;
    for (int i = threadIdx.x; i < a.m; i += blockDim.x) {
      const float* si = a.proj + (int64_t)i * D;
      float acc = 0.f;
      for (int k = 0; k < D; ++k) acc = fmaf(qsm[k], si[k], acc);
      a.sq[so + i] = acc;
    }
  }
}

// Code of dimension j in a packed row (LSB-first bitstream).
__device__ inline uint32_t code_at(const uint8_t* row, int j, int bits) {
  const int bit = bits * j;
  uint32_t v = row[bit >> 3] >> (bit & 7);
  if ((bit & 7) + bits > 8) v |= (uint32_t)row[(bit >> 3) + 1] << (8 - (bit & 7));
  return v & ((1u << bits) - 1u);
}

// Rows [0, n) of `row_bytes` bytes each, contiguous at src, into LDS rows of
// `stride` bytes starting at column `col` (dword copies when the rows, the
// column and the source are 4-byte aligned).
__device__ inline void stage_rows(uint8_t* dst, int stride, int col, const uint8_t* src, int row_bytes, int n) {
  if (row_bytes <= 0 || n <= 0) return;
  const int tid = threadIdx.x;
  // SB loads per thread are issued before the first LDS store: one memory
  // round trip per SB * NT elements (a load-store loop waits once per element)
  constexpr int SB = 8;
  if ((row_bytes & 3) == 0 && (col & 3) == 0 && (reinterpret_cast<uintptr_t>(src) & 3) == 0) {
    const int rw = row_bytes >> 2, total = n * rw;
    const uint32_t* sw = reinterpret_cast<const uint32_t*>(src);
    for (int e0 = tid; e0 < total; e0 += SB * NT) {
      uint32_t v[SB];
#pragma unroll
      for (int u = 0; u < SB; ++u) v[u] = e0 + u * NT < total ? sw[e0 + u * NT] : 0u;
#pragma unroll
      for (int u = 0; u < SB; ++u) {
        const int e = e0 + u * NT;
        if (e < total) {
          const int t = e / rw, k = e - t * rw;
          *reinterpret_cast<uint32_t*>(dst + t * stride + col + 4 * k) = v[u];
        }
      }
    }
  } else {
    const int total = n * row_bytes;
    for (int e0 = tid; e0 < total; e0 += SB * NT) {
      uint8_t v[SB];
#pragma unroll
      for (int u = 0; u < SB; ++u) v[u] = e0 + u * NT < total ? src[e0 + u * NT] : (uint8_t)0;
#pragma unroll
      for (int u = 0; u < SB; ++u) {
        const int e = e0 + u * NT;
        if (e < total) {
          const int t = e / row_bytes, k = e - t * row_bytes;
          dst[t * stride + col + k] = v[u];
        }
      }
    }
  }
}

// s[h] += sum_{j < nd} q[h][j0 + j] * lut[code j] for BITS-wide LSB-first
// codes in a 4-byte-aligned LDS row; nd and j0 multiples of 16. The codes of
// 32 dims are BITS dwords, read once; shifts are compile-time constants. A
// trailing group of 16 codes (head_dim 96 split in halves of 48) reads the
// BITS dwords of a full group, of which it uses the first 2 BITS bytes (the
// row stride, tile_stride, covers every dword read; bits read past a
// segment's codes are discarded).
template <int BITS, int D, int G>
__device__ inline void dot_codes(const uint8_t* row, int nd, const float* lut, const float (*q)[D], int j0,
                                 float (&s)[G]) {
  const uint32_t* rw = reinterpret_cast<const uint32_t*>(row);
  for (int jb = 0; jb < nd; jb += 32) {
    uint32_t wd[BITS];
#pragma unroll
    for (int i = 0; i < BITS; ++i) wd[i] = rw[(jb >> 5) * BITS + i];
    const bool half = nd - jb < 32;
#pragma unroll
    for (int j4 = 0; j4 < 32; j4 += 4) {
      if (j4 >= 16 && half) break;
      float cv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int bit = BITS * (j4 + u);
        uint32_t v = wd[bit >> 5] >> (bit & 31);
        if ((bit & 31) + BITS > 32) v |= wd[(bit >> 5) + 1] << (32 - (bit & 31));
        cv[u] = lut[v & ((1u << BITS) - 1u)];
      }
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float4 qq = *reinterpret_cast<const float4*>(&q[h][j0 + jb + j4]);
        s[h] = fmaf(qq.x, cv[0], s[h]);
        s[h] = fmaf(qq.y, cv[1], s[h]);
        s[h] = fmaf(qq.z, cv[2], s[h]);
        s[h] = fmaf(qq.w, cv[3], s[h]);
      }
    }
  }
}

// Up to four row sets staged together (dword path: every source, row size
// and column 4-byte aligned): each pass requests SB dwords of every source
// before any LDS store, so the four sets cost one memory round trip per pass.
struct StageSrc {
  uint8_t* dst;
  int col;
  const uint8_t* src;
  int row_bytes;
};
__device__ inline bool stage_aligned(const StageSrc& q) {
  return q.row_bytes <= 0 || ((q.row_bytes & 3) == 0 && (q.col & 3) == 0 && (reinterpret_cast<uintptr_t>(q.src) & 3) == 0);
}
__device__ inline void stage_rows_multi(const StageSrc (&S)[4], int stride, int n) {
  if (n <= 0) return;
  bool ok = true;
#pragma unroll
  for (int q = 0; q < 4; ++q) ok = ok && stage_aligned(S[q]);
  if (!ok) {
#pragma unroll
    for (int q = 0; q < 4; ++q) stage_rows(S[q].dst, stride, S[q].col, S[q].src, S[q].row_bytes, n);
    return;
  }
  constexpr int SB = 8;
  const int tid = threadIdx.x;
  int tot[4], rw[4], mx = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    rw[q] = S[q].row_bytes > 0 ? S[q].row_bytes >> 2 : 0;
    tot[q] = n * rw[q];
    mx = max(mx, tot[q]);
  }
  for (int e0 = tid; e0 < mx; e0 += SB * NT) {
    uint32_t v[4][SB];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int u = 0; u < SB; ++u) {
        const int e = e0 + u * NT;
        v[q][u] = e < tot[q] ? reinterpret_cast<const uint32_t*>(S[q].src)[e] : 0u;
      }
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int u = 0; u < SB; ++u) {
        const int e = e0 + u * NT;
        if (e < tot[q]) {
          const int t = e / rw[q], k = e - t * rw[q];
          *reinterpret_cast<uint32_t*>(S[q].dst + t * stride + S[q].col + 4 * k) = v[q][u];
        }
      }
  }
}

template <int D, int G>
__device__ inline void dot_codes_bits(int bits, const uint8_t* row, int nd, const float* lut, const float (*q)[D],
                                      int j0, float (&s)[G]) {
  switch (bits) {
    case 1: dot_codes<1, D, G>(row, nd, lut, q, j0, s); break;
    case 2: dot_codes<2, D, G>(row, nd, lut, q, j0, s); break;
    case 3: dot_codes<3, D, G>(row, nd, lut, q, j0, s); break;
    default: dot_codes<4, D, G>(row, nd, lut, q, j0, s); break;
  }
}

// zs[h] = sum_{i < m} sq[h][i] * z_i, z_i = +1 where sign bit i is set, else
// -1 (LSB-first bits in a 4-byte-aligned LDS row; m a multiple of 32)
template <int G, int MAXM>
__device__ inline void dot_signs(const uint8_t* row, int m, const float (*sq)[MAXM], float (&zs)[G]) {
  const uint32_t* rw = reinterpret_cast<const uint32_t*>(row);
  for (int ib = 0; ib < m; ib += 32) {
    const uint32_t wd = rw[ib >> 5];
#pragma unroll
    for (int i4 = 0; i4 < 32; i4 += 4) {
      float z[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) z[u] = ((wd >> (i4 + u)) & 1u) ? 1.f : -1.f;
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float4 qq = *reinterpret_cast<const float4*>(&sq[h][ib + i4]);
        zs[h] = fmaf(qq.x, z[0], zs[h]);
        zs[h] = fmaf(qq.y, z[1], zs[h]);
        zs[h] = fmaf(qq.z, z[2], zs[h]);
        zs[h] = fmaf(qq.w, z[3], zs[h]);
      }
    }
  }
}

// One chunk of CHUNK tokens of one segment for the G query heads of kv head g:
// thread t scores token t (packed tokens from code rows staged in LDS,
// fp16 tokens from memory), the chunk's softmax weights go to LDS, then
// thread (dim j, token slice) accumulates the weighted values of dim j for
// every head; with QJL the sign sketches are staged too and the value term
// sum_t p_t gamma_t z_t is accumulated per projection.
template <int DP, int G>
__global__ __launch_bounds__(NT) void chunk_kernel(AttnArgs a) {
  // DP: an upper bound of the head_dim D (a multiple of 16), the row stride
  // of the query arrays
  const int D = a.D;
  const int TSL = NT / D > 0 ? NT / D : 1;       // token slices of the PV phase (threads per dim)
  const int PER = ((CHUNK / TSL) + 3) & ~3;      // tokens per slice (whole float4 groups of weights)
  constexpr int MAXM = 256;
  // LDS row strides of staged code rows (at most 4 bits per dim) and sign
  // rows, padded by one dword so that the rows of neighbouring tokens start
  // in different banks
  const int KR = tile_stride(a);
  constexpr int SR = MAXM / 8 + 4;
  __shared__ __align__(16) float qv[G][DP];  // rotated (compressed) or plain (fp16) scaled query
  __shared__ __align__(16) float w[G][CHUNK];   // p * n_v (or p) per token
  __shared__ float red[G][NT / 64];
  __shared__ float mx[G], lsum[G];
  __shared__ float klut[2][16], vlut[2][16];
  // per-thread partial sums of the PV / QJL phases, over w once the PV loop is done
  static_assert(NT == CHUNK, "slice aliases w");
  float (*slice)[NT] = reinterpret_cast<float (*)[NT]>(&w[0][0]);
  // dynamic LDS sized per launch: the key and value code rows at the codecs'
  // row size, then (with a sketch only) p * gamma_v per token, S q per head and
  // the key and value sign rows; four workgroups of K3.5/V3.5 fit a CU
  extern __shared__ __align__(16) float sm[];
  uint8_t* ktile = reinterpret_cast<uint8_t*>(sm);  // key code rows: hi bytes, then lo bytes
  uint8_t* vtile = ktile + CHUNK * KR;              // value code rows
  float* qj = reinterpret_cast<float*>(vtile + CHUNK * KR);
  float (*pg)[CHUNK] = reinterpret_cast<float (*)[CHUNK]>(qj);
  float (*sqv)[MAXM] = reinterpret_cast<float (*)[MAXM]>(qj + G * CHUNK);
  uint8_t* ksg = reinterpret_cast<uint8_t*>(qj + G * CHUNK + G * MAXM);
  uint8_t* vsg = ksg + CHUNK * SR;
  // group g: query heads [g G, g G + G) of kv head g / gsub; query token qi
  // of sequence b (row vb of the workspace)
  const int c = blockIdx.x + a.c0, g = blockIdx.y, vb = blockIdx.z;
  const int nq = nq_of(a.d), b = vb / nq, qi = vb % nq;
  const int hq = a.d.hq, tid = threadIdx.x;
  const int row = b * a.d.hkv + g / a.gsub;

  // segment of this chunk
  int seg, base;
  if (c < a.nc) { seg = 0; base = c * CHUNK; }
  else if (c < a.nc + a.ns) { seg = 1; base = (c - a.nc) * CHUNK; }
  else { seg = 2; base = (c - a.nc - a.ns) * CHUNK; }
  const int len_c = seq_comp(a.d, b);
  const int len_s = a.d.sink_len ? clamp_len(a.d.sink_len[b], a.d.max_sink) : a.d.max_sink;
  const int len_r = a.d.res_len ? clamp_len(a.d.res_len[b], a.d.max_res) : a.d.max_res;
  const int len = seg == 0 ? len_c : seg == 1 ? len_s : len_r;
  const int nvalid = max(0, min(CHUNK, len - base));
  // causal: the n_q queries are the last n_q tokens of [sink | compressed |
  // residual]; query qi sees positions <= total - n_q + qi (cache.py:722-724)
  const int pos0 = (seg == 0 ? len_s : seg == 1 ? 0 : len_s + len_c) + base;  // position of token base
  const int lim = len_s + len_c + len_r - nq + qi;

  const bool packed = seg == 0;
  const bool qjl = packed && a.m > 0;
  for (int e = tid; e < G * D; e += NT) {
    const int h = e / D, j = e % D;
    const int64_t qo = ((int64_t)vb * hq + g * G + h) * D + j;
    qv[h][j] = packed ? a.qr[qo] : a.qs[qo];
  }
  if (qjl) {
    for (int e = tid; e < G * a.m; e += NT) {
      const int h = e / a.m, i = e % a.m;
      sqv[h][i] = a.sq[((int64_t)vb * hq + g * G + h) * a.m + i];
    }
  }
  if (tid < 16) {
    klut[0][tid] = tid < (1 << a.kb_hi) ? a.kc_hi[tid] : 0.f;
    klut[1][tid] = tid < (1 << a.kb_lo) ? a.kc_lo[tid] : 0.f;
    vlut[0][tid] = tid < (1 << a.vb_hi) ? a.vc_hi[tid] : 0.f;
    vlut[1][tid] = tid < (1 << a.vb_lo) ? a.vc_lo[tid] : 0.f;
  }
  // stage the chunk's code rows (and sign rows) in LDS
  if (packed) {
    const tq_store& ks = a.d.kstore;
    const tq_store& vs = a.d.vstore;
    const StageSrc S[4] = {
        {ktile, 0, ks.codes_hi + (int64_t)row * ks.hi_head_stride + (int64_t)base * a.k_row_hi, a.k_row_hi},
        {ktile, lo_col(a.k_row_hi),
         a.k_row_lo ? ks.codes_lo + (int64_t)row * ks.lo_head_stride + (int64_t)base * a.k_row_lo : nullptr,
         a.k_row_lo},
        {vtile, 0, vs.codes_hi + (int64_t)row * vs.hi_head_stride + (int64_t)base * a.v_row_hi, a.v_row_hi},
        {vtile, lo_col(a.v_row_hi),
         a.v_row_lo ? vs.codes_lo + (int64_t)row * vs.lo_head_stride + (int64_t)base * a.v_row_lo : nullptr,
         a.v_row_lo}};
    stage_rows_multi(S, KR, nvalid);
    if (qjl) {
      stage_rows(ksg, SR, 0, ks.signs + (int64_t)row * ks.sign_head_stride + (int64_t)base * a.row_sign, a.row_sign,
                 nvalid);
      stage_rows(vsg, SR, 0, vs.signs + (int64_t)row * vs.sign_head_stride + (int64_t)base * a.row_sign, a.row_sign,
                 nvalid);
    }
  }
  // the token's norms (and gammas) requested with the staging loads
  float nk_t = 0.f, nv_t = 1.f, gk_t = 0.f, gv_t = 0.f;
  if (packed && tid < nvalid) {
    nk_t = a.d.kstore.norms[(int64_t)row * a.d.kstore.norm_head_stride + base + tid];
    nv_t = a.d.vstore.norms[(int64_t)row * a.d.vstore.norm_head_stride + base + tid];
    if (qjl) {
      gk_t = a.d.kstore.gamma[(int64_t)row * a.d.kstore.gamma_head_stride + base + tid];
      gv_t = a.d.vstore.gamma[(int64_t)row * a.d.vstore.gamma_head_stride + base + tid];
    }
  }
  __syncthreads();

  // ---- scores: thread t owns token base + t
  float s[G];
#pragma unroll
  for (int h = 0; h < G; ++h) s[h] = -INFINITY;
  const int t = tid;
  if (t < nvalid && pos0 + t <= lim) {
#pragma unroll
    for (int h = 0; h < G; ++h) s[h] = 0.f;
    if (packed) {
      const uint8_t* kr = ktile + t * KR;
      dot_codes_bits<DP, G>(a.kb_hi, kr, a.ks, klut[0], qv, 0, s);
      if (a.ks < D) dot_codes_bits<DP, G>(a.kb_lo, kr + lo_col(a.k_row_hi), D - a.ks, klut[1], qv, a.ks, s);
      const float nk = nk_t;
#pragma unroll
      for (int h = 0; h < G; ++h) s[h] *= nk;
      if (qjl) {
        const float gk = gk_t;
        float zs[G];
#pragma unroll
        for (int h = 0; h < G; ++h) zs[h] = 0.f;
        dot_signs<G, MAXM>(ksg + t * SR, a.m, sqv, zs);
        const float coef = SQRT_HALF_PI / (float)D * gk;
#pragma unroll
        for (int h = 0; h < G; ++h) s[h] = fmaf(coef, zs[h], s[h]);
      }
    } else {
      const void* kp;
      int64_t ko;
      if (seg == 1) {
        kp = a.d.sink_k;
        ko = (int64_t)row * a.d.sink_head_stride + (int64_t)(base + t) * D;
      } else {
        const int st = seq_ring_start(a.d, b);
        const int pos = (st + base + t) % a.d.res_cap;
        kp = a.d.res_k;
        ko = (int64_t)row * a.d.res_head_stride + (int64_t)pos * D;
      }
      const int esz = a.d.kv_dtype == TQ_F32 ? 4 : 2;
      const uint8_t* kb = static_cast<const uint8_t*>(kp) + ko * esz;
      if ((reinterpret_cast<uintptr_t>(kb) & 15) == 0) {
        // the token's row in 16-byte pieces, KB of them requested at once
        constexpr int KB = 8;
        const int npc = D * esz / 16;  // pieces per row
        for (int c0 = 0; c0 < npc; c0 += KB) {
          uint4 raw[KB];
#pragma unroll
          for (int u = 0; u < KB; ++u) raw[u] = *reinterpret_cast<const uint4*>(kb + 16 * min(c0 + u, npc - 1));
#pragma unroll
          for (int u = 0; u < KB; ++u) {
            if (c0 + u >= npc) break;
            const uint32_t wd[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
            if (esz == 4) {
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const int j = 4 * (c0 + u) + e;
                const float kv = __uint_as_float(wd[e]);
#pragma unroll
                for (int h = 0; h < G; ++h) s[h] = fmaf(qv[h][j], kv, s[h]);
              }
            } else {
#pragma unroll
              for (int e = 0; e < 8; ++e) {
                const int j = 8 * (c0 + u) + e;
                const uint32_t hb = (wd[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
                const float kv = a.d.kv_dtype == TQ_BF16 ? __uint_as_float(hb << 16)
                                                         : (float)__builtin_bit_cast(_Float16, (uint16_t)hb);
#pragma unroll
                for (int h = 0; h < G; ++h) s[h] = fmaf(qv[h][j], kv, s[h]);
              }
            }
          }
        }
      } else {
        for (int j = 0; j < D; ++j) {
          const float kv = load_elem(kp, ko + j, a.d.kv_dtype);
#pragma unroll
          for (int h = 0; h < G; ++h) s[h] = fmaf(qv[h][j], kv, s[h]);
        }
      }
    }
  }

  // ---- chunk max per head
  const int lane = tid & 63, wv = tid >> 6;
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float v = s[h];
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    if (lane == 0) red[h][wv] = v;
  }
  __syncthreads();
  if (tid < G) {
    float v = red[tid][0];
    for (int k = 1; k < NT / 64; ++k) v = fmaxf(v, red[tid][k]);
    mx[tid] = v;
  }
  __syncthreads();
  float p[G];
#pragma unroll
  for (int h = 0; h < G; ++h) p[h] = (t < nvalid && mx[h] > -INFINITY) ? expf(s[h] - mx[h]) : 0.f;
  // weights for the PV phase
  {
    float nv = 1.f, gv = 0.f;
    if (packed && t < nvalid) {
      nv = nv_t;
      if (qjl) gv = gv_t;
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      w[h][t] = p[h] * nv;
      if (qjl) pg[h][t] = p[h] * gv;
    }
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float v = p[h];
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    if (lane == 0) red[h][wv] = v;
  }
  __syncthreads();
  if (tid < G) {
    float v = 0.f;
    for (int k = 0; k < NT / 64; ++k) v += red[tid][k];
    lsum[tid] = v;
  }
  __syncthreads();

  // ---- PV: thread (j, sl) accumulates dim j of every head over token slice
  // sl (TSL slices of CHUNK / TSL tokens), so each code is decoded once for
  // all G heads; the slices are summed through LDS. Weights of 4 tokens per
  // LDS read (tokens past nvalid have weight 0).
  const int n4 = (nvalid + 3) & ~3;
  float* outp = a.part;
  {
    const int j = tid % D, sl = tid / D;
    const int t_lo = sl * PER, t_hi = min(n4, t_lo + PER);
    float acc[G];
#pragma unroll
    for (int h = 0; h < G; ++h) acc[h] = 0.f;
    if (tid < D * TSL) {
      if (packed) {
        const bool hi = j < a.vs;
        const int bits = hi ? a.vb_hi : a.vb_lo;
        const int jl = hi ? j : j - a.vs;
        const int off = hi ? 0 : lo_col(a.v_row_hi);
        const float* lut = vlut[hi ? 0 : 1];
        for (int tt = t_lo; tt < t_hi; tt += 4) {
          float cv[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) cv[u] = lut[code_at(vtile + (tt + u) * KR + off, jl, bits)];
#pragma unroll
          for (int h = 0; h < G; ++h) {
            const float4 wq = *reinterpret_cast<const float4*>(&w[h][tt]);
            acc[h] = fmaf(wq.x, cv[0], acc[h]);
            acc[h] = fmaf(wq.y, cv[1], acc[h]);
            acc[h] = fmaf(wq.z, cv[2], acc[h]);
            acc[h] = fmaf(wq.w, cv[3], acc[h]);
          }
        }
      } else {
        // fp16 / bf16 / f32 tokens: VB tokens' values requested before any is
        // used (a load-use loop waits one memory round trip per token)
        constexpr int VB = 16;
        const void* vp = seg == 1 ? a.d.sink_v : a.d.res_v;
        const int st = seg == 1 ? 0 : seq_ring_start(a.d, b);
        const int tend = min(t_hi, nvalid);
        for (int tt0 = t_lo; tt0 < tend; tt0 += VB) {
          float vv[VB];
#pragma unroll
          for (int u = 0; u < VB; ++u) {
            const int tt = min(tt0 + u, tend - 1);
            const int64_t vo = seg == 1 ? (int64_t)row * a.d.sink_head_stride + (int64_t)(base + tt) * D
                                        : (int64_t)row * a.d.res_head_stride + (int64_t)((st + base + tt) % a.d.res_cap) * D;
            vv[u] = load_elem(vp, vo + j, a.d.kv_dtype);
          }
#pragma unroll
          for (int u = 0; u < VB; ++u) {
            if (tt0 + u < tend) {
#pragma unroll
              for (int h = 0; h < G; ++h) acc[h] = fmaf(w[h][tt0 + u], vv[u], acc[h]);
            }
          }
        }
      }
    }
    __syncthreads();  // every thread is past its reads of w (slice aliases it)
#pragma unroll
    for (int h = 0; h < G; ++h) slice[h][tid] = acc[h];
  }
  __syncthreads();
  for (int e = tid; e < G * D; e += NT) {
    const int h = e / D, j = e % D;
    float v = 0.f;
#pragma unroll
    for (int sl = 0; sl < TSL; ++sl) v += slice[h][sl * D + j];
    outp[(((int64_t)vb * hq + g * G + h) * a.nch + c) * a.ps + 2 + j] = v;
  }
  // QJL value term az[h][i] = sum_t p_t gamma_t z_t,i: thread (i, sl) over
  // token slice sl of NT / m, each sign bit read once for all G heads
  if (qjl) {
    __syncthreads();
    const int nsl = NT / a.m;  // m <= 256 = NT
    const int i = tid % a.m, sl = tid / a.m;
    const int per = CHUNK / nsl;
    const int t_lo = sl * per, t_hi = min(n4, t_lo + per);
    float acc[G];
#pragma unroll
    for (int h = 0; h < G; ++h) acc[h] = 0.f;
    if (sl < nsl) {
      for (int tt = t_lo; tt < t_hi; tt += 4) {
        float z[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) z[u] = ((vsg[(tt + u) * SR + (i >> 3)] >> (i & 7)) & 1u) ? 1.f : -1.f;
#pragma unroll
        for (int h = 0; h < G; ++h) {
          const float4 pq = *reinterpret_cast<const float4*>(&pg[h][tt]);
          acc[h] = fmaf(pq.x, z[0], acc[h]);
          acc[h] = fmaf(pq.y, z[1], acc[h]);
          acc[h] = fmaf(pq.z, z[2], acc[h]);
          acc[h] = fmaf(pq.w, z[3], acc[h]);
        }
      }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) slice[h][tid] = acc[h];
    __syncthreads();
    for (int e = tid; e < G * a.m; e += NT) {
      const int h = e / a.m, ii = e % a.m;
      float v = 0.f;
      for (int q = 0; q < nsl; ++q) v += slice[h][q * a.m + ii];
      outp[(((int64_t)vb * hq + g * G + h) * a.nch + c) * a.ps + 2 + D + ii] = v;
    }
  }
  if (tid < G) {
    float* pp = outp + (((int64_t)vb * hq + g * G + tid) * a.nch + c) * a.ps;
    pp[0] = mx[tid];
    pp[1] = lsum[tid];
  }
}

// Combine of the chunk partials of query head (b, h): the chunk weights
// exp(m_c - M) are computed once into LDS, then the weighted sums (rotated
// dims of the packed chunks, QJL projections, original-space dims of the fp16
// chunks) and the inverse rotation, with four independent accumulators so the
// loads of a loop overlap. 128 threads.
__global__ __launch_bounds__(128) void combine_kernel(AttnArgs a) {
  extern __shared__ float sm[];
  __shared__ float rmax[2], rsum[2];
  const int h = blockIdx.x, vb = blockIdx.y, D = a.D, tid = threadIdx.x;
  const int nq = nq_of(a.d), b = vb / nq, qi = vb % nq;
  const int hq = a.d.hq, nch = a.nch;
  const int64_t ps = a.ps;
  const float* pp = a.part + ((int64_t)vb * hq + h) * nch * ps;
  float* wc = sm;                       // [nch] chunk weights
  float* accr = sm + ((nch + 3) & ~3);  // [D] weighted rotated sum
  float* azs = accr + D;                // [m] weighted QJL projections
  float M = -INFINITY;
  for (int c = tid; c < nch; c += 128) M = fmaxf(M, pp[c * ps]);
  for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o));
  if ((tid & 63) == 0) rmax[tid >> 6] = M;
  __syncthreads();
  M = fmaxf(rmax[0], rmax[1]);
  float L = 0.f;
  for (int c = tid; c < nch; c += 128) {
    const float mc = pp[c * ps];
    const float wgt = mc > -INFINITY ? expf(mc - M) : 0.f;
    wc[c] = wgt;
    L = fmaf(wgt, pp[c * ps + 1], L);
  }
  for (int o = 32; o > 0; o >>= 1) L += __shfl_xor(L, o);
  if ((tid & 63) == 0) rsum[tid >> 6] = L;
  __syncthreads();
  L = rsum[0] + rsum[1];
  // sum over chunks [c0, c1) of wc[c] * pp[c * ps + col]; CU loads are
  // requested before they are used (one memory round trip per CU chunks)
  constexpr int CU = 16;
  auto wsum = [&](int c0, int c1, int col) {
    float r[CU];
#pragma unroll
    for (int u = 0; u < CU; ++u) r[u] = 0.f;
    int c = c0;
    for (; c + CU <= c1; c += CU) {
      float x[CU];
#pragma unroll
      for (int u = 0; u < CU; ++u) x[u] = pp[(c + u) * ps + col];
#pragma unroll
      for (int u = 0; u < CU; ++u) r[u] = fmaf(wc[c + u], x[u], r[u]);
    }
    for (; c < c1; ++c) r[0] = fmaf(wc[c], pp[c * ps + col], r[0]);
#pragma unroll
    for (int w = CU / 2; w > 0; w >>= 1)
#pragma unroll
      for (int u = 0; u < w; ++u) r[u] += r[u + w];
    return r[0];
  };
  // sum over rows i < n (a multiple of 4) of v[i] * mat[i * D + j], CU rows per batch
  auto matvec = [&](const float* v, const float* mat, int n, int j) {
    float r[CU];
#pragma unroll
    for (int u = 0; u < CU; ++u) r[u] = 0.f;
    int i = 0;
    for (; i + CU <= n; i += CU) {
      float x[CU];
#pragma unroll
      for (int u = 0; u < CU; ++u) x[u] = mat[(int64_t)(i + u) * D + j];
#pragma unroll
      for (int u = 0; u < CU; ++u) r[u] = fmaf(v[i + u], x[u], r[u]);
    }
    for (; i < n; ++i) r[0] = fmaf(v[i], mat[(int64_t)i * D + j], r[0]);
#pragma unroll
    for (int w = CU / 2; w > 0; w >>= 1)
#pragma unroll
      for (int u = 0; u < w; ++u) r[u] += r[u + w];
    return r[0];
  };
  for (int j = tid; j < D; j += 128) accr[j] = wsum(0, a.nc, 2 + j);
  for (int i = tid; i < a.m; i += 128) azs[i] = wsum(0, a.nc, 2 + D + i);
  __syncthreads();
  float* out = a.d.out + (((int64_t)b * hq + h) * nq + qi) * D;
  for (int j = tid; j < D; j += 128) {
    float o = matvec(accr, a.vrot, D, j) + wsum(a.nc, nch, 2 + j);
    if (a.m > 0) o = fmaf(SQRT_HALF_PI / (float)D, matvec(azs, a.proj, a.m, j), o);
    out[j] = (L > 0.f) ? o / L : 0.f;
  }
}

static void chunk_counts(const tq_attn_desc* d, int& nc, int& ns, int& nr) {
  nc = (d->max_comp + CHUNK - 1) / CHUNK;
  ns = (d->max_sink + CHUNK - 1) / CHUNK;
  nr = (d->max_res + CHUNK - 1) / CHUNK;
}

// G: query heads per launch group (1 .. 8)
template <int DP>
static void launch_chunks(const AttnArgs& a, int G, dim3 grid, hipStream_t s) {
  // dynamic LDS of chunk_kernel: the code rows, and the QJL arrays when the call has a sketch
  const size_t dl = 2 * (size_t)CHUNK * tile_stride(a) +
                    (a.m > 0 ? (size_t)G * (CHUNK + 256) * 4 + 2 * (size_t)CHUNK * (256 / 8 + 4) : 0);
  switch (G) {
    case 1: hipLaunchKernelGGL((chunk_kernel<DP, 1>), grid, dim3(NT), dl, s, a); break;
    case 2: hipLaunchKernelGGL((chunk_kernel<DP, 2>), grid, dim3(NT), dl, s, a); break;
    case 3: hipLaunchKernelGGL((chunk_kernel<DP, 3>), grid, dim3(NT), dl, s, a); break;
    case 4: hipLaunchKernelGGL((chunk_kernel<DP, 4>), grid, dim3(NT), dl, s, a); break;
    case 5: hipLaunchKernelGGL((chunk_kernel<DP, 5>), grid, dim3(NT), dl, s, a); break;
    case 6: hipLaunchKernelGGL((chunk_kernel<DP, 6>), grid, dim3(NT), dl, s, a); break;
    case 7: hipLaunchKernelGGL((chunk_kernel<DP, 7>), grid, dim3(NT), dl, s, a); break;
    default: hipLaunchKernelGGL((chunk_kernel<DP, 8>), grid, dim3(NT), dl, s, a); break;
  }
}

// Query heads per launch group of the general kernel for G query heads per
// kv head: the largest divisor of G that is at most 8.
static int group_heads(int G) {
  for (int k = 8; k > 1; --k)
    if (G % k == 0) return k;
  return 1;
}

// ---- QJL sketch terms around the K4/V2 kernels (K4 keys / V2 values with a
// 1-bit sketch, qjl.py:23-94 as in the general path): the key term of each
// compressed token's score (base 2) comes from a bias kernel for the
// uniform-batch kernels and is computed inside the persistent kernel (from
// the sketch and S q) for the others; the partials kernel stores the final
// scores, and after the merge a value kernel accumulates
// u_h = sum_t p_t gamma_t z_t per projection (p the normalised softmax
// weight of compressed token t) and a final kernel adds sqrt(pi/2)/d S^T u_h to
// the output, as combine_kernel does for the general path.
constexpr int QCH = 256;  // tokens per chunk of the QJL kernels (one chunk per value-kernel workgroup)
constexpr int QBC = 4;    // chunks per workgroup of the bias kernel (one sign-pattern table for all)

struct QjlArgs {
  tq_attn_desc d;
  const float* sq;      // (batch, hq, m) S (scale q), natural units (qjl_sq_kernel)
  const float* proj;    // (m, 128)
  int m;
  int ksign16, vsign16; // key / value sign rows 16-byte aligned with m a multiple of 128 (16-byte loads)
  float* bias;          // (batch*hkv*G, qb_hs) key term in base-2 score units
  const float* scores;  // (batch*hkv*G, qb_hs) final base-2 scores
  const float* ml;      // (batch, hq, 2) global max and sum of the merge
  float* upart;         // (batch, hq, nvc, m) value terms, one per value-kernel workgroup
  float* umax;          // (batch, hq, nvc) each value partial's reference max (value kernel with LOC)
  int64_t qb_hs;
  int nvc;              // value-kernel workgroups per (b, g), one partial each
  int qvc;              // chunks of QCH tokens per value-kernel workgroup
};

// S (scale q) of the G query heads of (b, g), natural units: 64 projections
// per workgroup, four threads per projection (thread t: projection 64 x + t /
// 4, dims 32 (t & 3) .. + 31 in float32 order, the four quarters added in a
// fixed order). The projection rows are requested before the queries arrive.
template <int G>
__global__ __launch_bounds__(256) void qjl_sq_kernel(QjlArgs a) {
  __shared__ float qsm[G][128];
  const int g = blockIdx.y, b = blockIdx.z, tid = threadIdx.x, m = a.m;
  const int i = 64 * blockIdx.x + (tid >> 2), kq = tid & 3;
  float4 s4[8];
  {
    const float* si = a.proj + (int64_t)min(i, m - 1) * 128 + 32 * kq;
#pragma unroll
    for (int k = 0; k < 8; ++k) s4[k] = *reinterpret_cast<const float4*>(si + 4 * k);
  }
  for (int e = tid; e < G * 128; e += 256)
    qsm[e >> 7][e & 127] =
        a.d.scale * load_elem(a.d.q, ((int64_t)b * a.d.hq + g * G + (e >> 7)) * 128 + (e & 127), a.d.q_dtype);
  __syncthreads();
  float acc[G];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const float* qh = &qsm[h][32 * kq];
    float x = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      x = fmaf(qh[4 * k], s4[k].x, x);
      x = fmaf(qh[4 * k + 1], s4[k].y, x);
      x = fmaf(qh[4 * k + 2], s4[k].z, x);
      x = fmaf(qh[4 * k + 3], s4[k].w, x);
    }
    // (q0 + q1) + (q2 + q3) over the four threads of the projection
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, true));  // lane ^ 1
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, true));  // lane ^ 2
    acc[h] = x;
  }
  if (kq == 0 && i < m) {
#pragma unroll
    for (int h = 0; h < G; ++h) const_cast<float*>(a.sq)[((int64_t)b * a.d.hq + g * G + h) * m + i] = acc[h];
  }
}

typedef _Float16 qh8 __attribute__((ext_vector_type(8)));
typedef float qf4 __attribute__((ext_vector_type(4)));
typedef uint32_t qu4 __attribute__((ext_vector_type(4)));

// The nw = m / 32 sign words of token row `p` (m / 8 bytes): 16-byte loads
// when the rows allow them (v16), else one word per load. NW4: words held,
// in groups of 4 (nw <= 4 NW4).
template <int NW4>
__device__ inline void load_sign_row(const uint8_t* p, int nw, bool v16, uint32_t (&sw)[4 * NW4]) {
  const uint32_t* wp = reinterpret_cast<const uint32_t*>(p);
  if (v16) {
#pragma unroll
    for (int q = 0; q < NW4; ++q) {
      const qu4 x = reinterpret_cast<const qu4*>(p)[q];
#pragma unroll
      for (int k = 0; k < 4; ++k) sw[4 * q + k] = x[k];
    }
  } else {
#pragma unroll
    for (int k = 0; k < 4 * NW4; ++k) sw[k] = k < nw ? wp[k] : 0u;
  }
}

// Key term of each compressed token: z_h = sum_k sign_k (S q_h)_k from a
// table of the 16 sign patterns of each 4 consecutive projections, lut[p][n][h]
// = sum_{j < 4} (bit j of n ? 1 : -1) (S q_h)_{4p + j} (one LDS read of G
// floats and G adds per 4 signs). Thread tid takes tokens (c QBC + i) QCH +
// tid, i < QBC: S q and all of its tokens' sign rows and gammas are requested
// up front, so the workgroup waits for one memory round trip.
template <int G, int NW4>
__global__ __launch_bounds__(NT) void qjl_bias_kernel(QjlArgs a) {
  constexpr int MAXM = 128 * NW4;
  __shared__ __align__(16) float lut[MAXM / 4][16][G];
  __shared__ float sqs[G][MAXM];
  const int c = blockIdx.x, g = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  const int row = b * a.d.hkv + g, m = a.m, nw = m / 32;
  const int comp = seq_comp(a.d, b);
  // past the sequence's last 32-token block the bias is never read (those
  // scores are masked after it is added)
  const int tend = min((int)a.qb_hs, (comp + 31) & ~31);
  if (c * QBC * QCH >= tend) return;
  constexpr int NSQ = (G * MAXM + NT - 1) / NT;
  float sqv[NSQ];
  {
    const float* sqp = a.sq + ((int64_t)b * a.d.hq + g * G) * m;  // the G rows are contiguous
#pragma unroll
    for (int i = 0; i < NSQ; ++i) sqv[i] = tid + NT * i < G * m ? sqp[tid + NT * i] : 0.f;
  }
  const tq_store& ks = a.d.kstore;
  uint32_t sw[QBC][4 * NW4];
  float gk[QBC];
#pragma unroll
  for (int i = 0; i < QBC; ++i) {
    const int tc = min((c * QBC + i) * QCH + tid, comp - 1);  // comp >= 1 here
    gk[i] = ks.gamma[(int64_t)row * ks.gamma_head_stride + tc];
    load_sign_row<NW4>(ks.signs + (int64_t)row * ks.sign_head_stride + (int64_t)tc * (m / 8), nw, a.ksign16 != 0, sw[i]);
  }
#pragma unroll
  for (int i = 0; i < NSQ; ++i)
    if (tid + NT * i < G * m) sqs[(tid + NT * i) / m][(tid + NT * i) % m] = sqv[i];
  __syncthreads();
  for (int e = tid; e < (m / 4) * 16 * G; e += NT) {
    const int h = e % G, n = (e / G) & 15, p = e / (16 * G);
    float v = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) v += ((n >> j) & 1) ? sqs[h][4 * p + j] : -sqs[h][4 * p + j];
    lut[p][n][h] = v;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < QBC; ++i) {
    const int t = (c * QBC + i) * QCH + tid;
    if (t >= tend) break;
    float zs[G];
#pragma unroll
    for (int h = 0; h < G; ++h) zs[h] = 0.f;
#pragma unroll
    for (int wi = 0; wi < 4 * NW4; ++wi) {
      if (wi >= nw) break;
      const uint32_t wd = sw[i][wi];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float* e = lut[8 * wi + k][(wd >> (4 * k)) & 15u];
#pragma unroll
        for (int h = 0; h < G; ++h) zs[h] += e[h];
      }
    }
    // the bias of the tokens past comp (up to the 32-token block) is 0
    const float coef = t < comp ? 1.4426950408889634f * SQRT_HALF_PI / 128.f * gk[i] : 0.f;
#pragma unroll
    for (int h = 0; h < G; ++h) a.bias[((int64_t)row * G + h) * a.qb_hs + t] = coef * zs[h];
  }
}

// max over the 64 lanes of a wave in VALU cross-lane moves: DPP rotations
// within each 16-lane row, then the four rows (every lane gets the result)
__device__ inline float wave_max_dpp(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, true)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x124, 0xF, 0xF, true)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x122, 0xF, 0xF, true)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x121, 0xF, 0xF, true)));
  const auto x = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(x[0]), __uint_as_float(x[1]));
  const auto y = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(y[0]), __uint_as_float(y[1]));
}

// max over the 64 lanes of a wave of non-negative floats, compared as their
// bit patterns (unsigned integers order them alike)
__device__ inline uint32_t wave_max_nonneg(float f) {
  uint32_t v = __float_as_uint(f);
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x124, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x122, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x121, 0xF, 0xF, true));
  const auto x = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = max(x[0], x[1]);
  const auto y = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return max(y[0], y[1]);
}

// the value of lane ^ 1 (DPP quad permutation 1, 0, 3, 2)
__device__ inline uint32_t lane_xor1(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, true);
}

// Chunks of QCH tokens per workgroup of the value kernel (the sign words of
// all of them are held in registers: fewer for the longer sketches).
template <int NW4>
constexpr int qjl_value_chunks() { return NW4 == 1 ? 4 : 2; }
static int qjl_value_chunks_host(int m) { return m > 128 ? qjl_value_chunks<2>() : qjl_value_chunks<1>(); }

// u_h = sum_t w_t z_t (w_t = 2^(s_t - M) gamma_t for head h, z_t the +-1
// sign row of token t) by MFMA 16x16x32 f16 over QV chunks of 256 tokens per
// workgroup, thread t = token t of each chunk:
//   A = W: row h the fp16 high part of head h's weights times 2^(14 - E_h)
//       (E_h the exponent of the workgroup's max weight of head h: none is
//       subnormal in fp16 but the tiny), row h + 8 the remainder; k = the 32
//       tokens of a block;
//   B = Z: k = the same tokens, column = one of 16 projections, built from a
//       word holding the 16 projection bits of two tokens in its halves: the
//       lane's bit shifted to bit 15 / 31 and or-ed into 0x3C00 gives 1 for a
//       clear bit and -1 for a set one, i.e. -z (the sums are negated back).
// Output rows h and h + 8 (lanes q4 and q4 + 2) added give head h. Wave w
// takes the projection tiles w, w + 4, ... Every chunk's loads are issued up
// front; one accumulator per tile runs over the chunks. The weights stay
// unnormalised (O(gamma), whatever the context length); -2^(E_h - 14) / L_h is
// applied in float32 to the sums.
// LOC: M is the workgroup's own max score of head h instead of the merged
// one (the kernel then runs before the merge, which weights the partial by
// 2^(M_loc - M) / L: umax holds M_loc), and E_h the exponent of the
// workgroup's largest residual norm (every weight is at most that norm); the
// sums are scaled by -2^(E_h - 14) alone.
template <int G, int NW4, bool LOC = false>
__global__ __launch_bounds__(NT) void qjl_value_kernel(QjlArgs a) {
  static_assert(NT == QCH, "thread t = token t of the chunk");
  constexpr int QV = qjl_value_chunks<NW4>();
  constexpr int MAXM = 128 * NW4;
  constexpr int YS = QCH / 2 + 32;  // row of ysm (+32 words: the rows the even and odd threads write sit 32 banks apart)
  // A operands, word (bk, q4, row, pair) at bk ASB + q4 ASQ + 4 row + pair:
  // the 16 rows of a (bk, q4) group contiguous (a lane's 16-byte read, 16
  // lanes over all banks); groups padded so that the words one wave writes
  // (two blocks x 4 groups x 4 pairs x 2 row halves) fall in 64 banks
  constexpr int ASQ = 68, ASB = 4 * ASQ;
  // ysm[c][p]: projections 16c .. 16c + 15 of token 2p (low half) and 2p + 1 (high half)
  __shared__ __align__(16) uint32_t ysm[MAXM / 16][YS];
  __shared__ __align__(16) uint32_t aw[QCH / 32 * ASB];
  __shared__ uint32_t wm[NT / 64][G];  // per wave and head: the max weight (float bits); LOC: the max score
  __shared__ uint32_t wg[NT / 64];     // LOC: per wave the largest residual norm (float bits)
  const int cg = blockIdx.x, g = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  const int row = b * a.d.hkv + g, m = a.m, hq = a.d.hq, nw = m / 32;
  const int comp = seq_comp(a.d, b);
  const int base0 = cg * QV * QCH, ntok = min(QV * QCH, comp - base0);
  if (ntok <= 0) return;  // past the sequence: qjl_final_kernel reads no partial of it
  const tq_store& vs = a.d.vstore;
  const int lane = tid & 63, w = tid >> 6, r = lane & 15, q4 = lane >> 4;
  const int t = tid;
  // ---- every chunk's sign row, gamma and scores of token t; the heads' max and sum
  uint32_t sw[QV][4 * NW4];
  float gv[QV], sc[QV][G], Mh[G], Lh[G];
  {
    if constexpr (!LOC) {
      const float* mlp = a.ml + ((int64_t)b * hq + g * G) * 2;
#pragma unroll
      for (int h = 0; h < G; ++h) {
        Mh[h] = mlp[2 * h];
        Lh[h] = mlp[2 * h + 1];
      }
    }
    const uint8_t* srow = vs.signs + (int64_t)row * vs.sign_head_stride + (int64_t)base0 * (m / 8);
    const float* grow = vs.gamma + (int64_t)row * vs.gamma_head_stride + base0;
    const float* sp = a.scores + (int64_t)row * G * a.qb_hs + base0;
#pragma unroll
    for (int c = 0; c < QV; ++c) {
      const int tc = min(c * QCH + t, ntok - 1);  // tokens past the sequence re-read its last one (weight 0)
      load_sign_row<NW4>(srow + tc * (m / 8), nw, a.vsign16 != 0, sw[c]);
      gv[c] = grow[tc];
#pragma unroll
      for (int h = 0; h < G; ++h) sc[c][h] = sp[h * a.qb_hs + tc];
    }
  }
  // ---- unnormalised weights and their per-wave max per head over the chunks
  float wt[QV][G];
  int eh[G];
  if constexpr (LOC) {
    // the workgroup's max score per head and largest residual norm
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float mx = -INFINITY;
#pragma unroll
      for (int c = 0; c < QV; ++c) mx = c * QCH + t < ntok ? fmaxf(mx, sc[c][h]) : mx;
      const float wmx = wave_max_dpp(mx);
      if (lane == 0) wm[w][h] = __float_as_uint(wmx);
    }
    float gx = 0.f;
#pragma unroll
    for (int c = 0; c < QV; ++c) gx = c * QCH + t < ntok ? fmaxf(gx, gv[c]) : gx;
    const uint32_t gmx = wave_max_nonneg(gx);
    if (lane == 0) wg[w] = gmx;
    __syncthreads();
    uint32_t gb = wg[0];
#pragma unroll
    for (int ww = 1; ww < NT / 64; ++ww) gb = max(gb, wg[ww]);
    const int eg = gb == 0u ? 0 : max((int)((gb >> 23) & 0xFFu), 1) - 127;
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float mh = __uint_as_float(wm[0][h]);
#pragma unroll
      for (int ww = 1; ww < NT / 64; ++ww) mh = fmaxf(mh, __uint_as_float(wm[ww][h]));
      Mh[h] = mh;
      Lh[h] = 1.f;
      eh[h] = eg;
#pragma unroll
      for (int c = 0; c < QV; ++c)
        wt[c][h] = c * QCH + t < ntok ? __builtin_amdgcn_exp2f(sc[c][h] - mh) * gv[c] : 0.f;
    }
    if (tid < G) {
      float mo = Mh[0];
#pragma unroll
      for (int h = 1; h < G; ++h) mo = tid == h ? Mh[h] : mo;
      a.umax[((int64_t)b * hq + g * G + tid) * a.nvc + cg] = mo;
    }
  } else {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float mx = 0.f;
#pragma unroll
      for (int c = 0; c < QV; ++c) {
        const float p = c * QCH + t < ntok && Lh[h] > 0.f ? __builtin_amdgcn_exp2f(sc[c][h] - Mh[h]) : 0.f;
        wt[c][h] = p * gv[c];
        mx = fmaxf(mx, wt[c][h]);
      }
      const uint32_t wmx = wave_max_nonneg(mx);
      if (lane == 0) wm[w][h] = wmx;
    }
    __syncthreads();
    // E_h: the exponent of the workgroup's max weight (weights are >= 0)
#pragma unroll
    for (int h = 0; h < G; ++h) {
      uint32_t mb = wm[0][h];
#pragma unroll
      for (int ww = 1; ww < NT / 64; ++ww) mb = max(mb, wm[ww][h]);
      eh[h] = mb == 0u ? 0 : max((int)((mb >> 23) & 0xFFu), 1) - 127;
    }
  }
  const bool odd = (t & 1) != 0;
  const uint32_t shl = 15u - (uint32_t)r;
  // the sign-bit mask and the halves 1.0 in registers, so that each operand
  // word is one shift and one bit-field insert
  uint32_t bmask = 0x80008000u, bone = 0x3C003C00u;
  asm volatile("" : "+v"(bmask), "+s"(bone));
  constexpr int QT = MAXM / 16 / (NT / 64);
  qf4 acc[QT];
#pragma unroll
  for (int k = 0; k < QT; ++k) acc[k] = qf4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < QV; ++c) {
    const int nvalid = ntok - c * QCH;  // uniform
    if (nvalid <= 0) break;
    if (c > 0) __syncthreads();  // the previous chunk's operand reads are done
    // ---- sign pairs: token 2p's word and token 2p + 1's word of projections
    // 32k .. 32k + 31 give ysm[2k][p] (low halves, by the even thread) and
    // ysm[2k + 1][p] (high halves, by the odd thread)
#pragma unroll
    for (int k = 0; k < 4 * NW4; ++k) {
      if (k >= nw) break;
      const uint32_t nb = lane_xor1(sw[c][k]);
      ysm[2 * k + (odd ? 1 : 0)][t >> 1] =
          odd ? __builtin_amdgcn_perm(sw[c][k], nb, 0x07060302u) : __builtin_amdgcn_perm(nb, sw[c][k], 0x05040100u);
    }
    // ---- A operands: thread t of block bk = t >> 5, q4 group (t >> 3) & 3,
    // token pair (t >> 1) & 3; the even thread writes the high-part pair of
    // row h, the odd one the remainder pair of row h + 8; rows of absent heads zero
    {
      const int bk = t >> 5, qq = (t >> 3) & 3, j = (t >> 1) & 3;
#pragma unroll
      for (int h = 0; h < 8; ++h) {
        uint32_t val = 0u;
        if (h < G) {
          const float x = wt[c][h] * __builtin_amdgcn_ldexpf(1.f, 14 - eh[h]);
          const _Float16 hi = (_Float16)x, lo = (_Float16)(x - (float)hi);
          const uint32_t own =
              (uint32_t)__builtin_bit_cast(uint16_t, hi) | ((uint32_t)__builtin_bit_cast(uint16_t, lo) << 16);
          const uint32_t nb = lane_xor1(own);
          val = odd ? __builtin_amdgcn_perm(own, nb, 0x07060302u) : __builtin_amdgcn_perm(nb, own, 0x05040100u);
        }
        aw[bk * ASB + qq * ASQ + 4 * (h + (odd ? 8 : 0)) + j] = val;
      }
    }
    __syncthreads();
    // ---- the MFMAs of the wave's projection tiles over the chunk's blocks
    const int nblk = (min(nvalid, QCH) + 31) >> 5;
    qu4 av[QCH / 32];
#pragma unroll
    for (int bk = 0; bk < QCH / 32; ++bk) av[bk] = *reinterpret_cast<const qu4*>(&aw[bk * ASB + q4 * ASQ + 4 * r]);
#pragma unroll
    for (int k = 0; k < QT; ++k) {
      const int ct = w + (NT / 64) * k;
      if (ct >= m / 16) break;
#pragma unroll
      for (int bk = 0; bk < QCH / 32; ++bk) {
        if (bk >= nblk) break;
        const qu4 y = *reinterpret_cast<const qu4*>(&ysm[ct][16 * bk + 4 * q4]);
        qu4 bv;
#pragma unroll
        for (int e = 0; e < 4; ++e) bv[e] = ((y[e] << shl) & bmask) | (bone & ~bmask);
        acc[k] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(qh8, av[bk]), __builtin_bit_cast(qh8, bv),
                                                        acc[k], 0, 0, 0);
      }
    }
  }
  // lane (column r, q4) ends with rows 4 q4 + i: head 4 q4 + i for q4 < 2;
  // its scale -2^(E_h - 14) / L_h (the B operands hold -z)
  float hsc[G];
#pragma unroll
  for (int h = 0; h < G; ++h)
    hsc[h] = LOC ? -__builtin_amdgcn_ldexpf(1.f, eh[h] - 14)
                 : Lh[h] > 0.f ? -__builtin_amdgcn_ldexpf(1.f, eh[h] - 14) / Lh[h] : 0.f;
  float osc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) osc[i] = q4 == 0 ? hsc[min(i, G - 1)] : hsc[min(4 + i, G - 1)];
  float* uo = a.upart + (((int64_t)b * hq + g * G + 4 * q4) * a.nvc + cg) * m + r;  // row 4 q4 of the lane
  const int64_t ust = (int64_t)a.nvc * m;                                            // next head
#pragma unroll
  for (int k = 0; k < QT; ++k) {
    const int ct = w + (NT / 64) * k;
    if (ct >= m / 16) break;
    // rows 4 q4 + i: add the remainder rows (lane ^ 32 holds rows + 8)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const auto sw2 =
          __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[k][i]), __float_as_uint(acc[k][i]), false, false);
      const float v = __uint_as_float(sw2[0]) + __uint_as_float(sw2[1]);
      const int hh = 4 * q4 + i;
      if (q4 < 2 && hh < G) uo[i * ust + 16 * ct] = v * osc[i];
    }
  }
}

// Thread t: projection i = t & 127 (and i + 128) over the value partials of
// parity t >> 7 (the chunks holding compressed tokens of the sequence), then
// output dim j = t & 127 over projection rows of parity t >> 7; eight
// independent sums each, so the loads go out eight at a time.
__global__ __launch_bounds__(256) void qjl_final_kernel(QjlArgs a) {
  __shared__ float us[2][256];
  __shared__ float os[2][128];
  const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, m = a.m;
  const int lo = tid & 127, par = tid >> 7;
  const float* up = a.upart + ((int64_t)b * a.d.hq + h) * a.nvc * m;
  const int nvb = min(a.nvc, ((seq_comp(a.d, b) + QCH - 1) / QCH + a.qvc - 1) / a.qvc);  // partials written
  for (int i = lo; i < m; i += 128) {
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int c = par;
    for (; c + 14 < nvb; c += 16) {
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] += up[(int64_t)(c + 2 * k) * m + i];
    }
    for (; c < nvb; c += 2) v[0] += up[(int64_t)c * m + i];
    us[par][i] = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
  }
  __syncthreads();
  for (int i = tid; i < m; i += 256) us[0][i] += us[1][i];
  __syncthreads();
  const int j = lo;
  float z[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  int i = 8 * par;  // rows i .. i + 7 of every 16
  for (; i + 7 < m; i += 16) {
#pragma unroll
    for (int k = 0; k < 8; ++k) z[k] = fmaf(us[0][i + k], a.proj[(int64_t)(i + k) * 128 + j], z[k]);
  }
  os[par][j] = ((z[0] + z[1]) + (z[2] + z[3])) + ((z[4] + z[5]) + (z[6] + z[7]));
  __syncthreads();
  if (tid < 128) a.d.out[((int64_t)b * a.d.hq + h) * 128 + j] += SQRT_HALF_PI / 128.f * (os[0][j] + os[1][j]);
}

// Workspace of the QJL fast route: [fast partials | sq | bias | scores | ml | upart], 256-byte pieces.
struct QjlLayout {
  size_t part, pro, bias, scores, ml, upart, umax, total;
  int64_t qb_hs;
  int nvc;
};

static size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

static int device_cus() {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0;
    hipDeviceProp_t p;
    if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&p, dev) == hipSuccess)
      cus = p.multiProcessorCount;
    if (cus <= 0) cus = 256;
  }
  return cus;
}

// Plan of the K4/V2 path for a call (tq_decode_fast.h): workgroups, chunks
// per workgroup and partial slots.
struct FastPlan {
  int nwg, chunks, vmax;
};

static FastPlan fast_plan(const tq_attn_desc* d) {
  FastPlan p;
  const bool uniform = !d->comp_len && !d->sink_len && !d->res_len;
  fast_plan_host(d->batch, d->hkv, d->max_comp, d->max_sink, d->max_res, uniform, device_cus(), p.nwg, p.chunks,
                 p.vmax);
  return p;
}

// Workgroups per (sequence, kv head) of the uniform-batch kernels, their
// compressed blocks and fp16 tokens per workgroup: about one workgroup per
// CU in total, at most UNI_BLOCKS_PER_WAVE compressed blocks per wave and
// UNI_FP16_PER_WG fp16 tokens per workgroup. False when the call is not
// uniform (per-sequence lengths given) or needs more than UNI_MAX_WG
// workgroups: the persistent kernel takes it.
static bool uniform_geometry(const tq_attn_desc* d, int& nwg, int& bpw, int& fpw, bool ragged_ok = false) {
  nwg = bpw = fpw = 0;
  if (!ragged_ok && (d->comp_len || d->sink_len || d->res_len)) return false;
  const int nbc = (d->max_comp + 31) / 32;
  const int n16 = d->max_sink + d->max_res;
  const int groups = d->batch * d->hkv > 0 ? d->batch * d->hkv : 1;
  const int target = (device_cus() + groups - 1) / groups;
  const int per_wg = FAST_WAVES * UNI_BLOCKS_PER_WAVE;
  int lo = (nbc + per_wg - 1) / per_wg;
  const int lo16 = (n16 + UNI_FP16_PER_WG - 1) / UNI_FP16_PER_WG;
  if (lo16 > lo) lo = lo16;
  if (lo < 1) lo = 1;
  int hi = (nbc + FAST_WAVES - 1) / FAST_WAVES;  // at least one block per wave
  if (hi < lo) hi = lo;
  nwg = target < lo ? lo : (target > hi ? hi : target);
  bpw = (nbc + nwg - 1) / nwg;
  fpw = (n16 + nwg - 1) / nwg;
  return nwg <= UNI_MAX_WG;
}

// The uniform-batch kernels take a uniform call (their merge applies the
// value codec's float32 rotation).
static bool uniform_route(const tq_codec* vc, const tq_attn_desc* d, int& nwg, int& bpw, int& fpw,
                          bool ragged_ok = false) {
  return vc->rotation != nullptr && uniform_geometry(d, nwg, bpw, fpw, ragged_ok);
}

// Partials workspace of the K4/V2 routes of a call: the larger of the uniform
// kernels' (nwg per (b, g), original space) and the persistent kernel's slots
// (the route also depends on the value codec, which the sizing does not see).
static size_t fast_part_bytes(const tq_attn_desc* d) {
  const int G = d->hkv > 0 ? d->hq / d->hkv : 1;
  int nwg, bpw, fpw;
  // the partial slots, then the ragged plan's per-sequence table
  size_t b = al256((size_t)fast_plan(d).vmax * G * PACKED_PART_FLOATS * 4) + (size_t)d->batch * 8;
  // (a grid over the maximal lengths: the other widths' kernels take ragged calls too)
  if (uniform_geometry(d, nwg, bpw, fpw, true)) {
    const size_t u = (size_t)d->batch * d->hkv * nwg * G * PACKED_PART_FLOATS * 4;
    if (u > b) b = u;
  }
  return b;
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// The K4/V2 partials kernel reads keys / values / norms / queries in 16-byte
// pieces: every base and head stride must keep them 16-byte aligned. The value
// codec needs its exact fp16 table (value_table_err).
static bool fast_eligible(const tq_codec* kc, const tq_codec* vc, const tq_attn_desc* d, bool qjl_ok = false) {
  const int G = d->hq / d->hkv;
  if (d->n_q > 1) return false;  // one query token per sequence
  if (!(kc->rotation_parts != nullptr && kc->decode_table != nullptr && vc->decode_table != nullptr &&
        kc->n_host_centroids == 16 && vc->n_host_centroids == 4 && vc->d == 128 && kc->d == 128 &&
        kc->bits_hi == 4 && kc->split == 128 &&
        vc->bits_hi == 2 && vc->split == 128 && vc->value_table_err <= 2e-7f && (!d->qjl || qjl_ok) &&
        (d->kv_dtype == TQ_F16 || d->kv_dtype == TQ_BF16) && (G == 1 || G == 2 || G == 4 || G == 8)))
    return false;
  // bf16 sink / ring tokens: the uniform-batch kernels only (the persistent
  // kernel of ragged batches reads fp16)
  int nwg, bpw, fpw;
  if (d->kv_dtype == TQ_BF16 && !uniform_route(vc, d, nwg, bpw, fpw)) return false;
  if (d->qjl && d->max_comp > 0 &&
      !((reinterpret_cast<uintptr_t>(d->kstore.signs) & 3) == 0 && d->kstore.sign_head_stride % 4 == 0 &&
        (reinterpret_cast<uintptr_t>(d->vstore.signs) & 3) == 0 && d->vstore.sign_head_stride % 4 == 0 &&
        (reinterpret_cast<uintptr_t>(d->kstore.gamma) & 3) == 0))
    return false;
  if (!aligned16(d->q)) return false;
  if (d->max_comp > 0 &&
      !(aligned16(d->kstore.codes_hi) && d->kstore.hi_head_stride % 16 == 0 && aligned16(d->kstore.norms) &&
        d->kstore.norm_head_stride % 4 == 0 && (reinterpret_cast<uintptr_t>(d->vstore.codes_hi) & 1) == 0 &&
        d->vstore.hi_head_stride % 2 == 0 && aligned16(d->vstore.norms) && d->vstore.norm_head_stride % 4 == 0))
    return false;
  if (d->max_sink > 0 && !(aligned16(d->sink_k) && aligned16(d->sink_v) && d->sink_head_stride % 8 == 0)) return false;
  if (d->max_res > 0 && !(aligned16(d->res_k) && aligned16(d->res_v) && d->res_head_stride % 8 == 0)) return false;
  return true;
}

static QjlLayout qjl_layout(const tq_codec* kc, const tq_attn_desc* d) {
  QjlLayout L{};
  const int G = d->hkv > 0 ? d->hq / d->hkv : 1;
  const size_t heads = (size_t)d->batch * d->hq;
  const int m = kc->qjl_m;
  L.qb_hs = ((int64_t)d->max_comp + 31) / 32 * 32;
  if (L.qb_hs < 32) L.qb_hs = 32;
  const int qv = qjl_value_chunks_host(kc->qjl_m);
  L.nvc = ((d->max_comp + QCH - 1) / QCH + qv - 1) / qv;  // value-kernel workgroups per (b, g)
  if (L.nvc < 1) L.nvc = 1;
  size_t off = 0;
  L.part = off; off += al256(fast_part_bytes(d));
  L.pro = off; off += al256(heads * (size_t)m * 4);  // S q
  L.bias = off; off += al256((size_t)d->batch * d->hkv * G * (size_t)L.qb_hs * 4);
  L.scores = off; off += al256((size_t)d->batch * d->hkv * G * (size_t)L.qb_hs * 4);
  L.ml = off; off += al256(heads * 2 * 4);
  L.upart = off; off += al256(heads * (size_t)L.nvc * m * 4);
  L.umax = off; off += al256(heads * (size_t)L.nvc * 4);
  L.total = off;
  return L;
}

// Arguments of the K4/V2 partials + merge kernels for one call.
static void fill_fast(FastArgs& f, const tq_codec* kc, const tq_codec* vc, const tq_attn_desc* d, float* part) {
  f = FastArgs{};
  f.kc = d->kstore.codes_hi; f.k_hs = d->kstore.hi_head_stride;
  f.kn = d->kstore.norms; f.kn_hs = d->kstore.norm_head_stride;
  f.vc = d->vstore.codes_hi; f.v_hs = d->vstore.hi_head_stride;
  f.vn = d->vstore.norms; f.vn_hs = d->vstore.norm_head_stride;
  f.sink_k = static_cast<const uint16_t*>(d->sink_k); f.sink_v = static_cast<const uint16_t*>(d->sink_v);
  f.sink_hs = d->sink_head_stride;
  f.res_k = static_cast<const uint16_t*>(d->res_k); f.res_v = static_cast<const uint16_t*>(d->res_v);
  f.res_hs = d->res_head_stride;
  f.res_cap = d->res_cap; f.res_start0 = d->res_start0;
  f.comp_len_b = d->comp_len; f.sink_len_b = d->sink_len; f.res_len_b = d->res_len; f.res_start_b = d->res_start;
  f.max_comp = d->max_comp; f.max_sink = d->max_sink; f.max_res = d->max_res;
  f.q = d->q; f.q_dtype = d->q_dtype; f.out = d->out;
  f.batch = d->batch; f.hq = d->hq; f.hkv = d->hkv;
  f.qscale = d->scale * 1.4426950408889634f;
  f.rot16 = kc->rotation_parts; f.vrot = vc->rotation;
  f.klut = kc->decode_table; f.vlut = vc->decode_table;
  f.vscale = vc->value_scale;
  f.part = part;
  const FastPlan p = fast_plan(d);
  f.nwg = p.nwg; f.chunks = p.chunks; f.vmax = p.vmax;
  f.plan_tab = reinterpret_cast<int32_t*>(reinterpret_cast<uint8_t*>(part) +
                                          al256((size_t)p.vmax * (d->hq / d->hkv) * PACKED_PART_FLOATS * 4));
  f.uni = !d->comp_len && !d->sink_len && !d->res_len;
  if (f.uni) fast_uniform_plan(d->batch, d->hkv, d->max_comp, d->max_sink, d->max_res, f.nwg, f.chunks, f.plan_T,
                               f.plan_nu, f.plan_V);
}

// The K4/V2 partials (+ merge when merge != 0) of a call into `part`: the
// uniform-batch kernels when the call is uniform and fits their grid, else
// the persistent kernel. qb: the QJL key term is added (qjl_bias) and the
// scores stored; ml receives the merge's global max and sum when not NULL.
// fp16 high part | remainder << 16 of each host centroid (the first n)
static void centroid_pairs(const tq_codec* c, int n, uint32_t* out) {
  for (int i = 0; i < 16; ++i) {
    const float x = i < n ? c->host_centroids[i] : 0.f;
    const _Float16 xh = (_Float16)x;
    out[i] = (uint32_t)__builtin_bit_cast(uint16_t, xh) |
             ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(x - (float)xh)) << 16);
  }
}

// Arguments of the uniform-batch kernels (false when the call is ragged and
// ragged_ok is not set, or too long for their grid; a ragged call gets the
// grid of its maximal lengths and the per-sequence arrays, which only the
// other widths' kernels read): key centroids as fp16 pairs;
// 2-bit values through the codec's exact fp16 table and scale, 3- / 4-bit
// values as fp16 pairs of the centroids (scale 1).
static bool fill_uniform(UniformArgs& u, const tq_codec* kc, const tq_codec* vc, const tq_attn_desc* d, float* part,
                         bool ragged_ok = false) {
  u = UniformArgs{};
  if (!uniform_route(vc, d, u.nwg, u.bpw, u.fpw, ragged_ok)) return false;
  u.comp_len_b = d->comp_len; u.sink_len_b = d->sink_len; u.res_len_b = d->res_len;
  u.kc = d->kstore.codes_hi; u.k_hs = d->kstore.hi_head_stride;
  u.kn = d->kstore.norms; u.kn_hs = d->kstore.norm_head_stride;
  u.vc = d->vstore.codes_hi; u.v_hs = d->vstore.hi_head_stride;
  u.vn = d->vstore.norms; u.vn_hs = d->vstore.norm_head_stride;
  u.sink_k = d->sink_k; u.sink_v = d->sink_v; u.sink_hs = d->sink_head_stride;
  u.res_k = d->res_k; u.res_v = d->res_v; u.res_hs = d->res_head_stride;
  u.res_cap = d->res_cap; u.res_start0 = d->res_start0;
  u.res_start_b = d->res_start;  // the lengths are the maximal ones
  u.max_comp = d->max_comp; u.max_sink = d->max_sink; u.max_res = d->max_res;
  u.q = d->q; u.q_dtype = d->q_dtype; u.out = d->out;
  u.batch = d->batch; u.hq = d->hq; u.hkv = d->hkv;
  u.qscale = d->scale * 1.4426950408889634f;
  u.rot16 = kc->rotation_parts; u.vrot = vc->rotation;
  centroid_pairs(kc, 1 << kc->bits_hi, u.khl);
  if (vc->bits_hi == 2) {
    for (int i = 0; i < 4; ++i) u.vtab[i] = vc->value_table[i];
    u.vscale = vc->value_scale;
  } else {
    centroid_pairs(vc, 1 << vc->bits_hi, u.vhl);
    u.vscale = 1.f;
  }
  u.part = part;
  return true;
}

// (fout: the persistent kernel's arguments, for a merge launched later)
static int launch_k4v2(const tq_codec* kc, const tq_codec* vc, const tq_attn_desc* d, float* part, bool qb,
                       float* qjl_bias, float* scores, int64_t qb_hs, float* ml, int merge, hipStream_t s,
                       FastArgs* fout = nullptr) {
  const int G = d->hq / d->hkv;
  UniformArgs u;
  if (fill_uniform(u, kc, vc, d, part)) {
    u.qjl_bias = qjl_bias; u.scores = scores; u.qb_hs = qb_hs; u.ml = ml;
    return launch_uniform_decode(u, G, qb, merge, s, d->kv_dtype == TQ_BF16);
  }
  FastArgs f;
  fill_fast(f, kc, vc, d, part);
  f.qjl_bias = qjl_bias; f.scores = scores; f.qb_hs = qb_hs; f.ml = ml;
  // the persistent kernel computes the QJL key term itself (S q at the query
  // rotation, then the sketch against it)
  f.ksg = d->kstore.signs; f.ksg_hs = d->kstore.sign_head_stride;
  f.kgam = d->kstore.gamma; f.kgam_hs = d->kstore.gamma_head_stride;
  f.sproj = kc->qjl_proj;
  f.sscale = d->scale;
  f.qm = kc->qjl_m;
  if (fout) *fout = f;
  return launch_fast_decode(f, G, qb ? (kc->qjl_m <= 128 ? 1 : 2) : 0, merge, s);
}

// The uniform-batch kernels take this K4/V2 call (else the persistent kernel).
static bool k4v2_uniform(const tq_codec* kc, const tq_codec* vc, const tq_attn_desc* d) {
  UniformArgs u;
  return fill_uniform(u, kc, vc, d, nullptr);
}

// The uniform-batch MFMA kernels for the other integer widths (key and value
// bits 2..4 with one codebook each, K4/V2 excepted): d = 128, fp16 K/V, one
// query token, no sketch, G in {1, 2, 4, 8}; 2-bit values need the exact
// fp16 table; the rows every load touches aligned as the loads need (key
// codes 16-byte, value codes 4-byte, 2-byte for 2-bit values). Uniform and
// ragged calls (a grid over the maximal lengths; workgroups past a shorter
// sequence write empty partials).
static bool widths_eligible(const tq_codec* kc, const tq_codec* vc, const tq_attn_desc* d) {
  const int G = d->hq / d->hkv, kb = kc->bits_hi, vb = vc->bits_hi;
  if (d->n_q > 1 || d->qjl) return false;
  if (!(kc->d == 128 && vc->d == 128 && kc->split == 128 && vc->split == 128 && kb >= 2 && kb <= 4 && vb >= 2 &&
        vb <= 4 && !(kb == 4 && vb == 2)))
    return false;
  if (!(kc->rotation_parts && vc->rotation && kc->n_host_centroids == (1 << kb) &&
        vc->n_host_centroids == (1 << vb)))
    return false;
  if (vb == 2 && !(vc->value_table_err <= 2e-7f)) return false;
  if (d->kv_dtype != TQ_F16 || !(G == 1 || G == 2 || G == 4 || G == 8)) return false;
  if (!aligned16(d->q)) return false;
  const uintptr_t va = vb == 2 ? 1 : 3;
  if (d->max_comp > 0 &&
      !(aligned16(d->kstore.codes_hi) && d->kstore.hi_head_stride % 16 == 0 && aligned16(d->kstore.norms) &&
        d->kstore.norm_head_stride % 4 == 0 && (reinterpret_cast<uintptr_t>(d->vstore.codes_hi) & va) == 0 &&
        d->vstore.hi_head_stride % (int64_t)(va + 1) == 0 && aligned16(d->vstore.norms) &&
        d->vstore.norm_head_stride % 4 == 0))
    return false;
  if (d->max_sink > 0 && !(aligned16(d->sink_k) && aligned16(d->sink_v) && d->sink_head_stride % 8 == 0)) return false;
  if (d->max_res > 0 && !(aligned16(d->res_k) && aligned16(d->res_v) && d->res_head_stride % 8 == 0)) return false;
  return true;
}

// Width kind of a codec for the split-codebook kernels: bits_hi + bits_lo of a
// fractional codec split at dim 64 (7 = 3.5 bits, 5 = 2.5), the bits of an
// integer one (2 to 4), or 0 when the kernels do not take it.
static int split_kind(const tq_codec* c) {
  if (c->d != 128 || !c->centroids_hi || !c->centroids_lo) return 0;
  if (c->split == 64 && (c->bits_hi == 4 || c->bits_hi == 3) && c->bits_lo == c->bits_hi - 1)
    return c->bits_hi + c->bits_lo;
  if (c->split == 128 && c->bits_hi >= 2 && c->bits_hi <= 4) return c->bits_hi;
  return 0;
}

// The uniform-batch MFMA kernels for fractional widths (tq_decode_split.h):
// head_dim 128, a codec split at dim 64 into ceil(bits) / floor(bits) = 4 / 3
// or 3 / 2 on at least one side (the other fractional or integer 2-4 bits),
// fp16 K/V, one query token, no sketch, G in {1, 2, 4, 8}; key code rows read
// as dword pairs (4-byte aligned), value code rows in 16-byte pieces per
// 32-token block (16-byte aligned bases and head strides).
static bool split_eligible(const tq_codec* kc, const tq_codec* vc, const tq_attn_desc* d) {
  const int G = d->hq / d->hkv;
  if (d->n_q > 1 || d->qjl) return false;
  const int kk = split_kind(kc), vk = split_kind(vc);
  if (!kk || !vk || (kk <= 4 && vk <= 4)) return false;  // both integer: the widths kernels
  if (!(kc->rotation_parts && vc->rotation)) return false;
  if (d->kv_dtype != TQ_F16 || !(G == 1 || G == 2 || G == 4 || G == 8)) return false;
  if (!aligned16(d->q)) return false;
  auto al4 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3) == 0; };
  const bool kf = kk > 4, vf = vk > 4;  // fractional sides have a lo code row
  if (d->max_comp > 0 &&
      !(al4(d->kstore.codes_hi) && d->kstore.hi_head_stride % 4 == 0 &&
        (!kf || (al4(d->kstore.codes_lo) && d->kstore.lo_head_stride % 4 == 0)) && aligned16(d->vstore.codes_hi) &&
        d->vstore.hi_head_stride % 16 == 0 &&
        (!vf || (aligned16(d->vstore.codes_lo) && d->vstore.lo_head_stride % 16 == 0)) && al4(d->kstore.norms) &&
        al4(d->vstore.norms)))
    return false;
  if (d->max_sink > 0 && !(aligned16(d->sink_k) && aligned16(d->sink_v) && d->sink_head_stride % 8 == 0)) return false;
  if (d->max_res > 0 && !(aligned16(d->res_k) && aligned16(d->res_v) && d->res_head_stride % 8 == 0)) return false;
  return true;
}

// Arguments of the fractional-width kernels: the uniform-batch arguments plus
// the low-width code rows and the four device codebooks (false when the call
// is ragged or too long for the uniform grid).
static bool fill_split(UniformArgs& u, const tq_codec* kc, const tq_codec* vc, const tq_attn_desc* d, float* part) {
  if (!fill_uniform(u, kc, vc, d, part)) return false;
  u.kcl = d->kstore.codes_lo; u.kl_hs = d->kstore.lo_head_stride;
  u.vcl = d->vstore.codes_lo; u.vl_hs = d->vstore.lo_head_stride;
  u.kcen_hi = kc->centroids_hi; u.kcen_lo = kc->centroids_lo;
  u.vcen_hi = vc->centroids_hi; u.vcen_lo = vc->centroids_lo;
  u.vscale = 1.f;
  return true;
}

// The QJL route: S q, key-term bias, K4/V2 partials with the bias
// (scores stored) + merge (max and sum exported), value term, final S^T add.
static int qjl_fast_run(const tq_codec* kc, const tq_codec* vc, const tq_attn_desc* d, void* workspace,
                        size_t workspace_bytes, hipStream_t s) {
  const QjlLayout QL = qjl_layout(kc, d);
  if (!workspace || workspace_bytes < QL.total)
    return set_error(TQ_ERR_WORKSPACE, "workspace %zu bytes < %zu", workspace_bytes, QL.total);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  const int G = d->hq / d->hkv;
  QjlArgs qa;
  qa.d = *d;
  qa.sq = reinterpret_cast<float*>(ws + QL.pro);
  qa.proj = kc->qjl_proj;
  qa.m = kc->qjl_m;
  // 16-byte loads of the sign rows: rows of a multiple of 16 bytes at 16-byte alignment
  auto sign16 = [&](const tq_store& st) {
    return kc->qjl_m % 128 == 0 && aligned16(st.signs) && st.sign_head_stride % 16 == 0 ? 1 : 0;
  };
  qa.ksign16 = sign16(d->kstore);
  qa.vsign16 = sign16(d->vstore);
  const bool w8 = kc->qjl_m > 128;  // more than 4 sign words per token
  qa.bias = reinterpret_cast<float*>(ws + QL.bias);
  qa.scores = reinterpret_cast<float*>(ws + QL.scores);
  qa.ml = reinterpret_cast<float*>(ws + QL.ml);
  qa.upart = reinterpret_cast<float*>(ws + QL.upart);
  qa.umax = reinterpret_cast<float*>(ws + QL.umax);
  qa.qb_hs = QL.qb_hs;
  qa.nvc = QL.nvc;
  qa.qvc = qjl_value_chunks_host(kc->qjl_m);
  // the key term: S q and a bias kernel for the uniform-batch kernels; the
  // persistent kernel computes both from S and the sketch itself
  const bool uniform = k4v2_uniform(kc, vc, d);
  if (uniform) {
    const dim3 sgrid((unsigned)((kc->qjl_m + 63) / 64), d->hkv, d->batch);
    switch (G) {
      case 1: hipLaunchKernelGGL((qjl_sq_kernel<1>), sgrid, dim3(256), 0, s, qa); break;
      case 2: hipLaunchKernelGGL((qjl_sq_kernel<2>), sgrid, dim3(256), 0, s, qa); break;
      case 4: hipLaunchKernelGGL((qjl_sq_kernel<4>), sgrid, dim3(256), 0, s, qa); break;
      default: hipLaunchKernelGGL((qjl_sq_kernel<8>), sgrid, dim3(256), 0, s, qa); break;
    }
    TQ_LAUNCH_CHECK("tq_decode_attention qjl S q");
  }
  const dim3 bgrid((unsigned)((QL.qb_hs + QBC * QCH - 1) / (QBC * QCH)), d->hkv, d->batch);
  if (uniform) switch (G * 2 + (w8 ? 1 : 0)) {
    case 2: hipLaunchKernelGGL((qjl_bias_kernel<1, 1>), bgrid, dim3(NT), 0, s, qa); break;
    case 3: hipLaunchKernelGGL((qjl_bias_kernel<1, 2>), bgrid, dim3(NT), 0, s, qa); break;
    case 4: hipLaunchKernelGGL((qjl_bias_kernel<2, 1>), bgrid, dim3(NT), 0, s, qa); break;
    case 5: hipLaunchKernelGGL((qjl_bias_kernel<2, 2>), bgrid, dim3(NT), 0, s, qa); break;
    case 8: hipLaunchKernelGGL((qjl_bias_kernel<4, 1>), bgrid, dim3(NT), 0, s, qa); break;
    case 9: hipLaunchKernelGGL((qjl_bias_kernel<4, 2>), bgrid, dim3(NT), 0, s, qa); break;
    case 16: hipLaunchKernelGGL((qjl_bias_kernel<8, 1>), bgrid, dim3(NT), 0, s, qa); break;
    default: hipLaunchKernelGGL((qjl_bias_kernel<8, 2>), bgrid, dim3(NT), 0, s, qa); break;
  }
  TQ_LAUNCH_CHECK("tq_decode_attention qjl bias");
  const dim3 vgrid((unsigned)QL.nvc, d->hkv, d->batch);
  if (!uniform) {
    // persistent kernel: partials (key term inside), the value kernel with
    // each workgroup's own max, then the merge adding the value term
    FastArgs f;
    if (launch_k4v2(kc, vc, d, reinterpret_cast<float*>(ws + QL.part), true, nullptr, const_cast<float*>(qa.scores),
                    QL.qb_hs, nullptr, 0, s, &f) != 0)
      TQ_LAUNCH_CHECK("tq_decode_attention qjl fast");
    switch (G * 2 + (w8 ? 1 : 0)) {
      case 2: hipLaunchKernelGGL((qjl_value_kernel<1, 1, true>), vgrid, dim3(NT), 0, s, qa); break;
      case 3: hipLaunchKernelGGL((qjl_value_kernel<1, 2, true>), vgrid, dim3(NT), 0, s, qa); break;
      case 4: hipLaunchKernelGGL((qjl_value_kernel<2, 1, true>), vgrid, dim3(NT), 0, s, qa); break;
      case 5: hipLaunchKernelGGL((qjl_value_kernel<2, 2, true>), vgrid, dim3(NT), 0, s, qa); break;
      case 8: hipLaunchKernelGGL((qjl_value_kernel<4, 1, true>), vgrid, dim3(NT), 0, s, qa); break;
      case 9: hipLaunchKernelGGL((qjl_value_kernel<4, 2, true>), vgrid, dim3(NT), 0, s, qa); break;
      case 16: hipLaunchKernelGGL((qjl_value_kernel<8, 1, true>), vgrid, dim3(NT), 0, s, qa); break;
      default: hipLaunchKernelGGL((qjl_value_kernel<8, 2, true>), vgrid, dim3(NT), 0, s, qa); break;
    }
    TQ_LAUNCH_CHECK("tq_decode_attention qjl value");
    f.qjl_up = qa.upart;
    f.qjl_umax = qa.umax;
    f.qnvc = QL.nvc;
    f.qtok = QCH * qa.qvc;
    if (launch_fast_merge_qjl(f, G, w8 ? 2 : 1, s) != 0) TQ_LAUNCH_CHECK("tq_decode_attention qjl merge");
    return TQ_OK;
  }
  if (launch_k4v2(kc, vc, d, reinterpret_cast<float*>(ws + QL.part), true, qa.bias, const_cast<float*>(qa.scores),
                  QL.qb_hs, const_cast<float*>(qa.ml), 1, s) != 0)
    TQ_LAUNCH_CHECK("tq_decode_attention qjl fast");
  switch (G * 2 + (w8 ? 1 : 0)) {
    case 2: hipLaunchKernelGGL((qjl_value_kernel<1, 1>), vgrid, dim3(NT), 0, s, qa); break;
    case 3: hipLaunchKernelGGL((qjl_value_kernel<1, 2>), vgrid, dim3(NT), 0, s, qa); break;
    case 4: hipLaunchKernelGGL((qjl_value_kernel<2, 1>), vgrid, dim3(NT), 0, s, qa); break;
    case 5: hipLaunchKernelGGL((qjl_value_kernel<2, 2>), vgrid, dim3(NT), 0, s, qa); break;
    case 8: hipLaunchKernelGGL((qjl_value_kernel<4, 1>), vgrid, dim3(NT), 0, s, qa); break;
    case 9: hipLaunchKernelGGL((qjl_value_kernel<4, 2>), vgrid, dim3(NT), 0, s, qa); break;
    case 16: hipLaunchKernelGGL((qjl_value_kernel<8, 1>), vgrid, dim3(NT), 0, s, qa); break;
    default: hipLaunchKernelGGL((qjl_value_kernel<8, 2>), vgrid, dim3(NT), 0, s, qa); break;
  }
  TQ_LAUNCH_CHECK("tq_decode_attention qjl value");
  hipLaunchKernelGGL(qjl_final_kernel, dim3(d->hq, d->batch), dim3(256), 0, s, qa);
  TQ_LAUNCH_CHECK("tq_decode_attention qjl final");
  return TQ_OK;
}

// Dense (uncompressed fp16 / bf16) calls: head_dim 128, nothing compressed,
// 16-byte aligned rows. record = false only tests (no error message kept).
static int dense_check(const tq_attn_desc* d, int D, bool record = true) {
#define DENSE_FAIL(code, ...) return record ? set_error(code, __VA_ARGS__) : (code)
  if (D != 128) DENSE_FAIL(TQ_ERR_UNSUPPORTED, "dense decode attention: head_dim %d != 128", D);
  if (d->max_comp != 0) DENSE_FAIL(TQ_ERR_INVALID, "dense decode attention with compressed tokens (max_comp %d)", d->max_comp);
  if (d->n_q > 1) DENSE_FAIL(TQ_ERR_UNSUPPORTED, "dense decode attention: one query token (n_q %d)", d->n_q);
  if (d->batch <= 0 || d->hkv <= 0 || d->hq <= 0 || d->hq % d->hkv)
    DENSE_FAIL(TQ_ERR_INVALID, "bad head counts hq=%d hkv=%d batch=%d", d->hq, d->hkv, d->batch);
  const int G = d->hq / d->hkv;
  if (G != 1 && G != 2 && G != 4 && G != 8)
    DENSE_FAIL(TQ_ERR_UNSUPPORTED, "query heads per kv head %d not in {1,2,4,8}", G);
  if (d->batch > 65535 || d->hkv > 65535) DENSE_FAIL(TQ_ERR_UNSUPPORTED, "grid too large");
  if (d->max_sink < 0 || d->max_res < 0) DENSE_FAIL(TQ_ERR_INVALID, "negative segment length");
  if (!d->q || !d->out) DENSE_FAIL(TQ_ERR_INVALID, "q/out is NULL");
  if (!aligned16(d->q)) DENSE_FAIL(TQ_ERR_UNSUPPORTED, "dense decode attention: q must be 16-byte aligned");
  if (d->q_dtype < TQ_F16 || d->q_dtype > TQ_F32) DENSE_FAIL(TQ_ERR_UNSUPPORTED, "unknown q dtype");
  if (d->kv_dtype != TQ_F16 && d->kv_dtype != TQ_BF16)
    DENSE_FAIL(TQ_ERR_UNSUPPORTED, "dense decode attention needs fp16 or bf16 K/V");
  if (d->max_sink > 0 && (!d->sink_k || !d->sink_v)) DENSE_FAIL(TQ_ERR_INVALID, "sink pointers are NULL");
  if (d->max_res > 0 && (!d->res_k || !d->res_v || d->res_cap <= 0 || d->max_res > d->res_cap))
    DENSE_FAIL(TQ_ERR_INVALID, "residual ring pointers / capacity");
  if (d->max_res > 0 && !d->res_start && (d->res_start0 < 0 || d->res_start0 >= d->res_cap))
    DENSE_FAIL(TQ_ERR_INVALID, "ring start %d outside [0, %d)", d->res_start0, d->res_cap);
  if (d->max_sink > 0 && !(aligned16(d->sink_k) && aligned16(d->sink_v) && d->sink_head_stride % 8 == 0))
    DENSE_FAIL(TQ_ERR_UNSUPPORTED, "sink rows must be 16-byte aligned");
  if (d->max_res > 0 && !(aligned16(d->res_k) && aligned16(d->res_v) && d->res_head_stride % 8 == 0))
    DENSE_FAIL(TQ_ERR_UNSUPPORTED, "ring rows must be 16-byte aligned");
  return TQ_OK;
#undef DENSE_FAIL
}

static size_t dense_workspace(const tq_attn_desc* d) {
  int nwg, bpw;
  dense_geometry(d->batch, d->hkv, d->max_sink, d->max_res, device_cus(), nwg, bpw);
  const int G = d->hkv > 0 ? d->hq / d->hkv : 1;
  return nwg > 1 ? (size_t)d->batch * d->hkv * nwg * G * FAST_PART_FLOATS * 4 : 0;
}

static int dense_run(const tq_attn_desc* d, void* workspace, size_t workspace_bytes, hipStream_t s) {
  DenseArgs a;
  a.sink_k = d->sink_k; a.sink_v = d->sink_v; a.sink_hs = d->sink_head_stride;
  a.res_k = d->res_k; a.res_v = d->res_v; a.res_hs = d->res_head_stride;
  a.res_cap = d->res_cap; a.res_start0 = d->res_start0;
  a.sink_len_b = d->sink_len; a.res_len_b = d->res_len; a.res_start_b = d->res_start;
  a.max_sink = d->max_sink; a.max_res = d->max_res;
  a.q = d->q; a.q_dtype = d->q_dtype; a.out = d->out;
  a.hq = d->hq; a.hkv = d->hkv;
  a.qscale = d->scale * 1.4426950408889634f;
  dense_geometry(d->batch, d->hkv, d->max_sink, d->max_res, device_cus(), a.nwg, a.bpw);
  const size_t need = dense_workspace(d);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return set_error(TQ_ERR_WORKSPACE, "workspace %zu bytes < %zu", workspace_bytes, need);
  a.part = static_cast<float*>(workspace);
  if (launch_dense_decode(a, d->hq / d->hkv, d->kv_dtype == TQ_BF16, d->batch, 1, s) != 0)
    TQ_LAUNCH_CHECK("tq_dense_decode_attention");
  return TQ_OK;
}

// Scratch of tq_decode_attention_noalloc: a file-scope device array, one copy
// per GPU the library runs on, held until the process ends. Host code never
// passes `scratch` itself to a kernel (in host code the name is a host-side
// stand-in, not a device address): the address of each device's copy is
// looked up once per device with hipGetSymbolAddress and kept in
// g_scratch_addr.
static __device__ __align__(256) uint8_t scratch[TQ_NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
static void* g_scratch_addr[MAX_DEVICES];
static std::mutex g_scratch_mu;

// The current device's copy of `scratch` (looked up on the first call on
// that device, with that device current).
static int noalloc_scratch(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES)
    return set_error(TQ_ERR_LAUNCH, "no current HIP device (or device id >= %d)", MAX_DEVICES);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_addr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(TQ_ERR_LAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_addr[dev] = p;
  }
  *out = g_scratch_addr[dev];
  return TQ_OK;
}

}  // namespace tq

using namespace tq;

// The checks every decode-attention entry point runs before it sizes or
// touches any workspace: codecs, descriptor, head counts, grid limits,
// segment lengths, pointers, dtypes and the QJL arrays.
static int check_attention_call(const tq_codec* kc, const tq_codec* vc, const tq_attn_desc* d) {
  int rc = check_codec(kc);
  if (rc) return rc;
  if ((rc = check_codec(vc))) return rc;
  if (!d) return set_error(TQ_ERR_INVALID, "attention descriptor is NULL");
  if (kc->d != vc->d) return set_error(TQ_ERR_INVALID, "key/value head_dim differ");
  if (d->batch <= 0 || d->hkv <= 0 || d->hq <= 0 || d->hq % d->hkv)
    return set_error(TQ_ERR_INVALID, "bad head counts hq=%d hkv=%d batch=%d", d->hq, d->hkv, d->batch);
  const int G = d->hq / d->hkv;  // any integer ratio: the general kernel groups the heads by group_heads(G)
  if (d->n_q < 0) return set_error(TQ_ERR_INVALID, "n_q %d < 0", d->n_q);
  if ((int64_t)d->batch * (d->n_q > 1 ? d->n_q : 1) > 65535 || (int64_t)d->hkv * (G / group_heads(G)) > 65535 ||
      d->hq > 65535)
    return set_error(TQ_ERR_UNSUPPORTED, "grid too large");
  if (d->n_q > 1 && d->n_q > d->max_sink + d->max_comp + d->max_res)
    return set_error(TQ_ERR_INVALID, "n_q %d query tokens > the %d cached tokens", d->n_q,
                     d->max_sink + d->max_comp + d->max_res);
  if (d->max_comp < 0 || d->max_sink < 0 || d->max_res < 0)
    return set_error(TQ_ERR_INVALID, "negative segment length");
  if (!d->q || !d->out) return set_error(TQ_ERR_INVALID, "q/out is NULL");
  if (d->q_dtype < TQ_F16 || d->q_dtype > TQ_F32 || d->kv_dtype < TQ_F16 || d->kv_dtype > TQ_F32)
    return set_error(TQ_ERR_UNSUPPORTED, "unknown q/kv dtype");
  if (d->max_comp > 0 && (!d->kstore.codes_hi || !d->kstore.norms || !d->vstore.codes_hi || !d->vstore.norms))
    return set_error(TQ_ERR_INVALID, "compressed store pointers are NULL");
  if (d->max_sink > 0 && (!d->sink_k || !d->sink_v)) return set_error(TQ_ERR_INVALID, "sink pointers are NULL");
  if (d->max_res > 0 && (!d->res_k || !d->res_v || d->res_cap <= 0 || d->max_res > d->res_cap))
    return set_error(TQ_ERR_INVALID, "residual ring pointers / capacity");
  if (d->max_res > 0 && !d->res_start && (d->res_start0 < 0 || d->res_start0 >= d->res_cap))
    return set_error(TQ_ERR_INVALID, "ring start %d outside [0, %d)", d->res_start0, d->res_cap);
  const int row_v = row_bytes(vc->split, vc->bits_hi) + row_bytes(vc->d - vc->split, vc->bits_lo);
  if (row_v > 128) return set_error(TQ_ERR_UNSUPPORTED, "value row of %d bytes > 128", row_v);
  const bool qjl = d->qjl != 0;
  if (qjl) {
    if (!kc->qjl_proj || kc->qjl_m <= 0 || kc->qjl_m != vc->qjl_m || kc->qjl_proj != vc->qjl_proj)
      return set_error(TQ_ERR_INVALID, "QJL attention needs one projection shared by keys and values");
    if (kc->qjl_m > 256) return set_error(TQ_ERR_UNSUPPORTED, "qjl_m > 256");
    if (d->max_comp > 0 && (!d->kstore.signs || !d->kstore.gamma || !d->vstore.signs || !d->vstore.gamma))
      return set_error(TQ_ERR_INVALID, "QJL attention needs stored signs and gamma");
  }
  return TQ_OK;
}

extern "C" {

size_t tq_decode_workspace_bytes(const tq_codec* kcodec, const tq_attn_desc* d) {
  if (!kcodec || !d) return 0;
  int nc, ns, nr;
  chunk_counts(d, nc, ns, nr);
  const int D = kcodec->d;
  const int m = d->qjl ? kcodec->qjl_m : 0;
  const size_t nch = (size_t)(nc + ns + nr);
  const size_t heads = (size_t)d->batch * d->hq * (d->n_q > 1 ? d->n_q : 1);  // query rows
  size_t general = heads * D * 4 * 2 + heads * (size_t)m * 4 + heads * nch * part_stride(D, m) * 4;
  const size_t fast = d->hkv > 0 && d->hq % d->hkv == 0 ? fast_part_bytes(d) : 0;
  size_t bytes = general > fast ? general : fast;
  if (d->qjl && kcodec->d == 128 && kcodec->qjl_m > 0 && kcodec->qjl_m <= 256 && d->max_comp > 0 && d->hkv > 0 &&
      d->hq % d->hkv == 0) {
    const size_t qf = qjl_layout(kcodec, d).total;
    if (qf > bytes) bytes = qf;
  }
  if (d->max_comp == 0 && kcodec->d == 128) {
    const size_t dense = dense_workspace(d);
    if (dense > bytes) bytes = dense;
  }
  if (d->n_q > 1 && kcodec->d == 128) {
    const size_t pre = prefill_workspace(d);
    if (pre > bytes) bytes = pre;
  }
  return (bytes + 255) & ~(size_t)255;
}

size_t tq_attention_workspace_bytes(const tq_codec* kc, const tq_codec* vc, const tq_attn_desc* d) {
  if (!kc || !vc || !d) return 0;
  if (prefill_eligible(kc, vc, d)) return (prefill_workspace(d) + 255) & ~(size_t)255;
  return tq_decode_workspace_bytes(kc, d);
}

int tq_decode_attention(const tq_codec* kc, const tq_codec* vc, const tq_attn_desc* d, void* workspace,
                        size_t workspace_bytes, void* stream) {
  const int rc = check_attention_call(kc, vc, d);
  if (rc) return rc;
  const int G = d->hq / d->hkv;
  const bool qjl = d->qjl != 0;
  const size_t need = tq_attention_workspace_bytes(kc, vc, d);
  if (!workspace || workspace_bytes < need)
    return set_error(TQ_ERR_WORKSPACE, "workspace %zu bytes < %zu", workspace_bytes, need);

  hipStream_t s = static_cast<hipStream_t>(stream);
  // several query tokens per sequence: the query-tiled prefill kernels
  if (prefill_eligible(kc, vc, d)) return prefill_run(kc, vc, d, workspace, s);
  // nothing compressed yet: the dense kernel over the sink and ring
  if (d->max_comp == 0 && !(d->flags & TQ_ATTN_GENERAL) && (d->max_sink > 0 || d->max_res > 0) &&
      dense_check(d, kc->d, false) == TQ_OK)
    return dense_run(d, workspace, workspace_bytes, s);
  if (qjl && d->max_comp > 0 && fast_eligible(kc, vc, d, true) && !(d->flags & TQ_ATTN_GENERAL))
    return qjl_fast_run(kc, vc, d, workspace, workspace_bytes, s);
  if (fast_eligible(kc, vc, d) && !(d->flags & TQ_ATTN_GENERAL)) {
    if (launch_k4v2(kc, vc, d, static_cast<float*>(workspace), false, nullptr, nullptr, 0, nullptr, 1, s) != 0)
      TQ_LAUNCH_CHECK("tq_decode_attention (fast)");
    return TQ_OK;
  }
  if (widths_eligible(kc, vc, d) && !(d->flags & TQ_ATTN_GENERAL)) {
    UniformArgs u;
    if (fill_uniform(u, kc, vc, d, static_cast<float*>(workspace), true)) {
      if (launch_uniform_widths(u, d->hq / d->hkv, kc->bits_hi, vc->bits_hi, 1, s) != 0)
        TQ_LAUNCH_CHECK("tq_decode_attention (widths)");
      return TQ_OK;
    }
  }
  if (split_eligible(kc, vc, d) && !(d->flags & TQ_ATTN_GENERAL)) {
    UniformArgs u;
    if (fill_split(u, kc, vc, d, static_cast<float*>(workspace))) {
      if (launch_uniform_split(u, d->hq / d->hkv, split_kind(kc), split_kind(vc), 1, s) != 0)
        TQ_LAUNCH_CHECK("tq_decode_attention (fractional widths)");
      return TQ_OK;
    }
  }

  AttnArgs a;
  a.d = *d;
  a.D = kc->d;
  a.rot = kc->rotation;
  a.vrot = vc->rotation;
  a.kc_hi = kc->centroids_hi;
  a.kc_lo = kc->split < kc->d ? kc->centroids_lo : kc->centroids_hi;
  a.vc_hi = vc->centroids_hi;
  a.vc_lo = vc->split < vc->d ? vc->centroids_lo : vc->centroids_hi;
  a.proj = qjl ? kc->qjl_proj : nullptr;
  a.m = qjl ? kc->qjl_m : 0;
  a.kb_hi = kc->bits_hi;
  a.kb_lo = kc->split < kc->d ? kc->bits_lo : kc->bits_hi;
  a.ks = kc->split;
  a.vb_hi = vc->bits_hi;
  a.vb_lo = vc->split < vc->d ? vc->bits_lo : vc->bits_hi;
  a.vs = vc->split;
  a.k_row_hi = row_bytes(kc->split, kc->bits_hi);
  a.k_row_lo = row_bytes(kc->d - kc->split, a.kb_lo);
  a.v_row_hi = row_bytes(vc->split, vc->bits_hi);
  a.v_row_lo = row_bytes(vc->d - vc->split, a.vb_lo);
  a.row_sign = a.m / 8;
  chunk_counts(d, a.nc, a.ns, a.nr);
  a.nch = a.nc + a.ns + a.nr;
  a.ps = part_stride(a.D, a.m);
  a.c0 = 0;
  const int gh = group_heads(G);
  a.gsub = G / gh;
  const size_t heads = (size_t)d->batch * d->hq * (d->n_q > 1 ? d->n_q : 1);  // query rows
  float* ws = static_cast<float*>(workspace);
  a.qr = ws;
  a.qs = a.qr + heads * a.D;
  a.sq = a.qs + heads * a.D;
  a.part = a.sq + heads * a.m;

  const size_t pro_smem = (size_t)a.D * 4;
  const int nq = d->n_q > 1 ? d->n_q : 1;
  hipLaunchKernelGGL(prologue_kernel, dim3(d->hq, d->batch * nq), dim3(128), pro_smem, s, a);
  TQ_LAUNCH_CHECK("tq_decode_attention prologue");
  if (a.nch > 0) {
    dim3 grid(a.nch, d->hkv * a.gsub, d->batch * nq);
    // the query arrays of the kernel at the next instantiated width
    if (a.D <= 64) launch_chunks<64>(a, gh, grid, s);
    else if (a.D <= 96) launch_chunks<96>(a, gh, grid, s);
    else if (a.D <= 128) launch_chunks<128>(a, gh, grid, s);
    else launch_chunks<256>(a, gh, grid, s);
    TQ_LAUNCH_CHECK("tq_decode_attention chunks");
  }
  const size_t cmb_smem = (size_t)(((a.nch + 3) & ~3) + a.D + a.m) * 4;
  hipLaunchKernelGGL(combine_kernel, dim3(d->hq, d->batch * nq), dim3(128), cmb_smem, s, a);
  TQ_LAUNCH_CHECK("tq_decode_attention combine");
  return TQ_OK;
}

// Measurement hook of bench.py, not part of the ABI (include/tq_abi.h does not
// declare it): the partials kernel of the K4/V2 route alone (no merge, `out`
// not written), so its launches can be timed with events on their stream.
int tq_measure_decode_partials(const tq_codec* kc, const tq_codec* vc, const tq_attn_desc* d, void* workspace,
                               size_t workspace_bytes, void* stream) {
  if (!kc || !vc || !d || d->hkv <= 0 || d->hq % d->hkv || d->qjl)
    return set_error(TQ_ERR_UNSUPPORTED, "measurement: not a packed uniform or K4/V2 call");
  if (!workspace || workspace_bytes < fast_part_bytes(d)) return set_error(TQ_ERR_WORKSPACE, "workspace too small");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (fast_eligible(kc, vc, d)) {
    if (launch_k4v2(kc, vc, d, static_cast<float*>(workspace), false, nullptr, nullptr, 0, nullptr, 0, s) != 0)
      TQ_LAUNCH_CHECK("measurement partials");
    return TQ_OK;
  }
  UniformArgs u;
  if (split_eligible(kc, vc, d) && fill_split(u, kc, vc, d, static_cast<float*>(workspace))) {
    if (launch_uniform_split(u, d->hq / d->hkv, split_kind(kc), split_kind(vc), 0, s) != 0)
      TQ_LAUNCH_CHECK("measurement partials (fractional widths)");
    return TQ_OK;
  }
  if (!widths_eligible(kc, vc, d) || !fill_uniform(u, kc, vc, d, static_cast<float*>(workspace), true))
    return set_error(TQ_ERR_UNSUPPORTED, "measurement: not a packed uniform or K4/V2 call");
  if (launch_uniform_widths(u, d->hq / d->hkv, kc->bits_hi, vc->bits_hi, 0, s) != 0)
    TQ_LAUNCH_CHECK("measurement partials (widths)");
  return TQ_OK;
}

// Test hook, not part of the ABI: the route tq_decode_attention takes for a
// valid call, without launching anything: 0 the general kernel, 1 the dense
// kernel, 2 the K4/V2 kernels, 3 the K4/V2 kernels with the QJL terms, 4 the
// uniform-batch kernels of the other integer widths, 5 those of the
// fractional widths, 6 the query-tiled prefill kernels.
int tq_debug_decode_route(const tq_codec* kc, const tq_codec* vc, const tq_attn_desc* d) {
  if (!kc || !vc || !d || d->hkv <= 0 || d->hq % d->hkv) return -1;
  if (d->flags & TQ_ATTN_GENERAL) return 0;
  if (prefill_eligible(kc, vc, d)) return 6;
  if (d->max_comp == 0 && (d->max_sink > 0 || d->max_res > 0) && dense_check(d, kc->d, false) == TQ_OK) return 1;
  if (d->qjl && d->max_comp > 0 && fast_eligible(kc, vc, d, true)) return 3;
  if (fast_eligible(kc, vc, d)) return 2;
  int nwg, bpw, fpw;
  if (widths_eligible(kc, vc, d) && uniform_route(vc, d, nwg, bpw, fpw, true)) return 4;
  if (split_eligible(kc, vc, d) && uniform_route(vc, d, nwg, bpw, fpw)) return 5;
  return 0;
}

// Test hook, not part of the ABI: the grid of the uniform-batch kernels for a
// call, without launching anything: out[0..3] = workgroups per (sequence, kv
// head), compressed 32-token blocks per workgroup, fp16 tokens per workgroup
// and the blocks-per-wave instantiation (4 or 8) the launch selects. Returns
// -1 when the uniform-batch grid does not take the call.
int tq_debug_uniform_geometry(const tq_codec* kc, const tq_codec* vc, const tq_attn_desc* d, int32_t* out) {
  if (!kc || !vc || !d || !out || d->hkv <= 0 || d->hq % d->hkv) return -1;
  int nwg, bpw, fpw;
  if (!uniform_route(vc, d, nwg, bpw, fpw, true)) return -1;
  out[0] = nwg;
  out[1] = bpw;
  out[2] = fpw;
  out[3] = bpw > FAST_WAVES * 4 ? 8 : 4;  // the selection of launch_u / launch_w
  return 0;
}

size_t tq_decode_noalloc_scratch_bytes(void) { return TQ_NOALLOC_SCRATCH_BYTES; }

int tq_decode_attention_noalloc(const tq_codec* kc, const tq_codec* vc, const tq_attn_desc* d, void* stream) {
  // the call is validated before its scratch size is computed: a malformed
  // descriptor gets TQ_ERR_INVALID, not a size error
  const int vrc = check_attention_call(kc, vc, d);
  if (vrc) return vrc;
  const size_t need = tq_attention_workspace_bytes(kc, vc, d);
  if (need > TQ_NOALLOC_SCRATCH_BYTES)
    return set_error(TQ_ERR_WORKSPACE, "call needs %zu bytes of scratch; the no-allocation entry point holds %zu",
                     need, (size_t)TQ_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  const int rc = noalloc_scratch(&ws);
  if (rc) return rc;
  return tq_decode_attention(kc, vc, d, ws, TQ_NOALLOC_SCRATCH_BYTES, stream);
}

size_t tq_dense_decode_workspace_bytes(const tq_attn_desc* d, int32_t head_dim) {
  if (!d || head_dim != 128 || d->hkv <= 0 || d->batch <= 0) return 0;
  return (dense_workspace(d) + 255) & ~(size_t)255;
}

int tq_dense_decode_attention(const tq_attn_desc* d, int32_t head_dim, void* workspace, size_t workspace_bytes,
                              void* stream) {
  if (!d) return set_error(TQ_ERR_INVALID, "attention descriptor is NULL");
  const int rc = dense_check(d, head_dim);
  if (rc) return rc;
  return dense_run(d, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

}  // extern "C"
