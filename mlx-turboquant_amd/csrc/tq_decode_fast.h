// Arguments of the decode-attention kernels: the K4/V2 partials + merge
// kernels (tq_decode_fast.hip) and the dense fp16 / bf16 kernel
// (tq_decode_dense.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/tq_abi.h"

namespace tq {

constexpr int FAST_WAVES = 8;          // waves per workgroup of the K4/V2 partials kernel
constexpr int FAST_PART_FLOATS = 132;  // per query head per dense-kernel partial: M, L, pad, pad, out[128]
// per query head per K4/V2 partial: M, L, has_orig, pad, rotated out[128],
// original-space out[128] (both / L)
constexpr int PACKED_PART_FLOATS = 260;
constexpr int FAST_MAX_WG = 256;       // partials per (sequence, kv head) of the dense kernel

// Per-call arguments of the K4/V2 partials kernel and its merge kernel.
// Work plan: sequence b has P_b = ceil(comp_b / 32) packed blocks and
// ntl_b = ceil((sink_b + res_b) / 16) fp16 tiles; W_b = max(P_b, [ntl_b > 0])
// units per kv head. With U = hkv sum_b W_b the units of (b, g) are cut into
// n_b = ceil(W_b / T) chunks of T = ceil(U / (chunks nwg)) units (rounded up to
// a multiple of 8, the waves of a workgroup); chunk j takes packed blocks
// [j T, (j + 1) T) and fp16 tiles [j tpc, (j + 1) tpc), tpc = ceil(ntl_b / n_b),
// and is partial slot N_b + g n_b + j (N_b = hkv sum_{b' < b} n_b').
// Workgroup p of the nwg takes the chunks [p V / nwg, (p + 1) V / nwg) of
// the V = N_batch in total.
struct FastArgs {
  const uint8_t* kc;  int64_t k_hs;    // 4-bit key codes, 64-byte rows
  const float* kn;    int64_t kn_hs;   // key norms
  const uint8_t* vc;  int64_t v_hs;    // 2-bit value codes, 32-byte rows
  const float* vn;    int64_t vn_hs;   // value norms
  const uint16_t* sink_k; const uint16_t* sink_v; int64_t sink_hs;   // fp16, elements
  const uint16_t* res_k;  const uint16_t* res_v;  int64_t res_hs;    // fp16 ring
  int res_cap, res_start0;
  const int32_t* comp_len_b;
  const int32_t* sink_len_b;
  const int32_t* res_len_b;
  const int32_t* res_start_b;
  int max_comp, max_sink, max_res;
  const void* q; int q_dtype;
  float* out;
  int batch, hq, hkv;
  float qscale;          // scale * log2(e)
  const uint16_t* rot16; // (2, 128, 128) fp16 high part / remainder of R (key codec): query rotation
  const float* vrot;     // (128, 128) R float32, row-major (value codec): inverse rotation in the merge
  const uint64_t* klut;  // (256,) key decode table of the key codec (tq_codec.decode_table)
  const uint64_t* vlut;  // (256,) value decode table of the value codec
  float vscale;          // value centroid i = vscale * table value i
  float* part;           // (vmax, G, PACKED_PART_FLOATS) partials
  int nwg;               // workgroups of the partials kernel
  int chunks;            // target chunks per workgroup (1 when every sequence has the maximal lengths)
  int vmax;              // partial slots (upper bound of V)
  int uni;               // 1: every sequence has the maximal lengths; the plan below is set
  int plan_T, plan_nu, plan_V;  // uniform plan: units per chunk, chunks per (b, g), chunks
  // QJL sketch terms (partials kernel with QB): per (sequence, kv head, query
  // head) rows of qb_hs floats indexed by compressed token
  const float* qjl_bias; // added to each compressed token's base-2 score
  float* scores;         // final base-2 scores of the compressed tokens (written)
  int64_t qb_hs;
  float* ml;             // merge output: (batch, hq, 2) global max and sum, or NULL
  int32_t* plan_tab;     // (batch, 2): first partial slot N_b and chunks n_b per kv head of each sequence,
                         // written by the partials kernel when uni == 0 (workspace, after the partials)
  // QJL key term computed in the partials kernel (QB): the keys' sketch (sign
  // rows of qm / 8 bytes, one residual norm per token) against S (scale q) of
  // the segment's query heads, computed at the query rotation from S
  const uint8_t* ksg; int64_t ksg_hs;  // key sign rows (bytes)
  const float* kgam;  int64_t kgam_hs; // key residual norms (elements)
  const float* sproj;    // (qm, 128) S float32, row-major (zero rows past the sketch's projections)
  float sscale;          // scale (S q in natural units)
  int qm;                // projections of the sketch (a multiple of 32, at most 256): sign rows of qm / 8 bytes
  // QJL value term added by the merge (decode_merge_kernel with QV): per
  // (sequence, query head) qnvc value partials of qm floats, each the sum
  // over its tokens of 2^(s - umax) gamma (-z) times -2^(E - 14), weighted by
  // 2^(umax - M) / L in the merge, times sqrt(pi / 2) / 128 through S^T
  const float* qjl_up;   // (batch, hq, qnvc, qm)
  const float* qjl_umax; // (batch, hq, qnvc)
  int qnvc;              // value partials per (sequence, query head)
  int qtok;              // tokens per value partial
};

// Host-side sizing of the K4/V2 path for a call: workgroups, chunks per
// workgroup and the partial slots the workspace must hold.
void fast_plan_host(int batch, int hkv, int max_comp, int max_sink, int max_res, bool uniform, int cus,
                    int& nwg, int& chunks, int& vmax);
// The uniform plan (every sequence at the maximal lengths): T, n and V.
void fast_uniform_plan(int batch, int hkv, int max_comp, int max_sink, int max_res, int nwg, int chunks, int& T,
                       int& nu, int& V);
// Launches the partials kernel and, when merge != 0, the merge kernel. G in
// {1, 2, 4, 8}; qb 1 / 2: with the QJL key term of a sketch of at most 128 /
// 256 projections computed in the kernel (ksg, kgam, sproj, sscale, qm), the
// final scores stored.
int launch_fast_decode(const FastArgs& a, int G, int qb, int merge, hipStream_t s);
// The merge kernel alone, with the QJL value term of qjl_up (qv = 1 for
// sketches of at most 128 projections, 2 for at most 256).
int launch_fast_merge_qjl(const FastArgs& a, int G, int qv, hipStream_t s);

// Merge of per-workgroup partials in original space ([M, L, pad, pad,
// out[128] / L] per query head, nwg per (sequence, kv head)) into out
// (batch, hq, 128) float32: the dense kernel's partials.
int launch_partial_merge(float* part, int nwg, int G, int hq, int hkv, int batch, float* out, hipStream_t s);

// Arguments of the K4/V2 kernels for uniform batches (tq_decode_uniform.hip):
// grid (nwg, hkv, batch), workgroup c of (b, g) takes the compressed blocks
// [c bpw, (c + 1) bpw) and the fp16 tokens [c fpw, (c + 1) fpw) of the
// [sink | ring] list; partials with a rotated and an original-space part
// (PACKED_PART_FLOATS per query head, nwg per (b, g)).
constexpr int UNI_BLOCKS_PER_WAVE = 8;  // compressed blocks per wave at most (kernels for 4 and 8)
constexpr int UNI_FP16_PER_WG = 16;     // fp16 tokens per workgroup, staged in LDS
constexpr int UNI_MAX_WG = 256;         // workgroups per (sequence, kv head)

struct UniformArgs {
  const uint8_t* kc;  int64_t k_hs;    // 4-bit key codes, 64-byte rows
  const float* kn;    int64_t kn_hs;   // key norms
  const uint8_t* vc;  int64_t v_hs;    // 2-bit value codes, 32-byte rows
  const float* vn;    int64_t vn_hs;   // value norms
  const void* sink_k; const void* sink_v; int64_t sink_hs;   // fp16, elements
  const void* res_k;  const void* res_v;  int64_t res_hs;    // fp16 ring
  int res_cap, res_start0;
  const int32_t* res_start_b;  // per-sequence ring starts (NULL: res_start0); lengths are the maximal ones
  int max_comp, max_sink, max_res;
  const void* q; int q_dtype;
  float* out;
  int batch, hq, hkv;
  float qscale;          // scale * log2(e)
  const uint16_t* rot16; // (2, 128, 128) fp16 high part / remainder of R (key codec): query rotation
  const float* vrot;     // (128, 128) R float32, row-major (value codec): inverse rotation in the merge
  uint32_t khl[16];      // key centroid i: fp16 bits of c_hi = fp16(c) | fp16(c - c_hi) << 16
  uint32_t vtab[4];      // value table: fp16 bits of entry i (tq_codec.value_table)
  float vscale;          // value centroid i = vscale * table value i
  float* part;           // per-workgroup partials (workspace)
  int nwg, bpw, fpw;
  const float* qjl_bias; // QJL key term (partials kernel with QB), rows of qb_hs floats
  float* scores;         // final base-2 scores of the compressed tokens (written with QB)
  int64_t qb_hs;
  float* ml;             // merge output: (batch, hq, 2) global max and sum, or NULL
  uint32_t vhl[16];      // value centroid i (3- / 4-bit values): fp16 bits of c_hi | c_lo << 16
  // per-sequence lengths (NULL: the maximal ones); read by the kernels of the
  // other widths only (the K4/V2 instantiation serves uniform calls)
  const int32_t* comp_len_b;
  const int32_t* sink_len_b;
  const int32_t* res_len_b;
  // fractional widths (split codebooks, tq_decode_split.h): the low-width
  // code rows of keys and values and the four codebooks in device memory
  const uint8_t* kcl; int64_t kl_hs;
  const uint8_t* vcl; int64_t vl_hs;
  const float* kcen_hi; const float* kcen_lo;
  const float* vcen_hi; const float* vcen_lo;
};
// Launches the uniform-batch partials kernel (qb: with the QJL key bias,
// scores stored) and, when merge != 0, its merge kernel. G in {1, 2, 4, 8};
// bf16_kv: the sink / ring tokens are bf16 (else fp16).
int launch_uniform_decode(const UniformArgs& a, int G, bool qb, int merge, hipStream_t s, bool bf16_kv = false);
// The same kernels for the other integer widths (key bits kb, value bits vb
// in 2..4, (kb, vb) != (4, 2)), without the QJL term (tq_decode_widths.hip).
int launch_uniform_widths(const UniformArgs& a, int G, int kb, int vb, int merge, hipStream_t s);
// The split-codebook kernels (tq_decode_split.h): fractional widths (3.5 =
// 4 / 3 bits, 2.5 = 3 / 2, split at dim 64) on at least one side, the other
// side fractional or integer; no QJL term. A width kind is bits_hi + bits_lo
// of a fractional codec (7 or 5) or the bits of an integer one (2 to 4).
int launch_uniform_split(const UniformArgs& a, int G, int kkind, int vkind, int merge, hipStream_t s);

// Arguments of the dense (fp16 / bf16 K/V) decode-attention kernel: the
// fp16 segments of tq_attn_desc, head_dim 128.
struct DenseArgs {
  const void* sink_k; const void* sink_v; int64_t sink_hs;   // elements
  const void* res_k;  const void* res_v;  int64_t res_hs;    // ring
  int res_cap, res_start0;
  const int32_t* sink_len_b;
  const int32_t* res_len_b;
  const int32_t* res_start_b;
  int max_sink, max_res;
  const void* q; int q_dtype;
  float* out;
  int hq, hkv;
  float qscale;          // scale * log2(e)
  float* part;           // per-workgroup partials (workspace), unused when nwg == 1
  int nwg;               // workgroups per (sequence, kv head)
  int bpw;               // 32-token blocks per wave
};

constexpr int DENSE_WAVES = 4;  // waves per workgroup of the dense kernel

// Power of two 2^qe of one query head for the fp16 query operands of the
// K4/V2 and uniform-batch kernels (s = qscale, the scores' scale): a head
// with s ||q|| above `hi` is scaled down to at most `hi`; a head with
// s ||q|| below `lo` (the fp16 remainders of its rotated coordinates s (R q)_j
// would go subnormal) is scaled up with both 2^-qe ||q|| and 2^-qe s ||q||
// at most `hi`; otherwise 0. The scores of the head are multiplied by 2^qe.
__device__ inline int query_exponent(float qnorm, float qscale, float hi, float lo) {
  const float qn = qnorm * qscale;
  if (qn > hi) return (int)ceilf(log2f(qn / hi));
  if (qn < lo && qnorm > 0.f) return max(min((int)ceilf(log2f(qnorm * fmaxf(qscale, 1.f) / hi)), 0), -100);
  return 0;
}

void dense_geometry(int batch, int hkv, int max_sink, int max_res, int cus, int& nwg, int& bpw);
// bf: bf16 K/V (else fp16); merge 0 skips the merge launch (measurement)
int launch_dense_decode(const DenseArgs& a, int G, bool bf, int batch, int merge, hipStream_t s);

// Prefill attention (n_q > 1, tq_prefill.h): a wave owns PREFILL_WAVE_ROWS
// query rows (PREFILL_TILES 16-row MFMA column tiles), a workgroup
// PREFILL_WAVES waves; partials of PREFILL_PART_FLOATS floats per (key-range
// split, query row): max, sum, pad, pad, rotated output / sum.
constexpr int PREFILL_TILES = 2;
constexpr int PREFILL_WAVE_ROWS = 16 * PREFILL_TILES;
constexpr int PREFILL_WAVES = 8;
constexpr int PREFILL_PART_FLOATS = 132;
constexpr int PREFILL_TARGET_WG = 256;  // workgroups a launch aims for (one per CU)

struct PrefillArgs {
  int batch, hq, hkv, G, n_q, kvrows;
  int nrows, nrows_pad;         // query rows per kv row (n_q G) and that padded to whole waves
  int nd_pad, nbd, nbc;         // uncompressed tokens per kv row padded to 32; their blocks; compressed blocks
  int nsplit, bps;              // key-range splits and blocks per split
  int max_comp, max_sink, max_res;
  const int32_t* comp_len; const int32_t* sink_len; const int32_t* res_len; const int32_t* res_start;
  int res_start0, res_cap;
  const uint8_t* kc; int64_t k_hs;   // key code rows (16 KB bytes)
  const uint8_t* vc; int64_t v_hs;   // value code rows (16 VB bytes)
  const float* kn; int64_t kn_hs;
  const float* vn; int64_t vn_hs;
  const float* kcen; const float* vcen;  // codebooks (2^KB, 2^VB floats)
  const void* sink_k; const void* sink_v; int64_t sink_hs;
  const void* res_k; const void* res_v; int64_t res_hs;
  int kv_dtype;
  const void* q; int q_dtype;
  const float* rk; const float* rv;  // key / value codec R (128 x 128, row-major)
  float scale;
  // workspace
  float* qr;      // (kvrows, nrows_pad, 128) rotated queries
  uint16_t* dk;   // (kvrows, nd_pad, 2, 128) uncompressed keys: unit vector fp16 high part, remainder
  uint16_t* dv;   // (kvrows, nbd, 2, 128, 32) uncompressed values, transposed, PV k-slot order
  float* dnk;     // (kvrows, nd_pad) their norms
  float* dnv;
  float* part;    // (nsplit, kvrows, nrows_pad, PREFILL_PART_FLOATS)
  float* out;     // (batch, hq, n_q, 128)
};

// The prefill route: eligibility, workspace bytes of a call, and the launch
// (preparation, partials, merge kernels) with the workspace carved as above.
bool prefill_eligible(const tq_codec* kc, const tq_codec* vc, const tq_attn_desc* d);
size_t prefill_workspace(const tq_attn_desc* d);
int prefill_run(const tq_codec* kc, const tq_codec* vc, const tq_attn_desc* d, void* workspace, hipStream_t s);

}  // namespace tq
