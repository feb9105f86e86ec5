// Arguments of the K4/V2 decode-attention kernels (per-workgroup partials, then a merge).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tq {

struct FastArgs {
  const uint8_t* kc;  int64_t k_hs;    // 4-bit key codes, 64-byte rows
  const float* kn;    int64_t kn_hs;   // key norms
  const uint8_t* vc;  int64_t v_hs;    // 2-bit value codes, 32-byte rows
  const float* vn;    int64_t vn_hs;   // value norms
  const void* sink_k; const void* sink_v; int64_t sink_hs;   // fp16, elements
  const void* res_k;  const void* res_v;  int64_t res_hs;    // fp16 ring
  int res_cap, res_start0;
  const int32_t* comp_len_b;
  const int32_t* sink_len_b;
  const int32_t* res_len_b;
  const int32_t* res_start_b;
  int max_comp, max_sink, max_res;
  const void* q; int q_dtype;
  float* out;
  int hq, hkv;
  float qscale;          // scale * log2(e)
  const uint16_t* rot16; // (2, 128, 128) fp16 high part / remainder of R (key codec)
  const uint16_t* rotT;  // (2, 128, 128) bf16 high part / remainder of R^T (value codec)
  const float* kcen;     // 16 key centroids
  const float* vcen;     // 4 value centroids
  float* part;           // per-workgroup partials (workspace)
  int nwg;               // workgroups per (sequence, kv head)
  int bpw;               // compressed 32-token blocks per workgroup (<= FAST_WAVES * FAST_BLOCKS_PER_WAVE)
  int fpw;               // fp16 (sink / residual) tokens per workgroup (<= FAST_FP16_PER_WG)
  int merge;             // 1: launch the merge kernel too; 0: partials only (measurement)
  // QJL sketch terms (the fast kernel with QB): per (sequence, kv head, query
  // head) rows of qb_hs floats indexed by compressed token
  const float* qjl_bias; // added to each compressed token's base-2 score
  float* scores;         // final base-2 scores of the compressed tokens (written)
  int64_t qb_hs;
  float* ml;             // merge output: (batch, hq, 2) global max and sum, or NULL
};

size_t fast_smem_bytes();
int fast_set_attributes();
int launch_fast_decode(const FastArgs& a, int G, int batch, hipStream_t s);
// the same kernels with the QJL key bias added to the scores and the scores stored (a.qjl_bias, a.scores)
int launch_fast_decode_qjl(const FastArgs& a, int G, int batch, hipStream_t s);

constexpr int FAST_WAVES = 8;            // waves per workgroup of the decode kernel
constexpr int FAST_BLOCKS_PER_WAVE = 4;  // compressed blocks per wave (two in flight at a time)
constexpr int FAST_FP16_PER_WG = 16;     // fp16 tokens per workgroup, staged in LDS
constexpr int FAST_MAX_WG = 256;         // workgroups per (sequence, kv head)
constexpr int FAST_PART_FLOATS = 132;    // per query head per workgroup: M, L, pad, pad, out[128] (original space, / L)

// Merge of per-workgroup partials (FAST_PART_FLOATS per query head, nwg per
// (sequence, kv head)) into out (batch, hq, 128) float32.
int launch_partial_merge(float* part, int nwg, int G, int hq, int hkv, int batch, float* out, hipStream_t s);

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

void dense_geometry(int batch, int hkv, int max_sink, int max_res, int cus, int& nwg, int& bpw);
// bf: bf16 K/V (else fp16); merge 0 skips the merge launch (measurement)
int launch_dense_decode(const DenseArgs& a, int G, bool bf, int batch, int merge, hipStream_t s);

}  // namespace tq
