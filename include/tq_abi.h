/*
 * tq_abi.h — C ABI of the MI355X (gfx950) TurboQuant KV-cache library.
 *
 * The reference (alex-rentel/mlx-turboquant) has no C ABI: its native code is
 * Metal source dispatched through mx.fast.metal_kernel. Each entry point below
 * replaces one reference operation on the compress / compressed-attention path;
 * the comment above it names the reference interface it stands in for.
 *
 * Conventions
 *   - Every pointer is a device pointer unless stated otherwise; the caller owns
 *     every buffer (including the attention workspace).
 *   - fp16 tensors are passed as `const void*` holding IEEE binary16 values.
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the null stream) and
 *     is stream-ordered; the functions do not synchronise.
 *   - Return value: TQ_OK (0) or a negative TQ_ERR_* code; tq_last_error()
 *     returns the message of the most recent failure on the calling thread.
 *   - Stores are rows of (batch b, head h) = row r = b*heads + h. Within a row,
 *     token t of a packed array starts at byte t*row_bytes; norms / gamma are
 *     one float per token.
 */
#ifndef TQ_ABI_H
#define TQ_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TQ_ABI_VERSION 3

/* Element types of floating-point inputs. */
enum { TQ_F16 = 0, TQ_BF16 = 1, TQ_F32 = 2 };

enum {
  TQ_OK = 0,
  TQ_ERR_INVALID = -1,     /* bad argument: reference raises ValueError / AssertionError */
  TQ_ERR_UNSUPPORTED = -2, /* width / head_dim not supported: reference ValueError */
  TQ_ERR_LAUNCH = -3,      /* HIP launch or runtime failure */
  TQ_ERR_WORKSPACE = -4    /* workspace too small */
};

/* Quantizer description shared by compress / dequantize / attention.
 * Integer widths: bits_hi == bits_lo == bits, split == d.
 * Fractional widths (e.g. 3.5): rotated dims [0, split) use bits_hi and
 * [split, d) use bits_lo with split == d/2 (mlx_turboquant/cache.py:63-84).
 * Both codebooks are the d-dimensional Lloyd-Max tables (codebook.py:146-174). */
typedef struct tq_codec {
  int32_t d;                   /* head_dim: a multiple of 16 in [16, 256] */
  int32_t bits_hi;             /* 1..4 */
  int32_t bits_lo;             /* 1..4 */
  int32_t split;               /* a multiple of 16 in [16, d] */
  const float* rotation;       /* (d, d) row-major orthogonal R (rotation.py:17-36) */
  const float* centroids_hi;   /* (2^bits_hi,) */
  const float* boundaries_hi;  /* (2^bits_hi - 1,) */
  const float* centroids_lo;   /* (2^bits_lo,)  (== _hi for integer widths) */
  const float* boundaries_lo;  /* (2^bits_lo - 1,) */
  const float* qjl_proj;       /* (qjl_m, d) Gaussian S (qjl.py:23-36) or NULL */
  int32_t qjl_m;               /* number of projections (multiple of 32) or 0 */
  int32_t flags;               /* TQ_CODEC_* bits */
  const uint16_t* rotation_parts; /* (2, d, d) 16-bit words, row-major, or NULL:
                                     [0] = fp16(R), [1] = fp16(R - [0]).
                                     The K4/V2 decode kernels rotate the query
                                     with the key codec's planes (the output
                                     goes back with the value codec's float32
                                     `rotation`); others ignore it. Arrays with
                                     more planes work: only [0, 1] are read. */
  /* Host-side tables, filled by tq_codec_prepare() from a host copy of
   * centroids_hi (codebooks of at most 16 entries; passed to kernels by value):
   * host_centroids = centroids_hi, n_host_centroids entries; and for 2-bit
   * codebooks an exact fp16 copy for the K4/V2 decode kernels (value side):
   * centroids_hi[i] == value_scale * fp16 value_table[i] to within
   * value_table_err (relative). The K4/V2 route runs only when the key
   * codec has rotation_parts, 16 host_centroids and its decode_table, and the
   * value codec its decode_table with value_table_err <= 2e-7 (else the
   * general kernels). */
  float host_centroids[16];
  int32_t n_host_centroids;
  uint16_t value_table[4];
  float value_scale;
  float value_table_err;
  /* (256,) 8-byte entries in device memory, or NULL: the decode table of the
   * K4/V2 kernels for code byte e. 4-bit codecs: fp16 bits of (c_hi[e & 15],
   * c_hi[e >> 4], c_lo[e & 15], c_lo[e >> 4]) in 16-bit lanes 0..3, c_hi =
   * fp16(c), c_lo = fp16(c - c_hi); 2-bit codecs: value_table[(e >> 2i) & 3]
   * in lane i. tq_codec_decode_table() computes it on the host. */
  const uint64_t* decode_table;
} tq_codec;

/* tq_codec.flags: route tq_compress calls with this codec through the
 * general compress kernel instead of the MFMA kernel (no reference
 * counterpart; lets tests compare the two kernels, per call). */
#define TQ_CODEC_GENERAL_COMPRESS 1

/* Fills the host-side tables of `codec` (host_centroids, value_table,
 * value_scale, value_table_err) from a host copy of centroids_hi
 * (n_centroids entries; the value table needs 4, other sizes set its error
 * to infinity; more than 16 leave host_centroids unset). Host only, no
 * device work. Returns TQ_OK. */
int tq_codec_prepare(tq_codec* codec, const float* centroids_host, int32_t n_centroids);

/* The 256 entries of decode_table for a prepared codec (host only, no device
 * work): the 4-bit form for n_host_centroids == 16, the 2-bit form for 4.
 * Returns TQ_ERR_UNSUPPORTED for other codebooks. The caller copies them to
 * device memory and sets codec->decode_table. */
int tq_codec_decode_table(const tq_codec* codec, uint64_t* table_host);

/* A compressed store: packed codes, norms and optional QJL sketch.
 * codes_hi rows are split*bits_hi/8 bytes, codes_lo rows (d-split)*bits_lo/8
 * (NULL for integer widths), signs rows qjl_m/8 bytes (LSB-first, bit i set
 * when projection i of the residual is >= 0). Head strides are in bytes for
 * codes/signs and in elements for norms/gamma. */
typedef struct tq_store {
  uint8_t* codes_hi;
  int64_t hi_head_stride;
  uint8_t* codes_lo;
  int64_t lo_head_stride;
  float* norms;
  int64_t norm_head_stride;
  uint8_t* signs;
  int64_t sign_head_stride;
  float* gamma;
  int64_t gamma_head_stride;
} tq_store;

/* Vector set addressed by (row, token): `rows` rows of `heads` heads per batch
 * element; per-batch token counts / offsets are optional device int32 arrays
 * (NULL = uniform `n_tok`, offset 0). */
typedef struct tq_span {
  int32_t rows;                  /* batch * heads */
  int32_t heads;                 /* heads per batch element */
  int32_t n_tok;                 /* tokens per row (upper bound when n_tok_b != NULL) */
  int32_t reserved;
  const int32_t* n_tok_b;        /* (batch,) tokens per row, or NULL */
  const int32_t* src_tok0_b;     /* (batch,) first source token, or NULL */
  const int32_t* dst_tok0_b;     /* (batch,) first destination token, or NULL */
} tq_span;

/* Library / error handling. */
int tq_abi_version(void);
const char* tq_last_error(void);
/* Returns 1 when the library holds a code object for the current device. */
int tq_device_supported(void);

/* Compress fp16 vectors: norm -> normalise -> rotate -> quantize -> pack, and
 * (when codec->qjl_proj != NULL and dst->signs != NULL) the QJL sign sketch and
 * residual norm of x - dequantize(codes).
 * Replaces TurboQuantKVCache._quantize_kv / _quantize_kv_fractional
 * (mlx_turboquant/cache.py:232-274), TurboQuantMSE.quantize
 * (quantizer.py:54-86) and metal_quantize_4bit (kernels.py:363-409); the QJL
 * part replaces qjl_quantize on the residual (qjl.py:47-67, cache.py:396-427).
 * x: x_dtype (TQ_F16 / TQ_BF16 / TQ_F32), element (r, t, i) at
 * x[r*x_head_stride + t*d + i]; the value is cast to float32 exactly. */
int tq_compress(const tq_codec* codec, const void* x, int32_t x_dtype, int64_t x_head_stride,
                const tq_span* span, const tq_store* dst, void* stream);


/* Dequantize: out = n * (c[idx] @ R) (+ QJL correction when apply_qjl and
 * the store holds a sketch), float32, element (r, t, i) at
 * out[r*out_head_stride + t*d + i].
 * Replaces metal_dequantize (kernels.py:313-360), _dequantize_kv /
 * _dequantize_kv_fractional (cache.py:276-343), TurboQuantMSE.dequantize
 * (quantizer.py:88-109) and qjl_dequantize (qjl.py:70-94). */
int tq_dequantize(const tq_codec* codec, const tq_store* src, const tq_span* span,
                  float* out, int64_t out_head_stride, int32_t apply_qjl, void* stream);

/* LSB-first bit packing of uint8 codes, rows of d codes.
 * Replaces pack_indices / unpack_indices (packing.py:211-236). */
int tq_pack_codes(const uint8_t* idx, int64_t n_rows, int32_t d, int32_t bits,
                  uint8_t* packed, void* stream);
int tq_unpack_codes(const uint8_t* packed, int64_t n_rows, int32_t d, int32_t bits,
                    uint8_t* idx, void* stream);

/* idx = #{k : y > boundaries[k]} for float32 y (codebook.py:203-225). */
int tq_quantize_scalar(const float* y, int64_t n, const float* boundaries,
                       int32_t n_boundaries, uint8_t* idx, void* stream);

/* Decode attention over a TurboQuant cache (one query token per head).
 * out[b, h] = softmax(scale * q[b,h] . K_b^T) V_b with K_b / V_b the tokens
 * [sink | compressed | residual] of sequence b and kv head h / (hq / hkv),
 * compressed tokens read from packed codes (no dequantized cache), with the
 * QJL correction of the stored sketch when `qjl` is set.
 * Replaces the decode step update_and_fetch -> concat -> SDPA
 * (cache.py:620-706, docs/attention_source_dump.txt:22-31) and the research
 * fused_qk_scores_* kernels (kernels.py:558-629); interface follows the
 * proposed fused_attention_from_packed (docs/FUSED_SDPA_RESULTS.md:116-127). */
typedef struct tq_attn_desc {
  int32_t batch, hq, hkv, qjl;
  float scale;
  int32_t max_comp, max_sink, max_res;  /* host upper bounds (size the grid) */
  int32_t q_dtype, kv_dtype;            /* TQ_F16 / TQ_BF16 / TQ_F32 of q and of sink/residual */
  const void* q;                        /* (batch, hq, d) */
  float* out;                           /* (batch, hq, d) float32 */
  tq_store kstore, vstore;              /* rows = batch * hkv */
  const int32_t* comp_len;              /* (batch,) device, 0 <= comp_len[b] <= max_comp, or NULL = max_comp */
  const void* sink_k;                   /* kv_dtype (batch*hkv, sink_cap, d) or NULL */
  const void* sink_v;
  int64_t sink_head_stride;             /* elements */
  const int32_t* sink_len;              /* (batch,) device, 0 <= sink_len[b] <= max_sink, or NULL = max_sink */
  const void* res_k;                    /* kv_dtype ring (batch*hkv, res_cap, d) or NULL */
  const void* res_v;
  int64_t res_head_stride;              /* elements */
  int32_t res_cap, res_start0;          /* ring capacity; ring start when res_start == NULL */
  const int32_t* res_start;             /* (batch,) device ring start in [0, res_cap), or NULL = res_start0 */
  const int32_t* res_len;               /* (batch,) device, 0 <= res_len[b] <= max_res, or NULL = max_res.
                                           Kernels clamp every entry into these bounds (an out-of-range
                                           entry gives a wrong result for its sequence, never an access
                                           outside the stores, sink or ring). */
  int32_t flags;                        /* TQ_ATTN_* bits */
  int32_t n_q;                          /* query tokens per sequence: 0 / 1 decode; > 1 the last n_q
                                           tokens of each sequence attend causally (query i sees
                                           positions <= total - n_q + i), q and out (batch, hq, n_q, d)
                                           (cache.py:722-724 "causal" prefill mask): query-tiled MFMA
                                           kernels for integer widths 2-4 at d = 128 without a sketch,
                                           the general kernel otherwise */
} tq_attn_desc;

/* tq_attn_desc.flags: force the general kernel (every width / QJL) even where
 * the K4/V2 partials + merge kernels apply. */
#define TQ_ATTN_GENERAL 1

/* Workspace: scratch for the per-workgroup partials of one call (no state is
 * kept between calls, no initial contents are needed). Calls sharing a
 * workspace must be ordered on one stream or must not overlap.
 * tq_decode_workspace_bytes is an upper bound over every route the key codec
 * and descriptor allow; tq_attention_workspace_bytes is the need of the route
 * tq_decode_attention takes for (kcodec, vcodec, desc) (for prefill calls on
 * the query-tiled kernels far less than the general kernel's partials). */
size_t tq_decode_workspace_bytes(const tq_codec* kcodec, const tq_attn_desc* desc);
size_t tq_attention_workspace_bytes(const tq_codec* kcodec, const tq_codec* vcodec, const tq_attn_desc* desc);
int tq_decode_attention(const tq_codec* kcodec, const tq_codec* vcodec,
                        const tq_attn_desc* desc, void* workspace,
                        size_t workspace_bytes, void* stream);

/* Decode attention that allocates nothing: tq_decode_attention with the
 * workspace taken from a scratch array the library holds in device memory,
 * one copy per GPU, TQ_NOALLOC_SCRATCH_BYTES bytes, kept until the process
 * ends. No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). It calls no hipMalloc / hipFree; the
 * caller still passes q, out and the cache buffers through `desc`.
 * Calls whose tq_attention_workspace_bytes exceeds TQ_NOALLOC_SCRATCH_BYTES
 * return TQ_ERR_WORKSPACE. Every call on one GPU shares that GPU's scratch:
 * calls that overlap on one GPU (different streams, no ordering between them)
 * race; calls ordered on one stream do not. Nothing is carried from one call
 * to the next (the scratch needs no initial contents). The first call on a
 * device looks up that device's copy of the array. */
#define TQ_NOALLOC_SCRATCH_BYTES (64u << 20)
size_t tq_decode_noalloc_scratch_bytes(void);
int tq_decode_attention_noalloc(const tq_codec* kcodec, const tq_codec* vcodec,
                                const tq_attn_desc* desc, void* stream);

/* Decode attention over uncompressed K/V (one query token per head),
 * head_dim 128, fp16 or bf16 K/V (kv_dtype), q fp16 / bf16 / fp32: the
 * sink and residual-ring segments of `desc` with no compressed tokens
 * (desc->max_comp must be 0; kstore, vstore and qjl are not read). A plain
 * (batch*hkv, T_cap, 128) cache is a sink of length T (sink_len NULL,
 * max_sink = T, sink_head_stride = T_cap * 128).
 * Replaces the decode attention of the layers the reference keeps on an
 * uncompressed mlx-lm KVCache (outlier / skipped layers, patch.py:219-226 and
 * :337-338, attended by mlx SDPA over the fp16 K/V). tq_decode_attention sends
 * its calls with max_comp == 0 here too (same kernels). Same workspace rules
 * as tq_decode_attention. */
size_t tq_dense_decode_workspace_bytes(const tq_attn_desc* desc, int32_t head_dim);
int tq_dense_decode_attention(const tq_attn_desc* desc, int32_t head_dim, void* workspace,
                              size_t workspace_bytes, void* stream);

/* Append one token per (sequence, kv head) to residual rings of keys and
 * values: rows (batch*heads, ring_cap, d) of `dtype` (TQ_F16 / TQ_BF16) with
 * head stride ring_head_stride elements; token (b, h) of k and v (batch,
 * heads, d), contiguous, goes to slot slot_b[b] (device int32 array) of row
 * b*heads + h. Sequences with slot_b[b] outside [0, ring_cap) are skipped.
 * d and ring_head_stride multiples of 8, pointers 16-byte aligned. No
 * counterpart in the reference, whose fp16 tail grows by concatenation in
 * update_and_fetch (cache.py:620-706); the fixed ring of this library takes
 * its place, and one launch writes both sides of a decode step. */
int tq_ring_append(const void* k, const void* v, int32_t dtype, void* ring_k, void* ring_v,
                   int64_t ring_head_stride, int32_t ring_cap, int32_t batch, int32_t heads, int32_t d,
                   const int32_t* slot_b, void* stream);

/* One decode step of a ragged batch in one launch: the tq_ring_append of
 * k / v (batch, heads, 128) at slot_b[b], and the one-token drain of ring
 * position src_b[b] of every sequence with drain_b[b] == 1 into the key and
 * value stores at token dst_b[b] — the results of tq_ring_append followed by
 * tq_compress of each side over the rings (a span of n_tok 1 and n_tok_b /
 * src_tok0_b / dst_tok0_b = drain_b / src_b / dst_b), bit for bit (without a
 * sketch: as tq_compress with TQ_CODEC_GENERAL_COMPRESS; the default MFMA
 * compress kernel agrees with it outside the near-boundary band).
 * `seq_ints` is HOST memory: n_ints >= 4*batch int32 = [slot_b | drain_b |
 * src_b | dst_b | anything the caller adds], each array `batch` long; all
 * n_ints are copied to the device array `seq_ints_dev` in stream order
 * (later calls may read the caller's part there, e.g. an attention
 * descriptor's length arrays); seq_ints may be reused once the call returns.
 * A drained slot must differ from the sequence's append slot. Both codecs
 * head_dim 128, with a sketch of <= 128 projections (stored where the store
 * has sign rows) or none, rings fp16 or bf16 (dtype) with head stride
 * ring_head_stride elements, k, v and rings 16-byte aligned; other codecs
 * return TQ_ERR_UNSUPPORTED (use tq_ring_append + tq_compress). Replaces a
 * decode step of update_and_fetch with the chunk_size = 1 drain policy and
 * the QJL sketch of the drained vector (cache.py:396-427, 529-533, 620-706),
 * per sequence of a ragged batch. */
int tq_ragged_step(const tq_codec* kcodec, const tq_codec* vcodec, const void* k, const void* v, int32_t dtype,
                   void* ring_k, void* ring_v, int64_t ring_head_stride, int32_t ring_cap, const tq_store* kstore,
                   const tq_store* vstore, int32_t batch, int32_t heads, const int32_t* seq_ints, int32_t n_ints,
                   int32_t* seq_ints_dev, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TQ_ABI_H */
