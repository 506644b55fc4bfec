/*
 * bmx_k2b.h — C-ABI of the MI355X (gfx950) packed-KV "k2b" decode path.
 *
 * Drop-in boundary for pherber3/bmx's packed k2b decode path.  Plain C, plain
 * pointers and sizes; every pointer argument named "device" is HIP device
 * memory.  Calls are asynchronous on the HIP stream passed in (NULL = default
 * stream); they do not allocate.  Return value 0 = success, otherwise a
 * BMX_E_* code, with a message from bmx_last_error().
 *
 * Packed page format (one layer, PT = 16 tokens, head_dim 128, C = 128*h_kv
 * channels, rank R; sections in this order, little-endian).  "Lane 16q+n" is
 * the MFMA lane that reads the bytes, so every lane's slice is contiguous.
 *   US     [4][16][R/4] fp16  low-rank key coefficients: US[q][n][i] =
 *                             Us[token n][(R/4)q + i]
 *   VNORM  [h_kv][16]   fp16  value norm per (head, token)
 *   KSCALE [C/4]        fp16  key-residual scales of the page's 64-token group in
 *                             pair order F[128h + 2j + e] = scale of channel
 *                             128h + j + 64e (j < 64, e < 2); page slot s
 *                             (= logical page index mod 4) holds F[sC/4, (s+1)C/4)
 *   KRES   [h_kv][64][3] u32  3-bit key residual, offset binary (code + 4); lane
 *                             16q+n holds token n; pair p = 4b+i (b, i < 4) is
 *                             channels (j, j+64), j = 16b + 4q + i; pair p < 15:
 *                             dword p/5, low code at bit 3(p%5), high code at bit
 *                             16 + 3(p%5); pair 15: bit k of the low / high code
 *                             at bit 15 / 31 of dword k
 *   VCODE  [h_kv][64][2] u32  2-bit Lloyd value codes; lane 16q+m holds the code
 *                             of channel 16b+m (b < 8), token 4q+t (t < 4) at
 *                             dword b/4, bit 8(b%4) + 2t
 * Bytes per token = 2R + 86*h_kv  (752 at h_kv 8, R 32; 720 at R 16), i.e.
 * exactly the k2b bits-per-entry: 3 (residual) + 16/64 (scales) + 2 (V codes)
 * + 16*h_kv/C (norms) + 16R/C (Us).  The frozen basis V (C x R fp16) is stored
 * once per sequence and layer, outside the pages.
 *
 * Codec geometry of the reference recipe: codec page 128 tokens
 * (packed_streaming.py:438), key-scale group 64 tokens (recipes.py:31-42),
 * 3-bit keys / 2-bit values.
 *
 * General geometry.  The reference's fused path takes any power-of-two
 * head_dim and rank and the recipe's residual group (packed_streaming.py:
 * 957-975, recipes.py:31-56).  Every other geometry this library takes --
 * head_dim d in {32, 64, 128}, rank R in {16, 32, 64, 128} (R <= C), residual
 * group in {16, 32, 64, 128} tokens, 2..4-bit keys -- uses the general page
 * (same 16 tokens, C = d*h_kv; sections in this order, each starting on a
 * 16-byte boundary):
 *   US     [16][R]          fp16  Us[token][r]
 *   VNORM  [h_kv][16]       fp16  value norm per (head, token)
 *   KSCALE [C*16/group]     fp16  the group's C scales (channel c = d*h + j
 *                                 at c); page slot s (= logical page index
 *                                 mod group/16) holds scales
 *                                 [s*C*16/group, (s+1)*C*16/group)
 *   KRES   [h_kv][16][d/2]  u8    residual codes, offset binary (code +
 *                                 2^(bits-1)), channel j of (head, token) in
 *                                 the low (j even) / high nibble of byte j/2
 *   VCODE  [h_kv][4][d]     u8    2-bit value codes: byte (head, a, j) holds
 *                                 tokens 4a .. 4a+3 of channel j, token 4a+t
 *                                 at bits 2t
 * The 4-bit residual container is the reference's own packed form
 * (pack_signed_codes, triton_dequant_attention.py:49-165).
 */
#ifndef BMX_K2B_H
#define BMX_K2B_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BMX_K2B_PAGE_TOKENS 16
#define BMX_K2B_HEAD_DIM 128
#define BMX_K2B_GROUP 64
#define BMX_K2B_CODEC_PAGE 128

#define BMX_K2B_F16 0
#define BMX_K2B_F32 1
#define BMX_K2B_BF16 2

/* Decode query / output dtype (bmx_k2b_decode_args.io_dtype and
 * bmx_rtn_decode_args.io_dtype): zero keeps fp32. */
#define BMX_K2B_IO_F32 0
#define BMX_K2B_IO_F16 1
#define BMX_K2B_IO_BF16 2

/* Recent-window dtype (bmx_k2b_decode_args.tail_dtype and
 * bmx_rtn_decode_args.tail_dtype), for k_tail, v_tail, new_k and new_v: zero
 * keeps fp16; bf16 holds a bf16 model's rows as the model made them (the
 * reference keeps the tail in the model dtype, packed_streaming.py:849). */
#define BMX_K2B_TAIL_F16 0
#define BMX_K2B_TAIL_BF16 1

#define BMX_OK 0
#define BMX_E_INVALID 1     /* bad argument (shape, pointer, unsupported geometry) */
#define BMX_E_WORKSPACE 2   /* workspace missing or too small */
#define BMX_E_HIP 3         /* a HIP runtime call failed */

enum bmx_k2b_section {
  BMX_K2B_SEC_US = 0,
  BMX_K2B_SEC_VNORM = 1,
  BMX_K2B_SEC_KSCALE = 2,
  BMX_K2B_SEC_KRES = 3,
  BMX_K2B_SEC_VCODE = 4
};

typedef struct {
  int32_t h_kv;        /* KV heads: 1..16 for pages/append/dequant, 1..8 for decode */
  int32_t rank;        /* low-rank key rank R: 16 or 32 (any of 16..128: general page) */
  int32_t n_q_groups;  /* query heads per KV head G, 1..16 */
  int32_t head_dim;    /* 0 or 128; 32 or 64: general page */
  int32_t k_group;     /* residual scale group in tokens: 0 or 64; 16, 32 or 128: general page */
  int32_t k_bits;      /* residual bits: 0 or 3; 2 or 4: general page */
} bmx_k2b_geom;

/* Message of the last failed call on this thread ("" if none). */
const char* bmx_last_error(void);

/* Bytes of one 16-token page, and the (offset, size) of one section. */
size_t bmx_k2b_page_bytes(const bmx_k2b_geom* geom);
int bmx_k2b_page_section(const bmx_k2b_geom* geom, int section, size_t* offset,
                         size_t* bytes);

/* ------------------------------------------------------------------------
 * Decode attention.  Replaces fused_decode_attention_k2b + _finalize_decode
 * (cache/triton_dequant_attention.py:1232-1368, 504-575, 409-461) and the
 * chunked_dequant_attention decode loop (cache/chunked_attention.py:478-530).
 *
 * For each sequence b: one query step (G query heads per KV head) attends to
 * the packed_len[b] committed tokens held in pages (keys rebuilt as
 * Us*V^T + residual*scale, RoPE applied at read with angle fl32(inv_freq*pos))
 * and to the tail_len[b] fp16 recent-window tokens (post-RoPE keys), with one
 * base-e softmax over their union.  Output = softmax(q.K^T * sm_scale) . V.
 * ---------------------------------------------------------------------- */
typedef struct {
  bmx_k2b_geom geom;
  int32_t batch;
  const void* q;              /* device [batch][h_kv][G][head_dim] post-RoPE, in io_dtype */
  void* out;                  /* device [batch][h_kv][G][head_dim] in io_dtype */
  const uint8_t* pages;       /* device page pool; page i at pages + i*page_bytes */
  int32_t n_pool_pages;       /* pages in the pool; table entries are clamped into
                                 [0, n_pool_pages) so a bad entry cannot fault */
  const int32_t* page_table;  /* device [batch][max_pages] logical -> physical page, or
                                 NULL: contiguous pages, logical page i of sequence b
                                 at physical page b * max_pages + i (the kernel then
                                 requests the first pages at once, without a table
                                 read: the layout PackedStreamingLayer allocates) */
  int32_t max_pages;          /* row stride of page_table (of the pool when NULL) */
  const int32_t* packed_len;  /* device [batch] committed tokens, multiple of 128;
                                 clamped to max_packed_len on the device */
  int32_t max_packed_len;     /* host upper bound of packed_len (sizes the grid) */
  const uint16_t* basis;      /* device fp16 [C][R] frozen key basis of sequence 0 */
  int64_t basis_stride;       /* elements between sequences' bases (0 = shared) */
  float inv_freq[64];         /* RoPE inverse frequencies (HF inv_freq, fp32; the first
                                 head_dim/2 are read) */
  float rope_scaling;         /* cos/sin multiplier (HF attention_scaling, 1.0) */
  float sm_scale;             /* softmax scale (HF module.scaling) */
  float codebook[4];          /* 2-bit Lloyd levels, ascending */
  uint32_t v_sign_bits[4];    /* bit c set <=> V Hadamard sign of channel c is -1 */
  const uint16_t* k_tail;     /* device fp16 (tail_dtype) post-RoPE recent-window keys */
  const uint16_t* v_tail;     /* device fp16 (tail_dtype) recent-window values */
  int64_t tail_stride_b;      /* element strides of k_tail/v_tail (head_dim contiguous) */
  int64_t tail_stride_h;
  int64_t tail_stride_t;
  const int32_t* tail_len;    /* device [batch] recent-window length (clamped to tail_cap), or
                                 NULL: every sequence's window holds tail_len_value rows */
  int32_t tail_cap;           /* host upper bound of tail_len, 0..4096 */
  int32_t split_tokens;       /* 0 = one workgroup per CU, split over the batch (default):
                                 a batch of 2..64 sequences shares them in proportion
                                 to the sequences' device lengths (the workspace then
                                 holds CU count - batch + 1 partial slots per row);
                                 > 0 (multiple of 64) = about max_packed_len / split_tokens
                                 workgroups per sequence.  Packed tokens are dealt in
                                 64-token groups, balanced over the workgroups; the
                                 recent window is scored by the split kernel in
                                 16-token tiles (at least one workgroup per tile, up
                                 to one per CU) and summed by the merge kernel. */
  void* workspace;            /* device scratch: split partials (fp16 records, fp32 max
                                 and sum) and window scores (fp32) */
  size_t workspace_bytes;
  void* split_end_event;      /* optional hipEvent_t recorded on the stream between
                                 the split kernel and the combine kernel (timing) */
  int32_t tail_len_value;     /* window length of every sequence when tail_len is NULL
                                 (0..tail_cap): a host value, no device read */
  const uint16_t* new_k;      /* with tail_len NULL, optionally the window's newest n_new
                                 rows (the step's own token) given apart: device fp16
                                 post-RoPE keys, row i of (b, h) at b*new_stride_b +
                                 h*new_stride_h + i*new_stride_t, rows tail_len_value -
                                 n_new .. tail_len_value - 1 of the window.  They are
                                 attended from here and copied into k_tail / v_tail, so
                                 the caller writes no window row for a decode step */
  const uint16_t* new_v;      /* device fp16 values of the same rows, same strides */
  int64_t new_stride_b;
  int64_t new_stride_h;
  int64_t new_stride_t;
  int32_t n_new;              /* rows given apart, 0..tail_len_value (0 = none) */
  int32_t io_dtype;           /* BMX_K2B_IO_F32 (0), _F16 or _BF16: the dtype of q and out
                                 (the model's: fused_decode_attention_k2b takes q in the
                                 model dtype, triton_dequant_attention.py:1232-1246) */
  int32_t tail_dtype;         /* BMX_K2B_TAIL_F16 (0) or _BF16: the dtype of the window
                                 rows (k_tail, v_tail, new_k, new_v) */
} bmx_k2b_decode_args;

size_t bmx_k2b_decode_workspace_bytes(const bmx_k2b_decode_args* args);
int bmx_k2b_decode(const bmx_k2b_decode_args* args, void* stream);

/* Allocation-free decode: no counterpart in the reference.  For callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments and results as
 * bmx_k2b_decode, except that workspace / workspace_bytes are ignored: the
 * split partials live in a static device array of
 * BMX_K2B_DECODE_SCRATCH_BYTES that every GPU the library runs on holds until
 * the process ends.  A call whose bmx_k2b_decode_workspace_bytes() exceeds it
 * fails with BMX_E_WORKSPACE.  All calls on one GPU share that array: calls
 * that overlap on one GPU (other streams, other threads) race and must be
 * serialized by the caller.  Calls no hipMalloc/hipFree. */
#define BMX_K2B_DECODE_SCRATCH_BYTES (32u << 20)
int bmx_k2b_decode_noalloc(const bmx_k2b_decode_args* args, void* stream);

/* ------------------------------------------------------------------------
 * Quantize-on-append (page commit).  Replaces the write path of
 * PackedStreamingLayer.update (cache/packed_streaming.py:582-730):
 * _pack_k_block -> quantize_packed("lowrank_rtn_channel") (codecs.py:786-796,
 * 677-695; quant/rtn.py:23-44) and _pack_v_block -> quantize_packed(
 * "turboquant_mse_perhead") (codecs.py:616-636, 734-745).
 *
 * Encodes n_codec_pages consecutive 128-token codec pages into 8 physical
 * pages each.  Keys: Us = M * basis32 (or us_first for codec page 0 of a
 * sequence, the SVD factor of the first page), Us16 = fp16(Us),
 * R = M - Us16*basis16^T, per channel and 64-token group
 * scale = max|R|/3, code = clamp(rint(R/scale), -4, 3).  Values per
 * (token, head): n = fp16(||v||), x = fwht((v/n)*signs)*sqrt(128),
 * code = #{midpoints < x}.
 * ---------------------------------------------------------------------- */
typedef struct {
  bmx_k2b_geom geom;
  int32_t n_codec_pages;
  const uint16_t* k_pre;      /* device fp16 pre-RoPE keys: (h, t, j) at
                                 h*k_stride_h + t*k_stride_t + j, t in [0, 128*n) */
  int64_t k_stride_h;
  int64_t k_stride_t;
  const void* v;              /* device values, same indexing, element type v_dtype */
  int64_t v_stride_h;
  int64_t v_stride_t;
  const float* basis32;       /* device fp32 [C][R] frozen basis (projection), 16-byte aligned */
  const uint16_t* basis16;    /* device fp16 [C][R] (= fp16(basis32)) */
  const float* us_first;      /* device fp32 [128][R] or NULL: Us of codec page 0 */
  float codebook[4];
  uint32_t v_sign_bits[4];
  uint8_t* pages;             /* device page pool */
  int32_t n_pool_pages;       /* pages in the pool (ids are clamped into range) */
  const int32_t* page_ids;    /* device [n_codec_pages*8] physical page of each
                                 16-token page, in token order */
  int32_t v_dtype;            /* BMX_K2B_F16 (0), BMX_K2B_F32 or BMX_K2B_BF16: values are
                                 encoded from the model's own precision, as the
                                 reference's .float() of the value slab */
} bmx_k2b_append_args;

int bmx_k2b_append(const bmx_k2b_append_args* args, void* stream);

/* ------------------------------------------------------------------------
 * Dequantize committed pages of one sequence to dense keys and values
 * (prefill path and checks).  Replaces _dequant_block / _dense_kv and the
 * dtype cast of _assemble_dense_kv (cache/chunked_attention.py:52-251).
 * apply_rope: 0 = keys pre-RoPE; 1 = RoPE with fp32 cos/sin of the exact
 * angle; 2 = RoPE as the reference's prefill applies it (cache/
 * packed_streaming.py:79-113, chunked_attention.py:148-194): HF's fp32 angle
 * fl(inv_freq_j * pos), cos/sin times rope_scaling rounded to fp16, the
 * rotation x*cos + rotate_half(x)*sin in fp32.  The result is rounded once
 * to out_dtype.
 * ---------------------------------------------------------------------- */
typedef struct {
  bmx_k2b_geom geom;
  const uint8_t* pages;
  int32_t n_pool_pages;       /* pages in the pool (ids are clamped into range) */
  const int32_t* page_table;  /* device [n_tokens/16] logical -> physical page */
  int32_t n_tokens;           /* multiple of the residual group (64 on the recipe's page) */
  const uint16_t* basis;      /* device fp16 [C][R] */
  float inv_freq[64];
  float rope_scaling;
  int32_t apply_rope;
  float codebook[4];
  uint32_t v_sign_bits[4];
  void* k_out;                /* device [h_kv][out_rows][head_dim] of out_dtype: rows 0 .. n_tokens - 1 */
  void* v_out;                /* of each head written */
  int32_t out_dtype;          /* BMX_K2B_F16 (0), BMX_K2B_F32 or BMX_K2B_BF16 */
  int32_t pos0;               /* RoPE position of the first listed token (0: the sequence's start) */
  int64_t out_rows;           /* rows per head in k_out / v_out, >= n_tokens (0: n_tokens) */
} bmx_k2b_dequant_args;

int bmx_k2b_dequant(const bmx_k2b_dequant_args* args, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* BMX_K2B_H */
