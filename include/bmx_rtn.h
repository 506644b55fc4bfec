/*
 * bmx_rtn.h — C-ABI of the MI355X (gfx950) packed-KV RTN decode path.
 *
 * Drop-in boundary for pherber3/bmx's fused RTN path: rtn_token keys
 * (post-RoPE) and rtn_token values, int codes times a per-(token, channel
 * group) fp16 scale.  Keys may also be rtn_channel (a per-(channel, token
 * group) scale: config 1 and KIVI, which the reference runs on its chunked
 * path only, cache/codecs.py:723-725).  Same conventions as bmx_k2b.h (shared
 * error channel bmx_last_error(), BMX_* codes, asynchronous calls that never
 * allocate).
 *
 * Replaces, in cache/triton_dequant_attention.py:
 *   fused_decode_attention_packed + _fused_decode_packed_kernel (:580-832)
 *   build_kv_stacked_packed (:1390-1451): the device stacks become a page pool
 *   _finalize_decode / _tail_partial / _fused_merge_kernel (:324-575)
 * and at page commit quantize_packed("rtn_token") (cache/codecs.py:720-722,
 * quant/rtn.py:23-44) for both keys and values.
 *
 * Page format "rtn" (PT = 16 tokens, head_dim 128, h_kv heads; little-endian;
 * codes are 4-bit offset binary, code + 8, for 2..4-bit RTN; gk, gv = group
 * of the key / value scales, 32, 64 or 128: channels, or tokens for
 * rtn_channel keys).  Sections, in this order:
 *   KSCALE [h_kv][16 t][128/gk] fp16   rtn_token: key scale of (token t, group)
 *          [2][h_kv][4 b][4 q][8 j] fp16  rtn_channel: scale of channel 32b + 8q +
 *                                      p(j), p = 0 4 1 5 2 6 3 7, for the token
 *                                      group that holds the page, as the pair
 *                                      hi = fp16(s) ([0]), lo = fp16(s - hi) ([1]):
 *                                      hi + lo is the fp32 scale to 2^-21
 *                                      relative (scales of 1/8 and up)
 *   VSCALE [h_kv][4 q][128/gv][4 i] fp16  value scale of (token 4q + i, group)
 *   KCODE  [h_kv][4 q][16 n][4 w] u32  token n, channels 32w + 8q .. +7, channel
 *                                      32w + 8q + j in nibble j of the word
 *   VCODE  [h_kv][4 q][16 c][8 b] u16  channel 16b + c, tokens 4q .. 4q + 3,
 *                                      token 4q + j in nibble j
 * ("lane 16q + n" of an MFMA reads each 16-byte code slice contiguously; the
 * two scale sections come first so that a workgroup stages them with one
 * cooperative copy.)  Bytes per token = h_kv * (128 + 2 * 128/gk + 2 * 128/gv)
 * for rtn_token keys (1152 at h_kv 8, gk = gv = 32), h_kv * (160 + 2 * 128/gv)
 * for rtn_channel keys (1344; the group's channel scale pairs repeated in each
 * of its pages).
 */
#ifndef BMX_RTN_H
#define BMX_RTN_H

#include <stddef.h>
#include <stdint.h>

#include "bmx_k2b.h"

#ifdef __cplusplus
extern "C" {
#endif

#define BMX_RTN_TOKEN 0     /* scale per (token, group of k_group channels) */
#define BMX_RTN_CHANNEL 1   /* scale per (channel, group of k_group tokens) */

typedef struct {
  int32_t h_kv;        /* KV heads: 1..8 for decode, 1..16 for append/dequant */
  int32_t n_q_groups;  /* query heads per KV head G, 1..16 */
  int32_t k_bits;      /* RTN bits of the keys, 2..4 */
  int32_t v_bits;      /* RTN bits of the values, 2..4 */
  int32_t k_group;     /* key scale group: 32, 64 or 128 channels (token arm) or tokens (channel arm) */
  int32_t v_group;     /* value scale group along head_dim: 32, 64 or 128 */
  int32_t k_arm;       /* BMX_RTN_TOKEN or BMX_RTN_CHANNEL */
} bmx_rtn_geom;

/* Bytes of one 16-token page (0 if the geometry is unsupported). */
size_t bmx_rtn_page_bytes(const bmx_rtn_geom* geom);

/* ------------------------------------------------------------------------
 * Quantize-on-append.  Replaces quantize_packed("rtn_token") of
 * PackedStreamingLayer.update for both sides (cache/packed_streaming.py:
 * 640-667 with K post-RoPE, 544-580), or quantize_packed("rtn_channel") for
 * the keys (codecs.py:723-725: groups of k_group tokens per channel): per
 * group scale = max|x| (clamped to 1e-12) / qmax in fp32, code =
 * clamp(round-half-even(x / scale), -qmax - 1, qmax), qmax = 2^(bits-1) - 1;
 * the page keeps a token-arm scale in fp16, as build_kv_stacked_packed stacks
 * it for the reference's fused pair, and a channel-arm scale as an fp16 (hi,
 * lo) pair, since the reference reads that arm with its fp32 scale
 * (dequant_packed, codecs.py:819-822).
 * n_codec_pages pages of 128 tokens become 8 * n_codec_pages physical pages
 * listed in page_ids.
 * ---------------------------------------------------------------------- */
typedef struct {
  bmx_rtn_geom geom;
  int32_t n_codec_pages;
  const void* k;              /* device [h_kv] x [128 * n_codec_pages] x [128] post-RoPE keys */
  int64_t k_stride_h;         /* element strides (dim 128 contiguous) */
  int64_t k_stride_t;
  int32_t k_dtype;            /* BMX_K2B_F16 / _F32 / _BF16 */
  const void* v;              /* device values, same shape */
  int64_t v_stride_h;
  int64_t v_stride_t;
  int32_t v_dtype;
  uint8_t* pages;             /* device page pool */
  const int32_t* page_ids;    /* device [8 * n_codec_pages] physical page ids, in order */
  int32_t n_pool_pages;
} bmx_rtn_append_args;

int bmx_rtn_append(const bmx_rtn_append_args* args, void* stream);

/* ------------------------------------------------------------------------
 * Decode attention.  Replaces fused_decode_attention_packed + _finalize_decode
 * (cache/triton_dequant_attention.py:731-832, 504-575): one query step per
 * sequence attends to its packed_len[b] committed tokens (keys and values
 * dequantized in-kernel, code * the page's scale) and to its tail_len[b] fp16
 * recent-window tokens, one base-e softmax over their union.  The fields
 * mean what they mean in bmx_k2b_decode_args.
 * ---------------------------------------------------------------------- */
typedef struct {
  bmx_rtn_geom geom;
  int32_t batch;
  const void* q;              /* device [batch][h_kv][G][128] post-RoPE, in io_dtype */
  void* out;                  /* device [batch][h_kv][G][128] in io_dtype */
  const uint8_t* pages;
  int32_t n_pool_pages;
  const int32_t* page_table;  /* device [batch][max_pages] */
  int32_t max_pages;
  const int32_t* packed_len;  /* device [batch], multiples of 128 */
  int32_t max_packed_len;
  float sm_scale;
  const uint16_t* k_tail;     /* device fp16 (tail_dtype) post-RoPE recent-window keys */
  const uint16_t* v_tail;
  int64_t tail_stride_b;
  int64_t tail_stride_h;
  int64_t tail_stride_t;
  const int32_t* tail_len;    /* device [batch], or NULL: tail_len_value for every sequence */
  int32_t tail_cap;           /* 0..4096 */
  int32_t split_tokens;       /* 0 = one workgroup per CU (default) */
  void* workspace;            /* device scratch: split partials and window scores */
  size_t workspace_bytes;
  int32_t tail_len_value;     /* as in bmx_k2b_decode_args: the host window length, and */
  const uint16_t* new_k;      /* the window's newest n_new rows given apart, attended */
  const uint16_t* new_v;      /* from here and copied into k_tail / v_tail */
  int64_t new_stride_b;
  int64_t new_stride_h;
  int64_t new_stride_t;
  int32_t n_new;
  int32_t io_dtype;           /* BMX_K2B_IO_F32 (0), _F16 or _BF16: the dtype of q and out */
  int32_t tail_dtype;         /* BMX_K2B_TAIL_F16 (0) or _BF16: the window rows' dtype */
} bmx_rtn_decode_args;

size_t bmx_rtn_decode_workspace_bytes(const bmx_rtn_decode_args* args);
int bmx_rtn_decode(const bmx_rtn_decode_args* args, void* stream);

/* ------------------------------------------------------------------------
 * Dequantize pages to dense keys and values (prefill): the dequant half of
 * chunked_attention._dense_kv and the dtype cast of _assemble_dense_kv
 * (cache/chunked_attention.py:148-251) for the RTN arms (code * the page's scale,
 * rounded once to out_dtype).  k_out/v_out: device [h_kv][out_rows][128],
 * rows 0 .. 16 * n_pages - 1 of each head written.
 * ---------------------------------------------------------------------- */
typedef struct {
  bmx_rtn_geom geom;
  const uint8_t* pages;
  int32_t n_pool_pages;
  const int32_t* page_ids;    /* device [n_pages] */
  int32_t n_pages;
  void* k_out;
  void* v_out;
  int32_t out_dtype;          /* BMX_K2B_F16 (0), BMX_K2B_F32 or BMX_K2B_BF16 */
  int64_t out_rows;           /* rows per head in k_out / v_out, >= 16 * n_pages (0: 16 * n_pages) */
} bmx_rtn_dequant_args;

int bmx_rtn_dequant(const bmx_rtn_dequant_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BMX_RTN_H */
