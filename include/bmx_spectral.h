/* C-ABI of the spectral (K4) key path on gfx950: the write kernels and the
 * dense dequantization a decode or prefill step attends over.
 *
 * Keys: a corpus-fitted spectral pack (enc, dec: C x C fp32; bits per
 * direction from the tier grid {0, 2, 3, 4, 5, 6, 8}; group 64 tokens) codes
 * the pre-RoPE keys as Y = M enc, RTN per direction over 64-token groups with
 * the MSE-refined step, and reads them back as Y_hat dec^T with RoPE applied
 * at read.  Reference: src/bmx/cache/spectral.py:763-841
 * (spectral_quantize_packed / spectral_dequant_packed), quant/rtn.py:10-53,
 * the write call in cache/packed_streaming.py:491-511 and the read in
 * cache/chunked_attention.py:106-116 (_dequant_block, arm "spectral"), whose
 * decode is the reference's chunked path (packed_streaming.py:1016-1032).
 * Values, v_codec BMX_SPECTRAL_V_PERHEAD: the k2b value codec (2-bit Lloyd
 * codes of the Hadamard-rotated values and an fp16 norm per head and token,
 * include/bmx_k2b.h, the reference's turboquant_mse_perhead) in value-only
 * pages of 16 tokens: VNORM [h_kv][16] fp16 at byte 0, VCODE [h_kv][64][2] u32
 * at byte 32 h_kv, bmx_spectral_v_page_bytes(h_kv) bytes per page.
 * v_codec BMX_SPECTRAL_V_FULL: the reference's full-C turboquant_mse
 * (codecs.py:616-675 at h = 1: one fp16 norm per token over all C channels,
 * one C-point randomized Hadamard, 2-bit codes of the C rotated channels;
 * C = 128 h_kv must be a power of two, h_kv 1, 2, 4 or 8): VNORM [16] fp16
 * at byte 0, VCODE [C / 128][64][2] u32 at byte 32, slice s holding rotated
 * channels 128 s .. 128 s + 127 in the per-head layout;
 * bmx_spectral_v_page_bytes_codec(h_kv, v_codec) bytes per page.  The norm
 * sums the squares in 8 strided fp32 FMA accumulators, then those left to
 * right (torch's CPU order for these rows).
 *
 * Key page: one per 64-token group.  Columns are the pack's coded directions
 * in tier order (tier ascending, direction ascending), each tier padded with
 * zero directions to a multiple of 8: c_pad columns.  SCALE [c_pad] fp16 at
 * byte 0 holds the group's step of each column; then slices of 8 columns,
 * slice s at byte offset off[s] = slice_tab[s] & 0xFFFFFF with tier
 * b = slice_tab[s] >> 24, container width w = 2 (b = 2), 4 (b = 3, 4) or
 * 8 (b = 5, 6, 8) bits: token t's 8 codes in the w bytes at off[s] + t w,
 * column k at bits [k w, (k + 1) w), stored as code + 2^(b - 1).  16 bytes of
 * padding end the page.  Codes and steps are computed in fp32 in a fixed
 * order: Y[t][j] = sum over c ascending of M[t][c] enc[c][j] and the step's
 * sums over the group's tokens left to right, no fused multiply-add.
 *
 * Lloyd payload (the reference's payload_quant "lloyd", recipe suffix "_lq":
 * spectral.py:648-700 _lloyd_quantize_packed / _lloyd_dequantize_packed):
 * with L.lloyd_levels set, a column of tier b codes its group against the
 * 2^b sorted levels of gaussian_codebook(b): the step starts at the sample
 * standard deviation of the group's 64 values (mean and squared deviations
 * summed left to right in fp64, divided by 64 and 63, square root, rounded to
 * fp32; at least 1e-12), the code of a value is the number of midpoints
 * (l_i + l_{i+1}) / 2 below value / step, and 3 rounds of step = <Y, l_code>
 * / <l_code, l_code> (fp32, left to right, both at least 1e-12) refit it
 * before the final codes.  The stored value is the level index itself
 * (0 .. 2^b - 1, no offset) and the key reads back as level * step.
 *
 * Every entry point returns BMX_OK (0) or a BMX_E_* code with a message from
 * bmx_last_error() (include/bmx_k2b.h). */
#ifndef BMX_SPECTRAL_H
#define BMX_SPECTRAL_H

#include <stdint.h>

#include "bmx_k2b.h"

#ifdef __cplusplus
extern "C" {
#endif

#define BMX_SPECTRAL_MAX_CPAD 1072   /* 1024 directions + padding of 6 tiers */
#define BMX_SPECTRAL_LLOYD_LEVELS 380 /* levels of tiers 2, 3, 4, 5, 6, 8 back to back */
#define BMX_SPECTRAL_V_PERHEAD 0      /* values: turboquant_mse_perhead (one Hadamard per head) */
#define BMX_SPECTRAL_V_FULL 1         /* values: turboquant_mse (one Hadamard over all C channels) */

typedef struct bmx_spectral_layout {
  int32_t h_kv;                /* key heads, 1..8; C = 128 h_kv */
  int32_t c_pad;               /* coded columns with padding: multiple of 8, 8..C + 48 */
  int32_t k_page_bytes;        /* bytes per key page (SCALE + slices + 16) */
  const int32_t* slice_tab;    /* device, c_pad / 8 entries: off | tier << 24 */
  const float* lloyd_levels;   /* NULL: the rtn payload.  Else the Lloyd payload's levels,
                                  device fp32 [BMX_SPECTRAL_LLOYD_LEVELS]: gaussian_codebook(b)
                                  of tier b at offset 2^b - 4 (b <= 6) and 124 (b = 8) */
} bmx_spectral_layout;

/* Replaces the spectral branch of PackedStreamingLayer._pack_k_block
 * (packed_streaming.py:491-511: spectral_quantize_packed on the block's
 * pre-RoPE keys) and its _pack_v_block for the paired turboquant_mse values
 * (packed_streaming.py:544-580), for n_groups 64-token groups at once. */
typedef struct bmx_spectral_append_args {
  bmx_spectral_layout L;
  int32_t n_groups;            /* 64-token groups to write */
  const void* k_pre;           /* pre-RoPE keys, element [h][t][d] at h k_sh + t k_st + d */
  int32_t k_dtype;             /* BMX_K2B_F16, _F32 or _BF16 (converted to fp32) */
  int64_t k_sh, k_st;
  const void* v;               /* values, element [h][t][d] at h v_sh + t v_st + d */
  int32_t v_dtype;
  int64_t v_sh, v_st;
  const float* enc_perm;       /* device [C][c_pad] fp32: enc's columns in page order, zero padding */
  uint8_t* k_pages;            /* key page pool */
  const int32_t* k_page_ids;   /* n_groups ids */
  int32_t n_k_pool;
  uint8_t* v_pages;            /* value page pool */
  const int32_t* v_page_ids;   /* 4 n_groups ids (16 tokens each) */
  int32_t n_v_pool;
  float v_codebook[4];         /* 2-bit Lloyd levels (gaussian_codebook(2)) */
  uint32_t v_sign_bits[4];     /* Hadamard signs of the 128 channels (1 = negative) */
  int32_t v_codec;             /* BMX_SPECTRAL_V_PERHEAD or BMX_SPECTRAL_V_FULL */
  uint32_t v_sign_bits_c[32];  /* V_FULL: signs of the C channels, bit c % 32 of word c / 32 */
} bmx_spectral_append_args;

/* Replaces _dequant_block(arm "spectral") + apply_rope for the keys and
 * _dequant_block(arm "turboquant_mse") for the values (chunked_attention.py:
 * 52-194), n_tokens tokens of one sequence into dense [h_kv][n_tokens][128]. */
typedef struct bmx_spectral_dequant_args {
  bmx_spectral_layout L;
  int32_t n_tokens;            /* multiple of 64 */
  const uint8_t* k_pages;
  const int32_t* k_page_table; /* n_tokens / 64 key page ids */
  int32_t n_k_pool;
  const uint8_t* v_pages;
  const int32_t* v_page_table; /* n_tokens / 16 value page ids */
  int32_t n_v_pool;
  const uint16_t* dec_perm;    /* device fp16 dec, rows of each head, columns in page order
                                  with zero padding to c_pad32 = c_pad rounded up to 32,
                                  tiled [h_kv][c_pad32 / 32][8][16][32]: element (row
                                  16 i + r, column 32 k + c) of head h at
                                  (((h c_pad32 / 32 + k) 8 + i) 16 + r) 32 + c */
  int32_t apply_rope;          /* 0 none, 1 fp32 cos/sin, 2 cos/sin rounded to fp16 */
  float rope_scaling;
  float inv_freq[64];
  float v_codebook[4];
  uint32_t v_sign_bits[4];
  int32_t out_dtype;           /* BMX_K2B_F16, _F32 or _BF16 */
  void* k_out;                 /* [h_kv][out_rows][128]: rows 0 .. n_tokens - 1 of each head written */
  void* v_out;
  int32_t out_rows;            /* rows per head in k_out / v_out / scores, >= n_tokens (0: n_tokens);
                                  the rows after n_tokens are left for the caller (the recent window) */
  /* Decode form: with q set, the kernel also scores the rotated keys against
   * the step's queries, scores[h][g][t] = q[h][g] . k_rot[h][t] (fp32
   * accumulation of fp16 keys and queries, no softmax scale), for rows
   * 0 .. n_tokens - 1; k_out may then be NULL (no dense keys written).
   * Requires apply_rope != 0. */
  const void* q;               /* [h_kv][n_q_groups][128], dtype q_dtype, or NULL */
  int32_t q_dtype;             /* BMX_K2B_F16, _F32 or _BF16 */
  int32_t n_q_groups;          /* 1..16 */
  float* scores;               /* [h_kv][n_q_groups][out_rows] fp32 */
  /* Partial form (with q): instead of scores and values, each 64-token group's
   * or 128-token block's softmax partial per (head, query), in the rows
   * r = h G + g of 130 n_parts floats each: at r 130 n_parts + 2p, partial
   * p's m = max of the scaled scores and l = sum of exp(s - m) (the fp16
   * weights); at r 130 n_parts + 2 n_parts + 16 (k n_parts + p) + j, its
   * channel c = 16k + j: channel c of the Hadamard over the channel index's
   * bits 4..6 (unnormalized, pairs (a, b) -> (a + b, a - b); H8 over k) of
   * the rotated-domain sums of the weights times the token norms times the
   * codebook levels (fp32 accumulation of fp16 operands): the values are the
   * merged sums' Hadamard over bits 0..3 (H16 over j), the codec's signs and
   * 1/128;
   * n_parts = bmx_spectral_partial_count(args): one partial per 128-token
   * block when the two key pages of a block fit in LDS together
   * (2 k_page_bytes <= 57344), apply_rope is 2 and n_tokens a multiple of
   * 128, else one per 64-token group.  The caller merges the partials
   * (m = max m_i, l = sum l_i e^(m_i - m), out = signs * H16(sum acc_i
   * e^(m_i - m)) / (128 l)) with the window's.  v_out and scores may then be
   * NULL. */
  float* partials;
  float sm_scale;
  int32_t v_codec;             /* BMX_SPECTRAL_V_PERHEAD or BMX_SPECTRAL_V_FULL: with V_FULL the
                                  partials' sums are over the tokens' C-wide codes combined by
                                  H_{C/128} (row h: sign (-1)^popcount(h & s) for slice s), so that
                                  the merge's H16, signs and scale give head h's values */
  uint32_t v_sign_bits_c[32];  /* V_FULL: signs of the C channels */
} bmx_spectral_dequant_args;

/* The decode step's merge: the groups' softmax partials (the partial form
 * above) and the fp16 recent window's tokens, scored here, folded by the split
 * softmax's weights (m = max, weights e^(m_i - m)) into the attention output.
 * Replaces the online-softmax reassembly of chunked_dequant_attention
 * (chunked_attention.py:398-530) and the merge of _finalize_decode
 * (triton_dequant_attention.py:504-575) for the spectral step. */
typedef struct bmx_spectral_merge_args {
  int32_t h_kv, n_q_groups;    /* 1..8, 1..16 */
  int32_t n_groups;            /* groups in partials, 0..16384 (0: window only) */
  const float* partials;       /* [h_kv][n_q_groups][n_groups][130] fp32 */
  const void* q;               /* [h_kv][n_q_groups][128] post-RoPE, dtype q_dtype */
  int32_t q_dtype;
  const uint16_t* k_win;       /* fp16 (win_dtype) post-RoPE window keys, row t of head h at h win_stride_h + 128 t,
                                  16-byte aligned */
  const uint16_t* v_win;       /* fp16 (win_dtype) window values, same indexing */
  int32_t win_len;             /* 0..4096 */
  float sm_scale;
  void* out;                   /* [h_kv][n_q_groups][128], dtype out_dtype */
  int32_t out_dtype;
  uint32_t v_sign_bits[4];     /* the value codec's signs, applied to the partials' sums */
  int64_t win_stride_h;        /* elements between heads in k_win / v_win (0: 128 win_len) */
  int32_t v_codec;             /* BMX_SPECTRAL_V_PERHEAD (signs v_sign_bits, scale 1/128) or
                                  BMX_SPECTRAL_V_FULL (head h: signs 128 h .. of v_sign_bits_c,
                                  scale 1/C) */
  uint32_t v_sign_bits_c[32];
  int32_t win_dtype;           /* BMX_K2B_TAIL_F16 (0) or _BF16: the dtype of k_win and v_win */
} bmx_spectral_merge_args;

int64_t bmx_spectral_v_page_bytes(int32_t h_kv);
/* Value page bytes of either value codec, or -1 (V_FULL needs h_kv 1, 2, 4 or 8). */
int64_t bmx_spectral_v_page_bytes_codec(int32_t h_kv, int32_t v_codec);
int32_t bmx_spectral_merge(const bmx_spectral_merge_args* a, void* stream);
int32_t bmx_spectral_append(const bmx_spectral_append_args* a, void* stream);
int32_t bmx_spectral_dequant(const bmx_spectral_dequant_args* a, void* stream);
/* Partials per (head, query) row that the partial form of these arguments
 * writes, or -1; partials itself may still be NULL when this is asked. */
int32_t bmx_spectral_partial_count(const bmx_spectral_dequant_args* a);

#ifdef __cplusplus
}
#endif

#endif /* BMX_SPECTRAL_H */
