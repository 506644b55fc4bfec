// Prefill attention over dense K/V rows (gfx950, MFMA flash attention).
//
// Replaces the attention call of the reference's prefill path:
// _prefill_dense_attention (src/bmx/cache/chunked_attention.py:320-395)
// dequantizes every committed page to dense rows, appends the fp16 window and
// hands q, K and V to torch's scaled_dot_product_attention with the model's
// mask.  The page dequant is bmx_k2b_dequant / bmx_rtn_dequant /
// bmx_spectral_dequant; this is the attention that follows it, for the masks
// a cached prefill carries: the causal mask of the last n_q positions over
// n_kv keys (bottom-right aligned; n_q == n_kv is the plain causal mask), or
// no mask.  Grouped-query heads read their K/V head in place (no expansion).
#ifndef BMX_PREFILL_H
#define BMX_PREFILL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BMX_PREFILL_F16 0
#define BMX_PREFILL_BF16 1

#define BMX_PREFILL_E_INVALID 1
#define BMX_PREFILL_E_HIP 2

typedef struct bmx_prefill_args {
  // query head hq (= kv head h * n_q_groups + g), position i: 128 contiguous
  // elements at q + hq * q_stride_h + i * q_stride_t
  const void* q;
  int64_t q_stride_h, q_stride_t;
  // key / value rows of kv head h, position j: 128 contiguous elements at
  // k + h * kv_stride_h + j * kv_stride_t (v the same)
  const void* k;
  const void* v;
  int64_t kv_stride_h, kv_stride_t;
  void* out;              // [h_kv * n_q_groups][n_q][128], contiguous
  int h_kv, n_q_groups, n_q, n_kv;
  int head_dim;           // 128
  int dtype;              // BMX_PREFILL_F16 / _BF16: q, k, v and out
  int causal;             // 1: query i sees keys j <= i + n_kv - n_q (needs n_q <= n_kv); 0: every key
  float sm_scale;
  int n_split;            // key ranges per row tile (1..16), 0: chosen by the library
  void* workspace;        // bmx_prefill_workspace_bytes(); may be NULL when that is 0
  size_t workspace_bytes;
} bmx_prefill_args;

// Device scratch the call needs (split partials), for the n_split it will
// use; 0 when one key range covers the rows (no partials).
size_t bmx_prefill_workspace_bytes(const bmx_prefill_args* a);
// 0, or BMX_PREFILL_E_INVALID / BMX_PREFILL_E_HIP with bmx_last_error() set
int bmx_prefill(const bmx_prefill_args* a, void* stream);

#ifdef __cplusplus
}
#endif

#endif
