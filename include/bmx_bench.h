// Dense fp16 decode attention: the comparator bench.py measures the packed
// path against (the packed decode has to beat a measured fp16 decode at the
// same context).  No counterpart in the reference, which compares against
// dense attention in PyTorch; this is the same computation written as a
// bandwidth kernel, so that the bar is the HBM rate of fp16 K/V, not the
// efficiency of a library GEMM at a decode shape.  Not used by the cache.
#ifndef BMX_BENCH_H
#define BMX_BENCH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BMX_BENCH_E_INVALID 1
#define BMX_BENCH_E_HIP 2

typedef struct bmx_fp16_decode_args {
  const void* q;        // [h_kv][n_q_groups][128] fp16
  const void* k;        // fp16 rows of 128: row t of head h at h * stride_h + t * stride_t (elements)
  const void* v;        // same layout as k
  int64_t stride_h, stride_t;
  int h_kv, n_q_groups;   // n_q_groups: 1, 2, 4 or 8
  int T;                  // tokens
  int n_split;            // workgroups per head
  float sm_scale;
  void* out;              // [h_kv][n_q_groups][128] fp16
  void* workspace;        // bmx_fp16_decode_workspace_bytes()
  size_t workspace_bytes;
} bmx_fp16_decode_args;

size_t bmx_fp16_decode_workspace_bytes(int h_kv, int n_q_groups, int n_split);
// 0, or BMX_BENCH_E_INVALID / BMX_BENCH_E_HIP
int bmx_fp16_decode(const bmx_fp16_decode_args* a, void* stream);

#ifdef __cplusplus
}
#endif

#endif
