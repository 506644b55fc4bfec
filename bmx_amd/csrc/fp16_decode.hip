// Dense fp16 split-KV decode attention on gfx950: the comparator the packed
// path is measured against (a decode step over fp16 K/V of every token, the
// bytes an fp16 KV cache reads).  Not a path of the packed cache.
//
// fp16_decode_split_kernel: grid (splits, h_kv), block 256 (4 waves).  The
// workgroup streams its head's token range in 64-token chunks, the next
// chunk's K and V rows loaded into registers while the current one is used:
//   * scores: thread (token i / 4, quarter i % 4) takes 32 channels of one
//     key row (64 contiguous bytes), dots them with the G queries (packed
//     fp16 dot products, fp32 sums) and the quarters meet by quad DPP;
//   * softmax: wave g takes query g's 64 scores (one per lane), online over
//     the chunks (running max and sum, base 2);
//   * P.V: thread (token lane i / 32, channel quad i % 32) takes tokens
//     lane + 8k of the chunk, 4 channels each (8 contiguous bytes), and sums
//     p * v in fp32; the 8 token lanes meet in LDS at the end.
// fp16_decode_merge_kernel: one workgroup per (head, query): the splits'
// partials by their softmax weights, 8 split lanes in parallel.
//
// Both are plain bandwidth kernels: every K and V byte is read once, with
// 16-byte (keys) and 8-byte (values) coalesced loads.

#include "bmx_bench.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <string>

namespace bmx {
namespace {

constexpr int kFdD = 128;          // head dim
constexpr int kFdChunk = 64;       // tokens per chunk
constexpr int kFdThreads = 256;
constexpr int kFdMaxG = 8;

typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t fd_u4 __attribute__((ext_vector_type(4)));
typedef uint32_t fd_u2 __attribute__((ext_vector_type(2)));

struct FdArgs {
  const uint16_t* q;      // [h_kv][G][128] fp16
  const uint16_t* k;      // [h_kv] rows of 128 fp16, row t of head h at h * sh + t * st
  const uint16_t* v;
  int64_t sh, st;
  int T, G, n_split, h_kv;
  float qscale;           // sm_scale * log2(e)
  float* part;            // [h_kv][G][n_split][2 + 128]: m, l, channel sums
};

__device__ __forceinline__ f16x2_t h2(uint32_t u) { return __builtin_bit_cast(f16x2_t, u); }

template <int G>
__global__ __launch_bounds__(kFdThreads) void fp16_decode_split_kernel(const FdArgs a) {
  const int split = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int n_chunks = (a.T + kFdChunk - 1) / kFdChunk;
  const int c0 = (int)((int64_t)split * n_chunks / a.n_split), c1 = (int)((int64_t)(split + 1) * n_chunks / a.n_split);
  __shared__ float s_sc[kFdMaxG][kFdChunk];
  __shared__ float s_p[kFdMaxG][kFdChunk];
  __shared__ float s_alpha[kFdMaxG];
  __shared__ float s_red[8][kFdMaxG][kFdD];   // the token lanes' channel sums at the end
  // scores: token tt, quarter qq (channels 32 qq .. + 31)
  const int tt = tid >> 2, qq = tid & 3;
  uint32_t qv[G][16];   // the queries' 32 channels of this quarter, fp16 pairs
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const uint4* src = reinterpret_cast<const uint4*>(a.q + ((int64_t)h * a.G + g) * kFdD + 32 * qq);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 w = src[i];
      qv[g][4 * i] = w.x; qv[g][4 * i + 1] = w.y; qv[g][4 * i + 2] = w.z; qv[g][4 * i + 3] = w.w;
    }
  }
  // P.V: token lane tl (tokens tl + 8 k), channel quad cq (channels 4 cq .. + 3)
  const int tl = tid >> 5, cq = tid & 31;
  const uint16_t* kh = a.k + (int64_t)h * a.sh;
  const uint16_t* vh = a.v + (int64_t)h * a.sh;
  auto load_k = [&](int c, uint4 kw[4]) {
    const int t = min(c * kFdChunk + tt, a.T - 1);
    const fd_u4* src = reinterpret_cast<const fd_u4*>(kh + (int64_t)t * a.st + 32 * qq);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const fd_u4 w = __builtin_nontemporal_load(src + i);
      kw[i] = make_uint4(w[0], w[1], w[2], w[3]);
    }
  };
  auto load_v = [&](int c, uint2 vw[8]) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int t = min(c * kFdChunk + tl + 8 * k, a.T - 1);
      const fd_u2 w = __builtin_nontemporal_load(reinterpret_cast<const fd_u2*>(vh + (int64_t)t * a.st + 4 * cq));
      vw[k] = make_uint2(w[0], w[1]);
    }
  };
  __shared__ float s_m[kFdMaxG], s_l[kFdMaxG];   // query g's running max and sum (base 2)
  if (tid < kFdMaxG) {
    s_m[tid] = -INFINITY;
    s_l[tid] = 0.f;
  }
  float acc[G][4];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[g][i] = 0.f;
  uint4 kw[4], kn[4];
  uint2 vw[8], vn[8];
  if (c0 < c1) {
    load_k(c0, kw);
    load_v(c0, vw);
  }
  for (int c = c0; c < c1; ++c) {
    if (c + 1 < c1) {   // the next chunk in flight while this one is used
      load_k(c + 1, kn);
      load_v(c + 1, vn);
    }
    const int t_tok = c * kFdChunk + tt;
    // ---- scores of this thread's token for every query
    float sc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t w4[4] = {kw[i].x, kw[i].y, kw[i].z, kw[i].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) s = __builtin_amdgcn_fdot2(h2(w4[e]), h2(qv[g][4 * i + e]), s, false);
      }
      // the four quarters of the token (lanes 4tt .. 4tt + 3 of a row of 16)
      s += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, s), 0xB1, 0xF, 0xF, true));
      s += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, s), 0x4E, 0xF, 0xF, true));
      sc[g] = t_tok < a.T ? s * a.qscale : -INFINITY;
    }
    if (qq == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g) s_sc[g][tt] = sc[g];
    }
    __syncthreads();
    // ---- online softmax: wave g % 4 takes query g, lane = token
    for (int g = wave; g < G; g += 4) {
      const float x = s_sc[g][lane];
      float mx = x;
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
      const float m_old = s_m[g];
      const float m_new = fmaxf(m_old, mx);
      const float alpha = m_old == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_old - m_new);
      const float p = x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(x - m_new);
      float ps = p;
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) ps += __shfl_xor(ps, o);
      s_p[g][lane] = p;
      if (lane == 0) {
        s_alpha[g] = alpha;
        s_m[g] = m_new;
        s_l[g] = __builtin_fmaf(s_l[g], alpha, ps);
      }
    }
    __syncthreads();
    // ---- P.V over the chunk
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float al = s_alpha[g];
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[g][i] *= al;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const f16x2_t v01 = h2(vw[k].x), v23 = h2(vw[k].y);
      const float v4[4] = {(float)v01[0], (float)v01[1], (float)v23[0], (float)v23[1]};
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float p = s_p[g][tl + 8 * k];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[g][i] = __builtin_fmaf(p, v4[i], acc[g][i]);
      }
    }
    if (c + 1 < c1) {
#pragma unroll
      for (int i = 0; i < 4; ++i) kw[i] = kn[i];
#pragma unroll
      for (int k = 0; k < 8; ++k) vw[k] = vn[k];
    }
    __syncthreads();   // s_sc / s_p / s_alpha reused by the next chunk
  }
  // ---- the token lanes meet; (m, l) from their waves
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int i = 0; i < 4; ++i) s_red[tl][g][4 * cq + i] = acc[g][i];
  __syncthreads();
  for (int e = tid; e < G * kFdD; e += kFdThreads) {
    const int g = e / kFdD, ch = e % kFdD;
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) s += s_red[j][g][ch];
    a.part[(((int64_t)h * a.G + g) * a.n_split + split) * (2 + kFdD) + 2 + ch] = s;
  }
  if (tid < G) {
    float* dst = a.part + (((int64_t)h * a.G + tid) * a.n_split + split) * (2 + kFdD);
    dst[0] = s_m[tid];
    dst[1] = s_l[tid];
  }
}

struct FdMergeArgs {
  const float* part;
  int n_split, G;
  uint16_t* out;   // [h_kv][G][128] fp16
};

// block 256: thread (split lane sl = tid / 32, channel quad cq = tid % 32)
// takes splits sl, sl + 8, ... for channels 4 cq .. + 3, online; the 8 split
// lanes meet in LDS.
__global__ __launch_bounds__(256) void fp16_decode_merge_kernel(const FdMergeArgs a) {
  const int row = blockIdx.x, tid = threadIdx.x, sl = tid >> 5, cq = tid & 31;
  const float* base = a.part + (int64_t)row * a.n_split * (2 + kFdD);
  __shared__ float s_m[8], s_l[8];
  __shared__ float4 s_x[8][32];
  float m = -INFINITY, l = 0.f;
  float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int sp = sl; sp < a.n_split; sp += 8) {
    const float* p = base + (int64_t)sp * (2 + kFdD);
    const float ms = p[0];
    if (ms == -INFINITY) continue;
    const float4 v = *reinterpret_cast<const float4*>(p + 2 + 4 * cq);
    const float mn = fmaxf(m, ms);
    const float al = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mn), w = __builtin_amdgcn_exp2f(ms - mn);
    l = l * al + w * p[1];
    x = make_float4(x.x * al + w * v.x, x.y * al + w * v.y, x.z * al + w * v.z, x.w * al + w * v.w);
    m = mn;
  }
  if (cq == 0) {
    s_m[sl] = m;
    s_l[sl] = l;
  }
  s_x[sl][cq] = x;
  __syncthreads();
  if (tid < 32) {
    float M = -INFINITY;
#pragma unroll
    for (int j = 0; j < 8; ++j) M = fmaxf(M, s_m[j]);
    float den = 0.f;
    float4 num = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float w = s_m[j] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s_m[j] - M);
      den = __builtin_fmaf(w, s_l[j], den);
      const float4 v = s_x[j][tid];
      num = make_float4(num.x + w * v.x, num.y + w * v.y, num.z + w * v.z, num.w + w * v.w);
    }
    const float inv = den > 0.f ? 1.0f / den : 0.f;
    const _Float16 o[4] = {(_Float16)(num.x * inv), (_Float16)(num.y * inv), (_Float16)(num.z * inv),
                           (_Float16)(num.w * inv)};
    uint2 w2;
    __builtin_memcpy(&w2, o, 8);
    *reinterpret_cast<uint2*>(a.out + (int64_t)row * kFdD + 4 * tid) = w2;
  }
}

}  // namespace
}  // namespace bmx

using namespace bmx;

extern "C" size_t bmx_fp16_decode_workspace_bytes(int h_kv, int n_q_groups, int n_split) {
  if (h_kv < 1 || n_q_groups < 1 || n_split < 1) return 0;
  return (size_t)h_kv * n_q_groups * n_split * (2 + kFdD) * sizeof(float);
}

extern "C" int bmx_fp16_decode(const bmx_fp16_decode_args* a, void* stream) {
  if (!a || !a->q || !a->k || !a->v || !a->out || !a->workspace) return BMX_BENCH_E_INVALID;
  if (a->h_kv < 1 || a->n_q_groups < 1 || a->n_q_groups > kFdMaxG || a->T < 1 || a->n_split < 1 ||
      a->stride_t < kFdD || a->stride_t % 8 != 0 || a->stride_h % 8 != 0)
    return BMX_BENCH_E_INVALID;
  if (a->workspace_bytes < bmx_fp16_decode_workspace_bytes(a->h_kv, a->n_q_groups, a->n_split))
    return BMX_BENCH_E_INVALID;
  FdArgs k{};
  k.q = static_cast<const uint16_t*>(a->q);
  k.k = static_cast<const uint16_t*>(a->k);
  k.v = static_cast<const uint16_t*>(a->v);
  k.sh = a->stride_h;
  k.st = a->stride_t;
  k.T = a->T;
  k.G = a->n_q_groups;
  k.n_split = a->n_split;
  k.h_kv = a->h_kv;
  k.qscale = a->sm_scale * 1.4426950408889634f;
  k.part = static_cast<float*>(a->workspace);
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid(a->n_split, a->h_kv);
  switch (a->n_q_groups) {
    case 1: hipLaunchKernelGGL(fp16_decode_split_kernel<1>, grid, dim3(kFdThreads), 0, st, k); break;
    case 2: hipLaunchKernelGGL(fp16_decode_split_kernel<2>, grid, dim3(kFdThreads), 0, st, k); break;
    case 4: hipLaunchKernelGGL(fp16_decode_split_kernel<4>, grid, dim3(kFdThreads), 0, st, k); break;
    case 8: hipLaunchKernelGGL(fp16_decode_split_kernel<8>, grid, dim3(kFdThreads), 0, st, k); break;
    default: return BMX_BENCH_E_INVALID;
  }
  if (hipGetLastError() != hipSuccess) return BMX_BENCH_E_HIP;
  FdMergeArgs m{};
  m.part = k.part;
  m.n_split = a->n_split;
  m.G = a->n_q_groups;
  m.out = static_cast<uint16_t*>(a->out);
  hipLaunchKernelGGL(fp16_decode_merge_kernel, dim3(a->h_kv * a->n_q_groups), dim3(256), 0, st, m);
  return hipGetLastError() == hipSuccess ? 0 : BMX_BENCH_E_HIP;
}
