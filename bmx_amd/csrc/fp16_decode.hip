// Dense fp16 split-KV decode attention on gfx950: the comparator the packed
// path is measured against (a decode step over fp16 K/V of every token, the
// bytes an fp16 KV cache reads).  Not a path of the packed cache.
//
// fp16_decode_split_kernel: grid (splits, h_kv), block 256 (4 waves).  The
// workgroup's token range is cut into 32-token chunks and wave w takes
// tokens 8 w .. 8 w + 7 of each chunk (one "step").  Inside a wave, lane
// (row r = lane / 16, channel octet c = lane % 16) holds channels 8 c .. +7
// of tokens r and r + 4 of the step, for K and for V (16-byte loads; a
// 16-lane row reads 256 contiguous bytes).  The 4 rows are 4 independent
// online-softmax streams (token residue mod 4), so the loop has no exchange
// between rows or waves:
//   * scores: packed fp16 dot products over the lane's 8 channels, summed
//     over the row's 16 lanes by DPP (every lane of the row gets the sum);
//   * softmax: running max and sum per (row, query), base 2;
//   * P.V: the lane's own 8 channels of its tokens, fp32.
// Loads run NB - 1 steps ahead in a register ring of NB steps, so 12-20 KB
// per wave is in flight without any LDS.  The 16 streams of the workgroup
// meet in LDS at the end and leave one partial per (query, split).
// fp16_decode_merge_kernel: one workgroup per (head, query): the splits'
// partials by their softmax weights, 8 split lanes in parallel.
//
// Both are plain bandwidth kernels: every K and V byte is read once.

#include "bmx_bench.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <string>

namespace bmx {
namespace {

constexpr int kFdD = 128;          // head dim
constexpr int kFdChunk = 64;       // bound on the tokens of a workgroup step (offset checks)
constexpr int kFdThreads = 256;
constexpr int kFdMaxG = 8;
constexpr int kFdBufWord3 = 0x00020000;   // raw buffer descriptor, word 3

typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t fd_u4 __attribute__((ext_vector_type(4)));

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

template <int Ctrl>
__device__ __forceinline__ float dpp_mov(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), Ctrl, 0xF, 0xF, true));
}

// sum over the 16 lanes of a DPP row; every lane of the row gets it
__device__ __forceinline__ float row16_sum(float s) {
  s += dpp_mov<0xB1>(s);    // quad_perm [1,0,3,2]
  s += dpp_mov<0x4E>(s);    // quad_perm [2,3,0,1]
  s += dpp_mov<0x124>(s);   // row_ror 4
  s += dpp_mov<0x128>(s);   // row_ror 8
  return s;
}

// ring shape per query count: TPR tokens per row per step, NB steps in the
// ring (NB - 1 in flight), W waves per SIMD asked of the register allocator
// (measured at 64k tokens, 8 heads, 4 queries: 51.3 us per call at NB 4 with
// 3 waves, 52.3 at NB 5 with 2, 51.0-53.5 from NB 6 to 8)
template <int G>
struct FdRing {
  static constexpr int TPR = 2;
  static constexpr int NB = G >= 8 ? 4 : (G >= 4 ? 4 : 6);
  static constexpr int W = G >= 8 ? 2 : 3;
};

template <int G>
__global__ __launch_bounds__(kFdThreads) __attribute__((amdgpu_waves_per_eu(FdRing<G>::W)))
void fp16_decode_split_kernel(const FdArgs a) {
  constexpr int NB = FdRing<G>::NB, TPR = FdRing<G>::TPR;
  constexpr int kStepTok = 4 * TPR, kChunk = 4 * kStepTok;   // tokens per wave step, per workgroup step
  const int split = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, r = lane >> 4, c8 = lane & 15;
  const int n_chunks = (a.T + kChunk - 1) / kChunk;
  const int c0 = (int)((int64_t)split * n_chunks / a.n_split), c1 = (int)((int64_t)(split + 1) * n_chunks / a.n_split);
  const int n_steps = c1 - c0;
  // K and V of the head through buffer descriptors: rows past T read zeros
  // (and are masked), offsets are 32-bit
  const uint32_t nrec = (uint32_t)((int64_t)a.T * a.st * 2);
  const __amdgpu_buffer_rsrc_t krs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.k + (int64_t)h * a.sh), (short)0, nrec, kFdBufWord3);
  const __amdgpu_buffer_rsrc_t vrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.v + (int64_t)h * a.sh), (short)0, nrec, kFdBufWord3);
  // byte offset of token (step s, j): chunk base + kStepTok wave + r + 4 j
  const uint32_t lane_off = (uint32_t)(((int64_t)(kStepTok * wave + r) * a.st + 8 * c8) * 2);
  const uint32_t tok4_off = (uint32_t)(4 * a.st * 2);
  const uint32_t chunk_off = (uint32_t)((int64_t)kChunk * a.st * 2);

  uint32_t qv[G][4];   // the queries' channels 8 c8 .. +7, fp16 pairs
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const uint4 w = *reinterpret_cast<const uint4*>(a.q + ((int64_t)h * a.G + g) * kFdD + 8 * c8);
    qv[g][0] = w.x; qv[g][1] = w.y; qv[g][2] = w.z; qv[g][3] = w.w;
  }
  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[g][i] = 0.f;
  }
  fd_u4 kb[NB][TPR], vb[NB][TPR];
  auto issue = [&](int s, fd_u4 kd[TPR], fd_u4 vd[TPR]) {
    const uint32_t base = (uint32_t)(c0 + s) * chunk_off + lane_off;
#pragma unroll
    for (int j = 0; j < TPR; ++j) kd[j] = __builtin_amdgcn_raw_buffer_load_b128(krs, base + j * tok4_off, 0, 2);
#pragma unroll
    for (int j = 0; j < TPR; ++j) vd[j] = __builtin_amdgcn_raw_buffer_load_b128(vrs, base + j * tok4_off, 0, 2);
  };
#pragma unroll
  for (int b = 0; b < NB - 1; ++b)
    if (b < n_steps) issue(b, kb[b], vb[b]);

  for (int s0 = 0; s0 < n_steps; s0 += NB) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int s = s0 + b;
      if (s >= n_steps) break;
      if (s + NB - 1 < n_steps) issue(s + NB - 1, kb[(b + NB - 1) % NB], vb[(b + NB - 1) % NB]);
      const int t_first = (c0 + s) * kChunk + kStepTok * wave + r;   // token of j = 0; j adds 4 j
      // ---- scores of the lane's tokens for every query
      float p[G][TPR];
#pragma unroll
      for (int j = 0; j < TPR; ++j) {
        const fd_u4 kw = kb[b][j];
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float x = 0.f;
#pragma unroll
          for (int e = 0; e < 4; ++e) x = __builtin_amdgcn_fdot2(h2(kw[e]), h2(qv[g][e]), x, false);
          x = row16_sum(x);
          p[g][j] = t_first + 4 * j < a.T ? x * a.qscale : -INFINITY;
        }
      }
      // ---- online softmax per query: p becomes the weights, acc is rescaled
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float mx = p[g][0];
#pragma unroll
        for (int j = 1; j < TPR; ++j) mx = fmaxf(mx, p[g][j]);
        const float mn = fmaxf(m[g], mx);
        // a stream with no token yet (its tokens all past T) keeps m = -inf
        const float ms = mn == -INFINITY ? 0.f : mn;
        const float al = __builtin_amdgcn_exp2f(m[g] - ms);   // 0 when m was -inf
        float ps = 0.f;
#pragma unroll
        for (int j = 0; j < TPR; ++j) {
          p[g][j] = __builtin_amdgcn_exp2f(p[g][j] - ms);
          ps += p[g][j];
        }
        l[g] = __builtin_fmaf(l[g], al, ps);
        m[g] = mn;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[g][i] *= al;
      }
      // ---- P.V: token by token, its 8 channels in fp32
#pragma unroll
      for (int j = 0; j < TPR; ++j) {
        const fd_u4 vw = vb[b][j];
        float vf[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const f16x2_t p2 = h2(vw[e]);
          vf[2 * e] = (float)p2[0];
          vf[2 * e + 1] = (float)p2[1];
        }
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[g][i] = __builtin_fmaf(p[g][j], vf[i], acc[g][i]);
      }
    }
  }
  // ---- the 16 streams (4 waves x 4 rows) meet: stream st = 4 wave + r
  __shared__ float s_ml[16][G][2];
  __shared__ float s_x[16][G][kFdD];
  const int stream = 4 * wave + r;
#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int i = 0; i < 8; ++i) s_x[stream][g][8 * c8 + i] = acc[g][i];
    if (c8 == 0) {
      s_ml[stream][g][0] = m[g];
      s_ml[stream][g][1] = l[g];
    }
  }
  __syncthreads();
  for (int e = tid; e < G * kFdD; e += kFdThreads) {
    const int g = e / kFdD, ch = e % kFdD;
    float M = -INFINITY;   // streams that saw no token keep -inf and weigh 0
#pragma unroll
    for (int j = 0; j < 16; ++j) M = fmaxf(M, s_ml[j][g][0]);
    float L = 0.f, X = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float w = __builtin_amdgcn_exp2f(s_ml[j][g][0] - M);   // 0 for an empty stream
        L = __builtin_fmaf(w, s_ml[j][g][1], L);
        X = __builtin_fmaf(w, s_x[j][g][ch], X);
      }
    }
    float* dst = a.part + (((int64_t)h * a.G + g) * a.n_split + split) * (2 + kFdD);
    dst[2 + ch] = X;
    if (ch == 0) {
      dst[0] = M;
      dst[1] = L;
    }
  }
}

struct FdMergeArgs {
  const float* part;
  int n_split, G;
  uint16_t* out;   // [h_kv][G][128] fp16
};

// block 256: thread (split lane sl = tid / 32, channel quad cq = tid % 32)
// takes splits sl, sl + 8, ... for channels 4 cq .. + 3, 8 splits' loads at a
// time; the 8 split lanes meet in LDS.
__global__ __launch_bounds__(256) void fp16_decode_merge_kernel(const FdMergeArgs a) {
  const int row = blockIdx.x, tid = threadIdx.x, sl = tid >> 5, cq = tid & 31;
  const float* base = a.part + (int64_t)row * a.n_split * (2 + kFdD);
  __shared__ float s_m[8], s_l[8];
  __shared__ float4 s_x[8][32];
  float m = -INFINITY, l = 0.f;
  float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int sp0 = sl; sp0 < a.n_split; sp0 += 64) {
    float ms[8], ls[8];
    float4 vs[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int sp = sp0 + 8 * u;
      const float* p = base + (int64_t)min(sp, a.n_split - 1) * (2 + kFdD);
      ms[u] = sp < a.n_split ? p[0] : -INFINITY;
      ls[u] = p[1];
      vs[u] = *reinterpret_cast<const float4*>(p + 2 + 4 * cq);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (ms[u] == -INFINITY) continue;
      const float mn = fmaxf(m, ms[u]);
      const float al = __builtin_amdgcn_exp2f(m - mn), w = __builtin_amdgcn_exp2f(ms[u] - mn);
      l = l * al + w * ls[u];
      x = make_float4(x.x * al + w * vs[u].x, x.y * al + w * vs[u].y, x.z * al + w * vs[u].z,
                      x.w * al + w * vs[u].w);
      m = mn;
    }
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
  // one head's rows are addressed with 32-bit byte offsets (buffer loads)
  if ((int64_t)(a->T + kFdChunk) * a->stride_t * 2 > INT32_MAX) return BMX_BENCH_E_INVALID;
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
