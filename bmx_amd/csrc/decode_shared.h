// Decode pieces shared by the k2b and RTN split-KV paths on gfx950: the
// recent window's MFMA score tiles, the query fragments they use, and the
// merge kernel that combines the split partials with the window.
#pragma once

#include "k2b_common.h"

namespace bmx {

// ---------------------------------------------------------------------------
// Recent-window scores (any decode kernel whose arguments carry k_tail, ts_b,
// ts_h, ts_t, tail_cap, win_rescale, ws_win, h_kv, G).  Window tile j (tokens
// 16j .. 16j + 15 of the fp16 post-RoPE window) belongs to workgroup j mod
// max_splits and is scored on the MFMA like a packed page: A = its 16 key rows (lane: token lane & 15, quarter
// q = lane >> 4 holds channels 16bb + 4q + i and + 64, interleaved: the K order
// of the query fragments), B = the query fragments split into fp16 high and low
// parts (q = hi + lo to 2^-22 relative), so the scores carry the fp32 query.
// Base-2 scores go to ws_win[b][h][g][t]; the merge does the window's softmax
// and value sum.  Rows past tail_cap read row 0 of the head and are not stored.
// ---------------------------------------------------------------------------
template <class A>
__device__ __forceinline__ void load_win_tile(const A& a, int64_t tail_base, int j, int n, int q,
                                              uint2 kw[8]) {
  const int t = 16 * j + n;
  const uint16_t* row = a.k_tail + tail_base + (int64_t)(t < a.tail_cap ? t : 0) * a.ts_t + 4 * q;
#pragma unroll
  for (int bb = 0; bb < 4; ++bb) {
    kw[2 * bb] = *reinterpret_cast<const uint2*>(row + 16 * bb);
    kw[2 * bb + 1] = *reinterpret_cast<const uint2*>(row + 16 * bb + 64);
  }
}

template <class A>
__device__ __forceinline__ void score_win_tile(const A& a, int b, int h, int j, int n, int q,
                                               const uint2 kw[8], const half8_t qh[4], const half8_t ql[4]) {
  float4_t s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int bb = 0; bb < 4; ++bb) {
    const uint2 lo = kw[2 * bb], hi = kw[2 * bb + 1];   // channels +0..3 and +64..67
    union { uint4 u; half8_t v; } ka;
    ka.u = make_uint4(__builtin_amdgcn_perm(hi.x, lo.x, 0x05040100u), __builtin_amdgcn_perm(hi.x, lo.x, 0x07060302u),
                      __builtin_amdgcn_perm(hi.y, lo.y, 0x05040100u), __builtin_amdgcn_perm(hi.y, lo.y, 0x07060302u));
    s = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka.v, qh[bb], s, 0, 0, 0);
    s = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka.v, ql[bb], s, 0, 0, 0);
  }
  // lane: query n, tokens 16j + 4q + i
  if (n < a.G) {
    float* dst = a.ws_win + (((int64_t)b * a.h_kv + h) * a.G + n) * a.tail_cap;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * j + 4 * q + i;
      if (t < a.tail_cap) dst[t] = s[i] * a.win_rescale;
    }
  }
}

// Query fragments in the RoPE pair order, fp16 high and low parts: chunk bb
// holds B[8q + 2i + e][n] = x_n[16bb + 4q + i + 64e] (i < 4, e < 2), the order
// in which k2b's key pairs leave the rotation and the window tiles' K order;
// x = q * sc; column n is query n (zero if sc is 0).  qraw[u]: the lane's
// q_n[16(u & 3) + 4q .. + 3 + 64(u >> 2)].
__device__ __forceinline__ void query_fragments(const float4_t qraw[8], float sc, half8_t qh[4], half8_t ql[4]) {
#pragma unroll
  for (int bb = 0; bb < 4; ++bb)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float x = qraw[4 * e + bb][i] * sc;
        const _Float16 xh = (_Float16)x;
        qh[bb][2 * i + e] = xh;
        ql[bb][2 * i + e] = (_Float16)(x - (float)xh);
      }
}

// ---------------------------------------------------------------------------
// Combine: merge of the packed partials and the recent window.  One workgroup
// per (16-channel chunk, query row, sequence): the partials arrive already in
// the output domain, so a chunk needs only its own 16 channels of every split
// (contiguous, 64 B per split) plus every split's (max, sum); the window needs
// its scores (computed by the split kernel) and its 16 value channels of every
// token.  Thread i takes split i and window token i of each 256-wide block;
// every load of the first block is issued before any reduction.
// ---------------------------------------------------------------------------
constexpr int kCmbThreads = 256;
constexpr int kCmbWaves = kCmbThreads / 64;
constexpr int kChunk = 16;                  // channels per workgroup
constexpr int kChunks = kD / kChunk;
constexpr int kRedPad = kCmbThreads + 4;    // LDS row stride of the reductions

struct CombineKArgs {
  int h_kv, G, max_splits, tail_cap;
  float* out;
  const float* ws_acc;
  const float* ws_ml;
  const float* ws_win;
  const uint16_t* v_tail;
  int64_t ts_b, ts_h, ts_t;
  const int32_t* tail_len;
  uint32_t v_sign_bits[4];   // rotated: bit c set <=> value channel c carries Hadamard sign -1
  float packed_scale;        // rotated: 1 / (128 kappa), the Hadamard normalisation and the
                             // level scale; 1 otherwise
};

// Sum over the 16 lanes of a row (DPP-free butterfly; result in every lane).
__device__ __forceinline__ float row_sum16(float x) {
  x += __shfl_xor(x, 8);
  x += __shfl_xor(x, 4);
  x += __shfl_xor(x, 2);
  x += __shfl_xor(x, 1);
  return x;
}

// kRotated: the packed partials are sums of k2b's rotated value levels with
// the H8 half of the inverse Hadamard applied (the merge applies H16, the
// signs and packed_scale); otherwise they are plain channel sums.
template <bool kRotated>
__global__ __launch_bounds__(kCmbThreads) void combine_kernel(const CombineKArgs a) {
  const int ch = blockIdx.x, r = blockIdx.y, b = blockIdx.z;
  const int h = r / a.G;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int S = a.max_splits;
  const int64_t row = (int64_t)b * a.h_kv * a.G + r;   // (b, h, g) row
  const float* accb = a.ws_acc + (row * kChunks + ch) * (int64_t)S * kChunk;
  const float* mlb = a.ws_ml + row * S * 2;
  const float* swb = a.ws_win + row * a.tail_cap;
  const uint16_t* vb = a.v_tail + b * a.ts_b + h * a.ts_h + kChunk * ch;
  typedef float f2_t __attribute__((ext_vector_type(2)));
  __shared__ float s_red[2 * kCmbWaves];
  __shared__ float s_fin[2 * kChunk];
  __shared__ float s_x[kChunk * kRedPad];
  __shared__ float s_v[kChunk * kRedPad];

  float4_t v[4];
  f2_t ml = {-INFINITY, 0.f};
  uint4 vv[2];
  float sw = -INFINITY;
  // partial block k and window block k, no waits; the first block's window
  // rows are bounded by the host's tail_cap, so they do not wait for tail_len
  auto load_block = [&](int k, int t_end) {
    const int i0 = k * kCmbThreads;
    if (i0 < S) {
      const int i = min(i0 + tid, S - 1);
      ml = *reinterpret_cast<const f2_t*>(mlb + 2 * (int64_t)i);
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = *reinterpret_cast<const float4_t*>(accb + (int64_t)i * kChunk + 4 * u);
    }
    if (i0 < t_end) {
      const int t = min(i0 + tid, t_end - 1);
      sw = swb[t];
      vv[0] = *reinterpret_cast<const uint4*>(vb + (int64_t)t * a.ts_t);
      vv[1] = *reinterpret_cast<const uint4*>(vb + (int64_t)t * a.ts_t + 8);
    }
  };
  load_block(0, a.tail_cap);

  const int T = min(max(a.tail_len[b], 0), a.tail_cap);
  float4_t xp[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) xp[u] = float4_t{0.f, 0.f, 0.f, 0.f};
  float vacc[kChunk];
#pragma unroll
  for (int e = 0; e < kChunk; ++e) vacc[e] = 0.f;
  float mp = -INFINITY, mt = -INFINITY, lp = 0.f, lt = 0.f;   // lp, lt: this thread's share
  const int n_blk = (max(S, T) + kCmbThreads - 1) / kCmbThreads;
  for (int k = 0; k < n_blk; ++k) {   // uniform trip count
    if (k != 0) load_block(k, T);
    const int i0 = k * kCmbThreads;
    const bool own_p = i0 + tid < S;
    const float mi = own_p ? ml[0] : -INFINITY;
    const float st = i0 + tid < T ? sw : -INFINITY;
    // one joint block max of (partial max, window score)
    float r0 = mi, r1 = st;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      r0 = fmaxf(r0, __shfl_xor(r0, o));
      r1 = fmaxf(r1, __shfl_xor(r1, o));
    }
    if (lane == 0) {
      s_red[2 * wave] = r0;
      s_red[2 * wave + 1] = r1;
    }
    __syncthreads();
#pragma unroll
    for (int w = 0; w < kCmbWaves; ++w) {
      r0 = fmaxf(r0, s_red[2 * w]);
      r1 = fmaxf(r1, s_red[2 * w + 1]);
    }
    const float mp_new = fmaxf(mp, r0), mt_new = fmaxf(mt, r1);
    const float ap = mp == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mp - mp_new);
    const float at = mt == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mt - mt_new);
    const float wi = mi == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mi - mp_new);
    const float pt = st == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(st - mt_new);
    lp = lp * ap + (own_p ? ml[1] * wi : 0.f);
    lt = lt * at + pt;
#pragma unroll
    for (int u = 0; u < 4; ++u) xp[u] = xp[u] * ap + (own_p ? v[u] * wi : float4_t{0.f, 0.f, 0.f, 0.f});
    if (i0 < T) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t w = (e < 4 ? (&vv[0].x)[e] : (&vv[1].x)[e - 4]);
        vacc[2 * e] = __builtin_fmaf(pt, half_bits_to_float(w & 0xffff), vacc[2 * e] * at);
        vacc[2 * e + 1] = __builtin_fmaf(pt, half_bits_to_float(w >> 16), vacc[2 * e + 1] * at);
      }
    }
    mp = mp_new;
    mt = mt_new;
    __syncthreads();   // s_red is rewritten by the next block
  }
  // ---- gather: channel c of the packed sum over the splits (thread tid holds
  // split tid's share), of the window sum over the tokens, and the denominators ----
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int e = 0; e < 4; ++e) s_x[(4 * u + e) * kRedPad + tid] = xp[u][e];
#pragma unroll
  for (int e = 0; e < kChunk; ++e) s_v[e * kRedPad + tid] = vacc[e];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    lp += __shfl_xor(lp, o);
    lt += __shfl_xor(lt, o);
  }
  if (lane == 0) {
    s_red[2 * wave] = lp;
    s_red[2 * wave + 1] = lt;
  }
  __syncthreads();
  float lpt = 0.f, ltt = 0.f;
#pragma unroll
  for (int w = 0; w < kCmbWaves; ++w) {
    lpt += s_red[2 * w];
    ltt += s_red[2 * w + 1];
  }
  // thread (c = tid / 16, part = tid % 16) sums splits and tokens part + 16j
  const int c = tid >> 4, part = tid & 15;
  float x = 0.f, wv = 0.f;
#pragma unroll
  for (int j = 0; j < kCmbThreads / 16; ++j) {
    x += s_x[c * kRedPad + part + 16 * j];
    wv += s_v[c * kRedPad + part + 16 * j];
  }
  x = row_sum16(x);
  wv = row_sum16(wv);
  if (part == 0) {
    s_fin[c] = x;
    s_fin[kChunk + c] = wv;
  }
  __syncthreads();
  if (tid < kChunk) {
    float y = s_fin[tid];
    const int cg = kChunk * ch + tid;
    if constexpr (kRotated) {
      // lane c: H16 over the chunk's channel bits 0-3, then sign and 1/(128 kappa)
#pragma unroll
      for (int hb = 1; hb < kChunk; hb <<= 1) {
        const float p = __shfl_xor(y, hb);
        y = (tid & hb) ? p - y : y + p;
      }
      y = (sign_neg(a.v_sign_bits, cg) ? -y : y) * a.packed_scale;
    }
    const float M = fmaxf(mp, mt);
    const float wp = mp == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mp - M);
    const float wt = mt == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mt - M);
    const float inv = 1.0f / (lpt * wp + ltt * wt);
    a.out[row * kD + cg] = (y * wp + s_fin[kChunk + tid] * wt) * inv;
  }
}

}  // namespace bmx
