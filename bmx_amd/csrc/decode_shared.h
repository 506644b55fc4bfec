// Decode pieces shared by the k2b and RTN split-KV paths on gfx950: the
// recent window's MFMA score tiles, the query fragments they use, and the
// merge kernel that combines the split partials with the window.
#pragma once

#include "k2b_common.h"

namespace bmx {

constexpr int kSyncPolls = 1 << 22;   // bound of a wave's wait on another wave's ring slot

// Wait until the workgroup counter *c reaches target (LDS, acquire at
// workgroup scope); bounded, so a wave can never wait for ever.
__device__ __forceinline__ void wait_count(uint32_t* c, uint32_t target) {
  for (int it = 0; it < kSyncPolls; ++it) {
    if (__hip_atomic_load(c, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) return;
    __builtin_amdgcn_s_sleep(1);
  }
}

// One wave's arrival at the workgroup counter *c (release at workgroup scope:
// the wave's earlier LDS reads and writes are complete).
__device__ __forceinline__ void count_wave(uint32_t* c) {
  __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): every lane's LDS access has completed
  if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// ---------------------------------------------------------------------------
// Balanced split of a ragged batch.  Sequence b of n_seq (at most 64) gets
// 1 + floor((n_wg - n_seq) * groups_b / total) of the n_wg split workgroups,
// groups_b = its committed 64-token groups (packed_len clamped to max_len),
// and its workgroups follow those of sequences 0 .. b - 1.  Every lane of a
// wave computes the same shares; lane i returns sequence i's share, first
// workgroup and length (lanes >= n_seq: share 0).
// ---------------------------------------------------------------------------
constexpr int kMaxBalancedBatch = 64;

__device__ __forceinline__ void batch_shares(const int32_t* packed_len, int max_len, int n_seq, int n_wg,
                                             int& share, int& first, int& len) {
  const int lane = threadIdx.x & 63;
  len = lane < n_seq ? min(max(packed_len[lane], 0), max_len) & ~63 : 0;
  const int groups = len >> 6;
  int total = groups;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) total += __shfl_xor(total, o);
  share = lane < n_seq ? 1 + (int)(((int64_t)(n_wg - n_seq) * groups) / max(total, 1)) : 0;
  int incl = share;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(incl, o);
    if (lane >= o) incl += t;
  }
  first = incl - share;
}

// ---------------------------------------------------------------------------
// The newest rows of the recent window, given apart (a decode step's own
// token): rows [T - n, T) of every sequence's window (T = the window length,
// a host value) come from k / v instead of the window buffers, and are
// copied into the buffers (k_dst / v_dst, the window's own pointers) for
// the calls that follow: the keys by the split kernel that scores them, the
// values by the merge that reads them.
// ---------------------------------------------------------------------------
struct WinNew {
  const uint16_t* k;   // fp16 post-RoPE keys, row i of (b, h) at b * sb + h * sh + i * st
  const uint16_t* v;   // fp16 values, same indexing
  int64_t sb, sh, st;
  int n;               // rows given apart (0: none)
  int T;               // window length when given by the host (tail_len NULL), else -1
  uint16_t* k_dst;     // = k_tail
  uint16_t* v_dst;     // = v_tail
};

// row t of the window is one of the rows given apart: its index among them, else -1
__device__ __forceinline__ int fresh_row(const WinNew& w, int t) {
  const int i = t - (w.T - w.n);
  return (w.n > 0 && i >= 0 && t < w.T) ? i : -1;
}

// ---------------------------------------------------------------------------
// Recent-window scores (any decode kernel whose arguments carry k_tail, ts_b,
// ts_h, ts_t, tail_cap, win_rescale, ws_win, h_kv, G).  Window tile j (tokens
// 16j .. 16j + 15 of the fp16 post-RoPE window), scored by the workgroup the
// decode kernel deals it to, goes on the MFMA like a packed page: A = its 16 key rows (lane: token lane & 15, quarter
// q = lane >> 4 holds channels 16bb + 4q + i and + 64, interleaved: the K order
// of the query fragments), B = the query fragments split into fp16 high and low
// parts (q = hi + lo to 2^-22 relative), so the scores carry the fp32 query.
// A bf16 window (tail_bf16: a bf16 model's rows as the model made them) goes
// on the bf16 MFMA, its query split into bf16 high and low parts (2^-17).
// Base-2 scores go to ws_win[b][h][g][t]; the merge does the window's softmax
// and value sum.  Rows past tail_cap read row 0 of the head and are not stored.
// ---------------------------------------------------------------------------
template <class A>
__device__ __forceinline__ void load_win_tile(const A& a, int64_t tail_base, int j, int n, int q,
                                              uint2 kw[8], int64_t new_base) {
  const int t = 16 * j + n;
  const int i_new = fresh_row(a.nw, t);
  const uint16_t* row = i_new >= 0 ? a.nw.k + new_base + (int64_t)i_new * a.nw.st + 4 * q
                                   : a.k_tail + tail_base + (int64_t)(t < a.tail_cap ? t : 0) * a.ts_t + 4 * q;
#pragma unroll
  for (int bb = 0; bb < 4; ++bb) {
    kw[2 * bb] = *reinterpret_cast<const uint2*>(row + 16 * bb);
    kw[2 * bb + 1] = *reinterpret_cast<const uint2*>(row + 16 * bb + 64);
  }
}

template <class A>
__device__ __forceinline__ void score_win_tile(const A& a, int b, int h, int j, int n, int q,
                                               const uint2 kw[8], const half8_t qh[4], const half8_t ql[4],
                                               int64_t tail_base) {
  if (fresh_row(a.nw, 16 * j + n) >= 0) {   // a row given apart: into the window buffer
    uint16_t* dst = a.nw.k_dst + tail_base + (int64_t)(16 * j + n) * a.ts_t + 4 * q;
#pragma unroll
    for (int bb = 0; bb < 4; ++bb) {
      *reinterpret_cast<uint2*>(dst + 16 * bb) = kw[2 * bb];
      *reinterpret_cast<uint2*>(dst + 16 * bb + 64) = kw[2 * bb + 1];
    }
  }
  // the window dtype as a wave-uniform (scalar) value: a branch on it is a
  // scalar branch.  Read through a pointer it would be a vector value, and the
  // two MFMA forms would be selected by the exec mask, where the form not
  // taken still writes its result (an MFMA runs whatever the exec mask).
  const bool bf16 = __builtin_amdgcn_readfirstlane(a.tail_bf16) != 0;
  float4_t s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int bb = 0; bb < 4; ++bb) {
    const uint2 lo = kw[2 * bb], hi = kw[2 * bb + 1];   // channels +0..3 and +64..67
    union { uint4 u; half8_t v; } ka;
    ka.u = make_uint4(__builtin_amdgcn_perm(hi.x, lo.x, 0x05040100u), __builtin_amdgcn_perm(hi.x, lo.x, 0x07060302u),
                      __builtin_amdgcn_perm(hi.y, lo.y, 0x05040100u), __builtin_amdgcn_perm(hi.y, lo.y, 0x07060302u));
    if (bf16) {
      s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, ka.v),
                                                  __builtin_bit_cast(bf16x8_t, qh[bb]), s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, ka.v),
                                                  __builtin_bit_cast(bf16x8_t, ql[bb]), s, 0, 0, 0);
    } else {
      s = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka.v, qh[bb], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka.v, ql[bb], s, 0, 0, 0);
    }
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

// Query and output elements of a decode call in its I/O dtype: 0 = fp32,
// 1 = fp16, 2 = bf16 (BMX_K2B_IO_*; the model's own dtype, so a decode step
// needs no conversion kernel).  Four consecutive elements from element idx.
constexpr int kIoF32 = 0, kIoF16 = 1, kIoBF16 = 2;

__device__ __forceinline__ float4_t load_q4(const void* base, int64_t idx, int io) {
  if (io == kIoF32) return *reinterpret_cast<const float4_t*>(reinterpret_cast<const float*>(base) + idx);
  const uint2 r = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(base) + idx);
  if (io == kIoF16) {
    const half2_t lo = as_h2(r.x), hi = as_h2(r.y);
    return float4_t{(float)lo[0], (float)lo[1], (float)hi[0], (float)hi[1]};
  }
  return float4_t{__builtin_bit_cast(float, r.x << 16), __builtin_bit_cast(float, r.x & 0xffff0000u),
                  __builtin_bit_cast(float, r.y << 16), __builtin_bit_cast(float, r.y & 0xffff0000u)};
}

__device__ __forceinline__ uint32_t bf16_bits(float v) {   // round to nearest even, NaN kept
  uint32_t u = __builtin_bit_cast(uint32_t, v);
  u = (u & 0x7fffffffu) > 0x7f800000u ? (u | 0x00400000u) : u + 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ void store_o4(void* base, int64_t idx, float4_t v, int io) {
  if (io == kIoF32) {
    *reinterpret_cast<float4_t*>(reinterpret_cast<float*>(base) + idx) = v;
    return;
  }
  uint2 w;
  if (io == kIoF16) {
    const half2_t lo = {(_Float16)v[0], (_Float16)v[1]}, hi = {(_Float16)v[2], (_Float16)v[3]};
    w = make_uint2(as_u32(lo), as_u32(hi));
  } else {
    w = make_uint2(bf16_bits(v[0]) | (bf16_bits(v[1]) << 16), bf16_bits(v[2]) | (bf16_bits(v[3]) << 16));
  }
  *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(base) + idx) = w;
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

// The same fragments for the window tiles: fp16 high and low parts, or bf16
// ones (bit patterns in the half8_t registers) for a bf16 window.
__device__ __forceinline__ void window_fragments(const float4_t qraw[8], float sc, bool bf16, half8_t qh[4],
                                                 half8_t ql[4]) {
  if (!bf16) {
    query_fragments(qraw, sc, qh, ql);
    return;
  }
#pragma unroll
  for (int bb = 0; bb < 4; ++bb)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float x = qraw[4 * e + bb][i] * sc;
        const uint32_t hb = bf16_bits(x);
        qh[bb][2 * i + e] = __builtin_bit_cast(_Float16, (uint16_t)hb);
        ql[bb][2 * i + e] = __builtin_bit_cast(_Float16, (uint16_t)bf16_bits(x - __uint_as_float(hb << 16)));
      }
}

// ---------------------------------------------------------------------------
// Split partial records.  A (row, split) partial is its 128 channel sums
// divided by its softmax sum l, in fp16 (a weighted mean of value-sized
// numbers: 2^-12 relative rounding, half the bytes of fp32), chunk-major so a
// merge workgroup reads one 32-byte record per split: acc16[row][chunk][S][16];
// (m, l) stay fp32 in ml[row][S][2].  The merge weighs record s by
// l_s 2^(m_s - M).  An empty split (l = 0, m = -inf) stores zeros.
// Lane 16q + n (n < G: query n) writes channels 4q..4q+3 of each chunk.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void store_partial_record(uint16_t* acc16, float* ml, int64_t row, int S, int split,
                                                     int q, const float4_t acc[8], float m_run, float l_run) {
  const float inv_l = l_run > 0.f ? 1.0f / l_run : 0.f;
  uint16_t* dst = acc16 + (row * 8 * S + split) * 16 + 4 * q;   // chunk bt at + bt * S * 16
#pragma unroll
  for (int bt = 0; bt < 8; ++bt) {
    const half2_t lo = {(_Float16)(acc[bt][0] * inv_l), (_Float16)(acc[bt][1] * inv_l)};
    const half2_t hi = {(_Float16)(acc[bt][2] * inv_l), (_Float16)(acc[bt][3] * inv_l)};
    *reinterpret_cast<uint2*>(dst + (int64_t)bt * S * 16) = make_uint2(as_u32(lo), as_u32(hi));
  }
  if (q == 0) *reinterpret_cast<float2*>(ml + (row * S + split) * 2) = make_float2(m_run, l_run);
}

// Bytes of the partial records and (m, l) of rows x splits (the window scores follow).
__host__ __device__ __forceinline__ size_t partial_bytes(size_t rows, size_t splits) {
  return rows * splits * (kD * 2 + 2 * 4);
}

// ---------------------------------------------------------------------------
// Combine: merge of the packed partials and the recent window.  One workgroup
// of kCmbWaves waves per (16-channel chunk, query row, sequence): the partials
// arrive already in the output domain, so a chunk needs only its own 16
// channels of every split (contiguous, 64 B per split) plus every split's
// (max, sum); the window needs its scores (computed by the split kernel) and
// its 16 value channels of every token.  Splits and window tokens are dealt
// in blocks of 16: wave w takes blocks w, w + kCmbWaves, ...; lane (phase
// p = lane & 15, quarter c4 = lane >> 4) takes channels 4c4 .. 4c4 + 3 of
// element p of each of its blocks.  Every row of 16 lanes sees all of its
// wave's elements, so a wave's maxima and sums are row reductions (DPP);
// the waves' (max, sum, channel sums) then meet once in LDS, and only the
// final Hadamard crosses rows.  All loads of a wave's first pass are issued
// before any use.
// ---------------------------------------------------------------------------
constexpr int kCmbWaves = 4;
constexpr int kCmbThreads = 64 * kCmbWaves;
constexpr int kChunk = 16;                  // channels per merge unit
constexpr int kChunks = kD / kChunk;
constexpr int kCmbSplits = 4;               // split blocks per wave per pass
constexpr int kCmbTokens = 2;               // window-token blocks per wave per pass

struct CombineKArgs {
  int h_kv, G, max_splits, tail_cap;   // max_splits: partial slots per row
  int balanced, n_wg;                  // balanced: sequence b has its batch_shares() share of n_wg
  const int32_t* packed_len;
  int max_packed_len;
  void* out;               // [B][h_kv][G][128] in io_dtype
  int io_dtype;
  const uint16_t* ws_acc;   // partial records (store_partial_record)
  const float* ws_ml;
  const float* ws_win;
  const uint16_t* v_tail;
  int64_t ts_b, ts_h, ts_t;
  int tail_bf16;             // window (and rows given apart) in bf16, else fp16
  const int32_t* tail_len;   // NULL: every sequence's window holds nw.T rows
  WinNew nw;
  uint32_t v_sign_bits[4];   // rotated: bit c set <=> value channel c carries Hadamard sign -1
  float packed_scale;        // rotated: 1 / (128 kappa), the Hadamard normalisation and the
                             // level scale; 1 otherwise
};

// v from another lane of the same 16-lane row (DPP control CTRL), every lane written.
template <int CTRL>
__device__ __forceinline__ float dpp_row(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// All-reduce over the 16 lanes of a row with DPP (quad xor 1, quad xor 2,
// half-row mirror, row mirror): every lane gets the same value.
template <bool kMax>
__device__ __forceinline__ float row_reduce16(float x) {
  if constexpr (kMax) {
    x = fmaxf(x, dpp_row<0xB1>(x));    // quad_perm [1,0,3,2]
    x = fmaxf(x, dpp_row<0x4E>(x));    // quad_perm [2,3,0,1]
    x = fmaxf(x, dpp_row<0x141>(x));   // row_half_mirror
    x = fmaxf(x, dpp_row<0x140>(x));   // row_mirror
  } else {
    x += dpp_row<0xB1>(x);
    x += dpp_row<0x4E>(x);
    x += dpp_row<0x141>(x);
    x += dpp_row<0x140>(x);
  }
  return x;
}

// weight e^(m_i - M) of a part with running max m_i (0 for an empty part)
__device__ __forceinline__ float part_weight(float mi, float M) {
  return mi == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mi - M);
}

// kRotated: the packed partials are sums of k2b's rotated value levels with
// the H8 half of the inverse Hadamard applied (the merge applies H16, the
// signs and packed_scale); otherwise they are plain channel sums.
// kTok: window-token blocks per wave per pass: kCmbTokens (128 tokens per
// pass), or 4 for windows of more than 128 rows (up to 255 between commits),
// so that the window is one pass, one memory round trip.
template <bool kRotated, int kTok>
__global__ __launch_bounds__(kCmbThreads) void combine_kernel(const CombineKArgs a) {
  const int ch = blockIdx.x, r = blockIdx.y, b = blockIdx.z;
  const int h = r / a.G;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, p = lane & 15, c4 = lane >> 4;
  const int S_slots = a.max_splits;
  const int64_t row = (int64_t)b * a.h_kv * a.G + r;   // (b, h, g) row
  const uint16_t* accb = a.ws_acc + (row * kChunks + ch) * (int64_t)S_slots * kChunk + 4 * c4;
  const float* mlb = a.ws_ml + row * S_slots * 2;
  const float* swb = a.ws_win + row * a.tail_cap;
  const uint16_t* vb = a.v_tail + b * a.ts_b + h * a.ts_h + kChunk * ch + 4 * c4;
  const int64_t new_base = b * a.nw.sb + h * a.nw.sh + kChunk * ch + 4 * c4;
  typedef float f2_t __attribute__((ext_vector_type(2)));
  // element e of this lane in pass j0: p + 16 (wave + kCmbWaves u) + j0
  auto elem = [&](int j0, int u) { return j0 + p + 16 * (wave + kCmbWaves * u); };
  constexpr int kSplitPass = 16 * kCmbWaves * kCmbSplits;   // splits per pass of the workgroup
  constexpr int kTokenPass = 16 * kCmbWaves * kTok;   // window tokens per pass

  f2_t ml[kCmbSplits];
  float4_t pv[kCmbSplits];
  float ws[kTok];
  uint2 wv[kTok];
  int S = S_slots;   // the sequence's splits
  auto load_splits = [&](int j0) {
#pragma unroll
    for (int u = 0; u < kCmbSplits; ++u) {
      const int i = min(elem(j0, u), S - 1);
      ml[u] = *reinterpret_cast<const f2_t*>(mlb + 2 * (int64_t)i);
      const uint2 r = *reinterpret_cast<const uint2*>(accb + (int64_t)i * kChunk);
      const half2_t lo = as_h2(r.x), hi = as_h2(r.y);
      pv[u] = float4_t{(float)lo[0], (float)lo[1], (float)hi[0], (float)hi[1]};
    }
  };
  auto load_tokens = [&](int t0, int t_end) {   // t_end >= 1
#pragma unroll
    for (int u = 0; u < kTok; ++u) {
      const int t = min(elem(t0, u), t_end - 1);
      ws[u] = swb[t];
      const int i_new = fresh_row(a.nw, t);
      wv[u] = *reinterpret_cast<const uint2*>(i_new >= 0 ? a.nw.v + new_base + (int64_t)i_new * a.nw.st
                                                         : vb + (int64_t)t * a.ts_t);
    }
  };
  // first pass of both: the window rows bounded by the host's tail_cap (no
  // wait on tail_len), the partials by the sequence's split count (a ragged
  // batch reads it from the lengths, after the window loads are in flight)
  if (a.tail_cap > 0) load_tokens(0, a.tail_cap);
  if (a.balanced) {
    int share, first, len;
    batch_shares(a.packed_len, a.max_packed_len, gridDim.z, a.n_wg, share, first, len);
    S = __shfl(share, b);
  }
  load_splits(0);
  const int T = a.tail_len ? min(max(a.tail_len[b], 0), a.tail_cap) : a.nw.T;

  // ---- packed partials: online over passes ----
  float mp = -INFINITY, lp = 0.f;
  float4_t xp = {0.f, 0.f, 0.f, 0.f};
  for (int j0 = 0; j0 < S; j0 += kSplitPass) {
    if (j0 != 0) load_splits(j0);
    float mloc = -INFINITY;
#pragma unroll
    for (int u = 0; u < kCmbSplits; ++u)
      if (elem(j0, u) < S) mloc = fmaxf(mloc, ml[u][0]);
    const float mnew = fmaxf(mp, row_reduce16<true>(mloc));
    if (mnew != -INFINITY) {
      const float sc = part_weight(mp, mnew);
      xp *= sc;
      lp *= sc;
#pragma unroll
      for (int u = 0; u < kCmbSplits; ++u) {
        // lanes past the sequence's splits re-read its last: select, not weight by 0;
        // a record is a mean over its split: weight l 2^(m - M)
        const bool ok = elem(j0, u) < S && ml[u][0] != -INFINITY;
        const float w = ok ? __builtin_amdgcn_exp2f(ml[u][0] - mnew) * ml[u][1] : 0.f;
        xp += ok ? w * pv[u] : float4_t{0.f, 0.f, 0.f, 0.f};
        lp = ok ? lp + w : lp;
      }
      mp = mnew;
    }
  }
  // ---- window: online over passes ----
  float mt = -INFINITY, lt = 0.f;
  float4_t xt = {0.f, 0.f, 0.f, 0.f};
  for (int t0 = 0; t0 < T; t0 += kTokenPass) {
    if (t0 != 0) load_tokens(t0, T);
    float mloc = -INFINITY;
#pragma unroll
    for (int u = 0; u < kTok; ++u)
      if (elem(t0, u) < T) mloc = fmaxf(mloc, ws[u]);
    const float mnew = fmaxf(mt, row_reduce16<true>(mloc));
    if (mnew != -INFINITY) {
      const float sc = part_weight(mt, mnew);
      xt *= sc;
      lt *= sc;
#pragma unroll
      for (int u = 0; u < kTok; ++u) {
        // a row given apart goes into the window buffer (once: by query 0's merge)
        if (r % a.G == 0 && elem(t0, u) < T && fresh_row(a.nw, elem(t0, u)) >= 0)
          *reinterpret_cast<uint2*>(a.nw.v_dst + (vb - a.v_tail) + (int64_t)elem(t0, u) * a.ts_t) = wv[u];
        const float w = elem(t0, u) < T ? __builtin_amdgcn_exp2f(ws[u] - mnew) : 0.f;
        const float4_t vf = a.tail_bf16
            ? float4_t{__uint_as_float(wv[u].x << 16), __uint_as_float(wv[u].x & 0xffff0000u),
                       __uint_as_float(wv[u].y << 16), __uint_as_float(wv[u].y & 0xffff0000u)}
            : float4_t{half_bits_to_float(wv[u].x & 0xffff), half_bits_to_float(wv[u].x >> 16),
                       half_bits_to_float(wv[u].y & 0xffff), half_bits_to_float(wv[u].y >> 16)};
        xt += w * vf;
        lt += w;
      }
      mt = mnew;
    }
  }
  // ---- row sums (every row holds all of the wave's splits and tokens, for
  // its 4 channels), then the waves meet in LDS: per wave (mp, lp, mt, lt)
  // and the 16 channels' packed and window sums ----
  __shared__ float s_m[kCmbWaves][4];
  __shared__ float4_t s_y[kCmbWaves][4], s_z[kCmbWaves][4];
  float4_t y, z;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    y[i] = row_reduce16<false>(xp[i]);
    z[i] = row_reduce16<false>(xt[i]);
  }
  lp = row_reduce16<false>(lp);
  lt = row_reduce16<false>(lt);
  if (p == 0) {
    s_y[wave][c4] = y;
    s_z[wave][c4] = z;
    if (c4 == 0) {
      s_m[wave][0] = mp;
      s_m[wave][1] = lp;
      s_m[wave][2] = mt;
      s_m[wave][3] = lt;
    }
  }
  __syncthreads();
  if (wave != 0) return;
  float Mp = -INFINITY, Mt = -INFINITY;
#pragma unroll
  for (int w = 0; w < kCmbWaves; ++w) {
    Mp = fmaxf(Mp, s_m[w][0]);
    Mt = fmaxf(Mt, s_m[w][2]);
  }
  lp = lt = 0.f;
  y = z = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int w = 0; w < kCmbWaves; ++w) {
    const float wp = part_weight(s_m[w][0], Mp), wt = part_weight(s_m[w][2], Mt);
    lp = __builtin_fmaf(wp, s_m[w][1], lp);
    lt = __builtin_fmaf(wt, s_m[w][3], lt);
    y += wp * s_y[w][c4];
    z += wt * s_z[w][c4];
  }
  if constexpr (kRotated) {
    // H16 over the chunk's channel c = 4 c4 + i: bits 0-1 in registers, bits 2-3
    // across rows; then sign and 1/(128 kappa)
#pragma unroll
    for (int hb = 1; hb < 4; hb <<= 1)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (!(i & hb)) {
          const float u = y[i], w = y[i | hb];
          y[i] = u + w;
          y[i | hb] = u - w;
        }
#pragma unroll
    for (int rb = 1; rb < 4; rb <<= 1)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float o = __shfl_xor(y[i], 16 * rb);
        y[i] = (c4 & rb) ? o - y[i] : y[i] + o;
      }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int cg = kChunk * ch + 4 * c4 + i;
      y[i] = (sign_neg(a.v_sign_bits, cg) ? -y[i] : y[i]) * a.packed_scale;
    }
  }
  if (p == 0) {
    const float M = fmaxf(Mp, Mt);
    const float wp = part_weight(Mp, M), wt = part_weight(Mt, M);
    const float inv = 1.0f / (lp * wp + lt * wt);
    float4_t o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = (y[i] * wp + z[i] * wt) * inv;
    store_o4(a.out, row * kD + kChunk * ch + 4 * c4, o, a.io_dtype);
  }
}

// The merge launch: the window in one pass when it holds more than 128 rows.
template <bool kRotated>
inline void launch_combine(const CombineKArgs& c, int rows, int batch, hipStream_t st) {
  const dim3 grid(kChunks, rows, batch);
  if (c.tail_cap > 16 * kCmbWaves * kCmbTokens)
    hipLaunchKernelGGL((combine_kernel<kRotated, 4>), grid, dim3(kCmbThreads), 0, st, c);
  else
    hipLaunchKernelGGL((combine_kernel<kRotated, kCmbTokens>), grid, dim3(kCmbThreads), 0, st, c);
}

}  // namespace bmx
