// Split-KV decode attention over packed k2b pages, gfx950.
//
// Work decomposition.  One workgroup of 8 waves per (split, sequence); wave w
// owns KV head w for the whole split, and all waves walk the same 64-token
// groups (4 pages, one key-scale group):
//   * the group's pages are copied HBM -> LDS with direct-to-LDS loads
//     (global_load_lds_dwordx4), one group ahead of the compute, so the HBM
//     stream is deep without holding prefetch data in VGPRs;
//   * the RoPE cos/sin of the group's 64 positions is produced once per
//     workgroup (angle-addition recurrence from an exact start, corrected to
//     HF's fp32 angle fl(inv_freq * pos)) and shared by all heads through LDS;
//   * per page and head the wave rebuilds K^T (128 ch x 16 tok) on MFMA
//     (8 x mfma_16x16x32(V_h tile, Us^T)), adds the 3-bit residual * scale and
//     applies RoPE in registers (lane 16q+n owns token n, channels 16b+4q+i, so
//     the RoPE pair (j, j+64) is lane-local), scores the G query heads on MFMA
//     (the score layout, lane 16q+g: tokens 4q..4q+3 of query g, is exactly the
//     B operand of P.V), runs a base-2 online softmax with the accumulator
//     rescaled only when a running max grows, and accumulates P*norm against
//     the codebook levels on MFMA, i.e. V stays in the Hadamard-rotated domain.
// One extra workgroup per sequence attends the fp16 recent window with the same
// MFMA shapes and maps its accumulator into the rotated domain (signs, then the
// unnormalised Hadamard), so every partial merges the same way.  The combine
// kernel merges the partials, applies the one inverse Hadamard per (head,
// query), the signs and the normalisation.
//
// Reference semantics: cache/triton_dequant_attention.py:863-1115 (kernel),
// 409-461 (merge), 324-360 (tail), 504-575 (finalize);
// cache/chunked_attention.py:398-530 (decode loop).

#include "k2b_common.h"

namespace bmx {

constexpr int kWaves = 8;                   // waves per workgroup; wave w = head w
constexpr int kThreads = 64 * kWaves;
constexpr int kGroupPages = kGroup / kPT;   // 4 pages per 64-token group
constexpr int kCsBytes = kGroupPages * 8 * 64 * 16;  // cos/sin of one group, lane order

struct DecodeKArgs {
  int h_kv, G, split_tokens, max_splits, max_pages, max_packed_len, n_pool, tail_cap;
  const float* q;
  float* ws_acc;   // [B][max_splits + 1][h_kv][G][128]; row max_splits = recent window
  float* ws_ml;    // [B][max_splits + 1][h_kv][G][2]
  const uint8_t* pages;
  const int32_t* page_table;
  const int32_t* packed_len;
  const uint16_t* basis;
  int64_t basis_stride;
  const uint16_t* k_tail;
  const uint16_t* v_tail;
  int64_t ts_b, ts_h, ts_t;
  const int32_t* tail_len;
  PageLayout L;
  float qscale;        // sm_scale * log2(e)
  float rope_scaling;
  float inv_freq[64];
  float step_c[64];    // cos / sin of 64 * inv_freq_j (exact angle), the per-group step
  float step_s[64];
  float step8_c[64];   // cos / sin of 8 * inv_freq_j, between a thread's positions
  float step8_s[64];
  float codebook[4];
  uint32_t v_sign_bits[4];
};

// s_waitcnt vmcnt(0) without waiting on LDS / export counters (gfx9 encoding).
__device__ __forceinline__ void wait_vmem_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

__device__ __forceinline__ void lds_dma16(const void* src, void* lds_dst) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds_dst, 16, 0, 0);
}

// Query fragments (B operand of the scores): chunk kk covers channels
// {32kk + 4q + i, 32kk + 16 + 4q + i}; column n is query n (zero when n >= G).
__device__ __forceinline__ void load_query(const DecodeKArgs& a, int b, int h, int n, int q,
                                           half8_t qf[4]) {
  const float* qrow = a.q + (((int64_t)b * a.h_kv + h) * a.G + (n < a.G ? n : 0)) * kD;
  const float sc = (n < a.G) ? a.qscale : 0.0f;
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      qf[kk][i] = (_Float16)(qrow[32 * kk + 4 * q + i] * sc);
      qf[kk][4 + i] = (_Float16)(qrow[32 * kk + 16 + 4 * q + i] * sc);
    }
  }
}

// Base-2 online softmax over the 4 scores of this lane (tokens 4q..4q+3 of
// query g); lanes of one query share the running max.  The common case (no
// score above the running max) costs a lane-local max and a wave vote; only
// when some max grows do the lanes exchange maxima and rescale.
__device__ __forceinline__ void softmax_step(const float4_t& s, float& m_run, float& l_run,
                                             float4_t acc[8], float p[4]) {
  float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
  if (__any(mx > m_run)) {
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    l_run *= alpha;
#pragma unroll
    for (int bt = 0; bt < 8; ++bt) acc[bt] *= alpha;
    m_run = m_new;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_exp2f(s[i] - m_run);
  l_run += (p[0] + p[1]) + (p[2] + p[3]);
}

// Partial (acc, m, l) of this lane's query into the workspace row.
__device__ __forceinline__ void store_partial(const DecodeKArgs& a, int b, int split, int h, int n,
                                              int q, const float4_t acc[8], float m_run,
                                              float l_run) {
  l_run += __shfl_xor(l_run, 16);
  l_run += __shfl_xor(l_run, 32);
  if (n < a.G) {
    const int64_t row = (((int64_t)b * (a.max_splits + 1) + split) * a.h_kv + h) * a.G + n;
    float* dst = a.ws_acc + row * kD;
#pragma unroll
    for (int bt = 0; bt < 8; ++bt) *reinterpret_cast<float4_t*>(dst + 16 * bt + 4 * q) = acc[bt];
    if (q == 0) *reinterpret_cast<float2*>(a.ws_ml + row * 2) = make_float2(m_run, l_run);
  }
}

// ---------------------------------------------------------------------------
// fp16 recent window (post-RoPE keys, plain values) of one sequence: wave =
// head; each wave double-buffers its own 16-token K and V tiles (row-major
// 16 x 256 B) in a private LDS slice with direct-to-LDS loads, so the loop
// needs no workgroup barrier.  Rows past the window re-read the last valid row
// and are masked out of the softmax.
// ---------------------------------------------------------------------------
constexpr int kTailSlice = 2 * 2 * kPT * kD * 2;  // 2 buffers x (K, V) tiles, bytes per wave

__device__ void tail_partial(const DecodeKArgs& a, uint8_t* smem, int b) {
  const int tid = threadIdx.x, h = tid >> 6, lane = tid & 63;
  const int n = lane & 15, q = lane >> 4;
  const int T = min(max(a.tail_len[b], 0), a.tail_cap);
  if (T == 0 || h >= a.h_kv) return;
  uint8_t* slice = smem + h * kTailSlice;
  const uint16_t* kt = a.k_tail + b * a.ts_b + h * a.ts_h;
  const uint16_t* vt = a.v_tail + b * a.ts_b + h * a.ts_h;
  // one wave instruction moves 4 rows (64 lanes x 16 B)
  auto issue_chunk = [&](int t0, int buf) {
    uint8_t* kdst = slice + buf * (2 * kPT * kD * 2);
    uint8_t* vdst = kdst + kPT * kD * 2;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = min(t0 + 4 * r + (lane >> 4), T - 1);
      const int64_t off = (int64_t)row * a.ts_t + (lane & 15) * 8;
      lds_dma16(kt + off, kdst + r * 1024);
      lds_dma16(vt + off, vdst + r * 1024);
    }
  };
  half8_t qf[4];
  load_query(a, b, h, n, q, qf);
  float4_t acc[8];
#pragma unroll
  for (int bt = 0; bt < 8; ++bt) acc[bt] = float4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;
  issue_chunk(0, 0);
  for (int t0 = 0, buf = 0; t0 < T; t0 += kPT, buf ^= 1) {
    wait_vmem_all();
    __builtin_amdgcn_wave_barrier();
    if (t0 + kPT < T) issue_chunk(t0 + kPT, buf ^ 1);
    const uint16_t* kst = reinterpret_cast<const uint16_t*>(slice + buf * (2 * kPT * kD * 2));
    const uint16_t* vst = kst + kPT * kD;
    float4_t s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      union { uint2 u[2]; half8_t v; } ka;
      ka.u[0] = *reinterpret_cast<const uint2*>(kst + n * kD + 32 * kk + 4 * q);
      ka.u[1] = *reinterpret_cast<const uint2*>(kst + n * kD + 32 * kk + 16 + 4 * q);
      s = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka.v, qf[kk], s, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (t0 + 4 * q + i >= T) s[i] = -INFINITY;
    float p[4];
    softmax_step(s, m_run, l_run, acc, p);
    half4_t pb = {(_Float16)p[0], (_Float16)p[1], (_Float16)p[2], (_Float16)p[3]};
#pragma unroll
    for (int bt = 0; bt < 8; ++bt) {
      union { uint16_t u[4]; half4_t v; } va;
#pragma unroll
      for (int i = 0; i < 4; ++i) va.u[i] = vst[(4 * q + i) * kD + 16 * bt + n];
      acc[bt] = __builtin_amdgcn_mfma_f32_16x16x16f16(va.v, pb, acc[bt], 0, 0, 0);
    }
    // every lane's reads of this buffer precede the next overwrite of it
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
  }
  // into the rotated domain: x = H (signs * acc), H the unnormalised Sylvester
  // Hadamard, channel c = 16bt + 4q + i (bits: i -> 0,1; q -> 2,3; bt -> 4,5,6)
#pragma unroll
  for (int bt = 0; bt < 8; ++bt)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (sign_neg(a.v_sign_bits, 16 * bt + 4 * q + i)) acc[bt][i] = -acc[bt][i];
#pragma unroll
  for (int bt = 0; bt < 8; ++bt) {
    const float4_t x = acc[bt];
    const float y0 = x[0] + x[1], y1 = x[0] - x[1], y2 = x[2] + x[3], y3 = x[2] - x[3];
    acc[bt] = float4_t{y0 + y2, y1 + y3, y0 - y2, y1 - y3};
  }
#pragma unroll
  for (int hb = 16; hb <= 32; hb <<= 1) {
#pragma unroll
    for (int bt = 0; bt < 8; ++bt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float o = __shfl_xor(acc[bt][i], hb);
        acc[bt][i] = (lane & hb) ? (o - acc[bt][i]) : (acc[bt][i] + o);
      }
  }
#pragma unroll
  for (int sb = 1; sb < 8; sb <<= 1)
#pragma unroll
    for (int bt = 0; bt < 8; ++bt)
      if (!(bt & sb)) {
        const float4_t u = acc[bt], w = acc[bt | sb];
        acc[bt] = u + w;
        acc[bt | sb] = u - w;
      }
  store_partial(a, b, a.max_splits, h, n, q, acc, m_run, l_run);
}

template <int R>
__global__ __launch_bounds__(kThreads) void k2b_decode_split_kernel(const DecodeKArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int n = lane & 15;   // token within page (K side) / query column (score side)
  const int q = lane >> 4;   // quarter
  const int split = blockIdx.x, b = blockIdx.y;
  // Balanced static partition of the sequence's work units over the max_splits
  // workgroups: units [0, NG) are 64-token packed groups, [NG, NG + TU) the fp16
  // recent window (64 tokens per unit), owned by the last workgroup.
  const int len = min(a.packed_len[b], a.max_packed_len) & ~(kGroup - 1);
  const int NG = len / kGroup;
  const int T = min(max(a.tail_len[b], 0), a.tail_cap);
  const int TU = (T + kGroup - 1) / kGroup;
  const int U = NG + TU;
  const int S = a.max_splits;
  const int g0 = min((int)(((int64_t)split * U) / S), NG);
  const int g1 = min((int)(((int64_t)(split + 1) * U) / S), NG);
  const bool own_tail = (split == S - 1) && TU > 0;
  const int n_groups = g1 - g0;
  const int t_begin = g0 * kGroup;
  const int C = kD * a.h_kv;
  const int pb = a.L.bytes;
  uint8_t* ring = smem;                                      // [2][4 pages]
  float4_t* cs = reinterpret_cast<float4_t*>(smem + 2 * kGroupPages * pb);
  const int32_t* ptab = a.page_table + (int64_t)b * a.max_pages + t_begin / kPT;
  const bool active = wave < a.h_kv;
  const int h = active ? wave : 0;
  if (n_groups == 0) {  // uniform: nothing packed here; an empty partial keeps the merge blind
    if (active) {
      float4_t zero[8];
#pragma unroll
      for (int bt = 0; bt < 8; ++bt) zero[bt] = float4_t{0.f, 0.f, 0.f, 0.f};
      store_partial(a, b, split, h, n, q, zero, -INFINITY, 0.f);
    }
    if (own_tail) tail_partial(a, smem, b);
    return;
  }

  // ---- group copy HBM -> LDS (1 KB per wave instruction) ----
  const int chunks_pp = (pb + 1023) >> 10;
  auto issue_group = [&](int gi, int slot) {
    uint8_t* dst0 = ring + slot * kGroupPages * pb;
    for (int c = wave; c < kGroupPages * chunks_pp; c += kWaves) {
      const int pp = c / chunks_pp, off = (c - pp * chunks_pp) << 10;
      const int64_t pid = clamp_page(ptab[gi * kGroupPages + pp], a.n_pool);
      if (off + lane * 16 < pb)
        lds_dma16(a.pages + pid * pb + off + lane * 16, dst0 + pp * pb + off);
    }
  };
  issue_group(0, 0);

  // ---- cos/sin recurrence state: this thread owns frequency j = tid & 63 at
  // group-local positions tl = wave + 8k, k < 8 ----
  const int fj = tid & 63;
  const float fq = a.inv_freq[fj];
  float cc[8], ss[8];
  {
    double sd, cd;  // one exact-angle start per thread, then 8-position steps
    sincos((double)fq * (double)(t_begin + wave), &sd, &cd);
    cc[0] = (float)cd;
    ss[0] = (float)sd;
    const float c8 = a.step8_c[fj], s8 = a.step8_s[fj];
#pragma unroll
    for (int k = 1; k < 8; ++k) {
      cc[k] = cc[k - 1] * c8 - ss[k - 1] * s8;
      ss[k] = ss[k - 1] * c8 + cc[k - 1] * s8;
    }
  }
  const float stc = a.step_c[fj], sts = a.step_s[fj];

  // ---- per-wave constants ----
  constexpr int KQ = R / 4;
  typedef _Float16 hvec_t __attribute__((ext_vector_type(KQ)));
  hvec_t vh[8];
  const uint16_t* basis = a.basis + (int64_t)b * a.basis_stride;
#pragma unroll
  for (int bt = 0; bt < 8; ++bt)
    vh[bt] = *reinterpret_cast<const hvec_t*>(basis + (int64_t)(h * kD + 16 * bt + n) * R + KQ * q);
  half8_t qf[4];
  load_query(a, b, h, n, q, qf);
  uint32_t cbh[2], cbl[2];
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    const _Float16 h0 = (_Float16)a.codebook[2 * w], h1 = (_Float16)a.codebook[2 * w + 1];
    cbh[w] = half_bits(h0) | (half_bits(h1) << 16);
    cbl[w] = half_bits((_Float16)(a.codebook[2 * w] - (float)h0)) |
             (half_bits((_Float16)(a.codebook[2 * w + 1] - (float)h1)) << 16);
  }
  float4_t acc[8];
#pragma unroll
  for (int bt = 0; bt < 8; ++bt) acc[bt] = float4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;

  for (int gi = 0; gi < n_groups; ++gi) {
    wait_vmem_all();   // this wave's copies of group gi have landed
    __syncthreads();   // ... and every wave's; slot (gi+1)&1 and cs are free again
    if (gi + 1 < n_groups) issue_group(gi + 1, (gi + 1) & 1);

    // cos/sin of fl32(inv_freq * pos) for the group's 64 positions
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int tl = wave + 8 * k;
      const float tf = (float)(t_begin + gi * kGroup + tl);
      const float ang = fq * tf;
      const float e = __builtin_fmaf(fq, tf, -ang);          // exact: fq*tf - ang
      const float e2 = 0.5f * e * e;
      const float c_hf = __builtin_fmaf(ss[k], e, __builtin_fmaf(-cc[k], e2, cc[k]));
      const float s_hf = __builtin_fmaf(-cc[k], e, __builtin_fmaf(-ss[k], e2, ss[k]));
      // lane-order slot: page p, lane 16*qq + nn, read r = 2*bt + (i >> 1), half i & 1
      const int p = tl >> 4, nn = tl & 15;
      const int bt = fj >> 4, qq = (fj >> 2) & 3, i = fj & 3;
      float2* dst = reinterpret_cast<float2*>(cs + (p * 8 + 2 * bt + (i >> 1)) * 64 + 16 * qq + nn);
      dst[i & 1] = make_float2(c_hf * a.rope_scaling, s_hf * a.rope_scaling);
      const float cn = cc[k] * stc - ss[k] * sts;
      ss[k] = ss[k] * stc + cc[k] * sts;
      cc[k] = cn;
    }
    __syncthreads();
    if (!active) continue;

    const uint8_t* grp = ring + (gi & 1) * kGroupPages * pb;
    // key-residual scales of the group: 8 runs of 4 channels from the pages' KSCALE
    _Float16 sc[32];
    {
      const int quarter = C / 4;
#pragma unroll
      for (int bt = 0; bt < 8; ++bt) {
        const int c0 = h * kD + 16 * bt + 4 * q;
        const int slot = c0 / quarter, off = c0 - slot * quarter;
        const uint2 raw = *reinterpret_cast<const uint2*>(grp + slot * pb + a.L.kscale + 2 * off);
        const uint16_t r4[4] = {(uint16_t)(raw.x & 0xffff), (uint16_t)(raw.x >> 16),
                                (uint16_t)(raw.y & 0xffff), (uint16_t)(raw.y >> 16)};
#pragma unroll
        for (int i = 0; i < 4; ++i) __builtin_memcpy(&sc[4 * bt + i], &r4[i], 2);
      }
    }
    for (int pp = 0; pp < kGroupPages; ++pp) {
      const uint8_t* page = grp + pp * pb;
      // ---- K^T tile on MFMA ----
      const hvec_t us = *reinterpret_cast<const hvec_t*>(page + a.L.us + n * (2 * R) + q * (2 * KQ));
      float4_t kt[8];
#pragma unroll
      for (int bt = 0; bt < 8; ++bt) {
        const float4_t z = {0.f, 0.f, 0.f, 0.f};
        if constexpr (R == 32)
          kt[bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh[bt], us, z, 0, 0, 0);
        else
          kt[bt] = __builtin_amdgcn_mfma_f32_16x16x16f16(vh[bt], us, z, 0, 0, 0);
      }
      // ---- residual ----
      {
        const uint32_t* kr = reinterpret_cast<const uint32_t*>(page + a.L.kres + h * 768 + lane * 12);
        const uint32_t w0 = kr[0], w1 = kr[1], w2 = kr[2];
#pragma unroll
        for (int k = 0; k < 32; ++k)
          kt[k >> 2][k & 3] = __builtin_fmaf((float)sc[k], (float)kres_code(w0, w1, w2, k), kt[k >> 2][k & 3]);
      }
      // ---- RoPE at read: channel j pairs with j+64 (tile bt with bt+4) ----
#pragma unroll
      for (int bt = 0; bt < 4; ++bt) {
        const float4_t c01 = cs[(pp * 8 + 2 * bt) * 64 + lane];
        const float4_t c23 = cs[(pp * 8 + 2 * bt + 1) * 64 + lane];
        const float cosv[4] = {c01[0], c01[2], c23[0], c23[2]};
        const float sinv[4] = {c01[1], c01[3], c23[1], c23[3]};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float k1 = kt[bt][i], k2 = kt[bt + 4][i];
          kt[bt][i] = k1 * cosv[i] - k2 * sinv[i];
          kt[bt + 4][i] = k2 * cosv[i] + k1 * sinv[i];
        }
      }
      // ---- scores on MFMA: S[token][query] ----
      float4_t s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        half8_t ka;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          ka[i] = (_Float16)kt[2 * kk][i];
          ka[4 + i] = (_Float16)kt[2 * kk + 1][i];
        }
        s = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qf[kk], s, 0, 0, 0);
      }
      float p[4];
      softmax_step(s, m_run, l_run, acc, p);
      // ---- P*norm (B operand: tokens 4q..4q+3 of query g, twice) ----
      const uint2 nr = *reinterpret_cast<const uint2*>(page + a.L.vnorm + h * 32 + q * 8);
      half8_t pb8;
      pb8[0] = (_Float16)(p[0] * half_bits_to_float(nr.x & 0xffff));
      pb8[1] = (_Float16)(p[1] * half_bits_to_float(nr.x >> 16));
      pb8[2] = (_Float16)(p[2] * half_bits_to_float(nr.y & 0xffff));
      pb8[3] = (_Float16)(p[3] * half_bits_to_float(nr.y >> 16));
      pb8[4] = pb8[0]; pb8[5] = pb8[1]; pb8[6] = pb8[2]; pb8[7] = pb8[3];
      // ---- V codes -> codebook head/remainder (A operand), rotated-domain P.V:
      // K index 8q+i pairs level-head(token 4q+i), 8q+4+i level-remainder ----
      const uint2 vc = *reinterpret_cast<const uint2*>(page + a.L.vcode + h * 512 + lane * 8);
#pragma unroll
      for (int bt = 0; bt < 8; ++bt) {
        const uint32_t D = bt < 4 ? vc.x : vc.y;
        const int bb = bt & 3;
        const uint32_t s01 = ((D >> (4 * bb)) & 0x00030003u) * 0x202u + 0x01000100u;
        const uint32_t s23 = ((D >> (4 * bb + 2)) & 0x00030003u) * 0x202u + 0x01000100u;
        union { uint32_t u[4]; half8_t v; } va;
        va.u[0] = __builtin_amdgcn_perm(cbh[1], cbh[0], s01);
        va.u[1] = __builtin_amdgcn_perm(cbh[1], cbh[0], s23);
        va.u[2] = __builtin_amdgcn_perm(cbl[1], cbl[0], s01);
        va.u[3] = __builtin_amdgcn_perm(cbl[1], cbl[0], s23);
        acc[bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va.v, pb8, acc[bt], 0, 0, 0);
      }
    }
  }
  if (active) store_partial(a, b, split, h, n, q, acc, m_run, l_run);
  if (own_tail) {
    __syncthreads();  // the tail stages its tiles in the LDS the groups used
    tail_partial(a, smem, b);
  }
}

struct CombineKArgs {
  int h_kv, G, max_splits, tail_cap;
  float* out;
  const float* ws_acc;
  const float* ws_ml;
  const int32_t* tail_len;
  uint32_t v_sign_bits[4];
};

constexpr int kCombineThreads = 512;
constexpr int kCombineStrides = kCombineThreads / 32;  // partial strides per channel quad

// One workgroup per (query, head, sequence).  Thread (channel quad cq, stride
// ps) sums partials ps, ps + 16, ... of its quad with every load issued before
// the first use; the 16 stride sums meet in LDS; one wave applies the inverse
// Hadamard, the signs and the normalisation.
__global__ __launch_bounds__(kCombineThreads) void k2b_combine_kernel(const CombineKArgs a) {
  const int g = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const bool has_tail = min(max(a.tail_len[b], 0), a.tail_cap) > 0;
  const int n_parts = a.max_splits + (has_tail ? 1 : 0);  // tail partial sits at index max_splits
  const int64_t row0 = ((int64_t)b * (a.max_splits + 1) * a.h_kv + h) * a.G + g;
  const int64_t rstride = (int64_t)a.h_kv * a.G;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  float* s_w = reinterpret_cast<float*>(smem);               // [max_splits + 1]
  float4_t* s_x = reinterpret_cast<float4_t*>(s_w + ((a.max_splits + 4) & ~3));  // [16][32]
  float* s_red = reinterpret_cast<float*>(s_x + kCombineStrides * 32);  // [16]
  // (1) running max, weights, denominator (threads over partials)
  float mx = -INFINITY;
  for (int i = tid; i < n_parts; i += kCombineThreads) mx = fmaxf(mx, a.ws_ml[(row0 + i * rstride) * 2]);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if (lane == 0) s_red[wave] = mx;
  __syncthreads();
  float m_star = s_red[0];
#pragma unroll
  for (int w = 1; w < kCombineThreads / 64; ++w) m_star = fmaxf(m_star, s_red[w]);
  float lsum = 0.f;
  for (int i = tid; i < n_parts; i += kCombineThreads) {
    const float2 ml = *reinterpret_cast<const float2*>(a.ws_ml + (row0 + i * rstride) * 2);
    const float w = __builtin_amdgcn_exp2f(ml.x - m_star);
    s_w[i] = w;
    lsum += ml.y * w;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) lsum += __shfl_xor(lsum, o);
  __syncthreads();
  if (lane == 0) s_red[8 + wave] = lsum;
  __syncthreads();
  // (2) weighted sum of the rotated accumulators
  {
    const int cq = tid & 31, ps = tid >> 5;
    const float* base = a.ws_acc + row0 * kD + 4 * cq;
    float4_t x = {0.f, 0.f, 0.f, 0.f};
    constexpr int kBatch = 16;
    for (int i0 = ps; i0 < n_parts; i0 += kBatch * kCombineStrides) {
      float4_t v[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int i = i0 + u * kCombineStrides;
        v[u] = i < n_parts ? *reinterpret_cast<const float4_t*>(base + (int64_t)i * rstride * kD)
                           : float4_t{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int i = i0 + u * kCombineStrides;
        if (i < n_parts) x += v[u] * s_w[i];
      }
    }
    s_x[ps * 32 + cq] = x;
  }
  __syncthreads();
  if (wave != 0) return;
  // lane holds channels 2*lane, 2*lane + 1
  float x0 = 0.f, x1 = 0.f;
#pragma unroll
  for (int ps = 0; ps < kCombineStrides; ++ps) {
    const float4_t v = s_x[ps * 32 + (lane >> 1)];
    x0 += (lane & 1) ? v[2] : v[0];
    x1 += (lane & 1) ? v[3] : v[1];
  }
  {
    const float y0 = x0 + x1, y1 = x0 - x1;
    x0 = y0; x1 = y1;
  }
#pragma unroll
  for (int hb = 1; hb < 64; hb <<= 1) {
    const float p0 = __shfl_xor(x0, hb), p1 = __shfl_xor(x1, hb);
    const bool upper = (lane & hb) != 0;
    x0 = upper ? (p0 - x0) : (x0 + p0);
    x1 = upper ? (p1 - x1) : (x1 + p1);
  }
  float l_tot = 0.f;
#pragma unroll
  for (int w = 0; w < kCombineThreads / 64; ++w) l_tot += s_red[8 + w];
  const float scale = 1.0f / ((float)kD * l_tot);
  const int c0 = 2 * lane, c1 = 2 * lane + 1;
  const float o0 = (sign_neg(a.v_sign_bits, c0) ? -x0 : x0) * scale;
  const float o1 = (sign_neg(a.v_sign_bits, c1) ? -x1 : x1) * scale;
  float* dst = a.out + (((int64_t)b * a.h_kv + h) * a.G + g) * kD;
  *reinterpret_cast<float2*>(dst + c0) = make_float2(o0, o1);
}

}  // namespace bmx

using namespace bmx;

static int device_cu_count() {
  static int n = 0;
  if (n == 0) {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0)
      n = cus;
    else
      n = 256;  // MI355X
  }
  return n;
}

// Workgroups per sequence: one wave of workgroups over the device's CUs (one
// 8-wave workgroup per CU), or as many as split_tokens asks for; never more
// than the sequence has 64-token work units.
static int choose_splits(const bmx_k2b_decode_args* a) {
  const int units = (a->max_packed_len + kGroup - 1) / kGroup + (a->tail_cap + kGroup - 1) / kGroup;
  int S;
  if (a->split_tokens > 0)
    S = (a->max_packed_len + a->tail_cap + a->split_tokens - 1) / a->split_tokens;
  else
    S = device_cu_count() / a->batch;
  if (S > units) S = units;
  return S < 1 ? 1 : S;
}

static size_t ws_bytes(const bmx_k2b_decode_args* a, int splits) {
  const size_t rows = (size_t)a->batch * (splits + 1) * a->geom.h_kv * a->geom.n_q_groups;
  return rows * (kD + 2) * sizeof(float);
}

extern "C" size_t bmx_k2b_decode_workspace_bytes(const bmx_k2b_decode_args* a) {
  if (!a || a->batch < 1) return 0;
  return ws_bytes(a, choose_splits(a));
}

static int fail(int code, const std::string& msg) {
  bmx_set_error(msg);
  return code;
}

template <int R>
static hipError_t launch_split(const DecodeKArgs& k, dim3 grid, size_t smem, hipStream_t st) {
  static size_t attr_bytes = 0;
  if (attr_bytes < smem) {
    hipError_t e = hipFuncSetAttribute((const void*)k2b_decode_split_kernel<R>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    if (e != hipSuccess) return e;
    attr_bytes = smem;
  }
  hipLaunchKernelGGL(k2b_decode_split_kernel<R>, grid, dim3(kThreads), smem, st, k);
  return hipGetLastError();
}

extern "C" int bmx_k2b_decode(const bmx_k2b_decode_args* a, void* stream) {
  if (!a) return fail(BMX_E_INVALID, "bmx_k2b_decode: args is NULL");
  const bmx_k2b_geom& g = a->geom;
  if (g.h_kv < 1 || g.h_kv > kWaves) return fail(BMX_E_INVALID, "bmx_k2b_decode: h_kv must be 1..8");
  if (g.rank != 16 && g.rank != 32) return fail(BMX_E_INVALID, "bmx_k2b_decode: rank must be 16 or 32");
  if (g.n_q_groups < 1 || g.n_q_groups > 16)
    return fail(BMX_E_INVALID, "bmx_k2b_decode: n_q_groups must be 1..16");
  if (a->batch < 1) return fail(BMX_E_INVALID, "bmx_k2b_decode: batch must be >= 1");
  if (a->max_packed_len < 0 || a->max_packed_len % kCodec != 0)
    return fail(BMX_E_INVALID, "bmx_k2b_decode: max_packed_len must be a multiple of 128");
  if (a->max_packed_len > 0 && a->max_pages * kPT < a->max_packed_len)
    return fail(BMX_E_INVALID, "bmx_k2b_decode: max_pages*16 < max_packed_len");
  if (a->tail_cap < 0 || a->tail_cap > 4096)
    return fail(BMX_E_INVALID, "bmx_k2b_decode: tail_cap must be 0..4096");
  if (a->split_tokens < 0 || a->split_tokens % kGroup != 0)
    return fail(BMX_E_INVALID, "bmx_k2b_decode: split_tokens must be a multiple of 64");
  if (!a->q || !a->out || !a->packed_len || !a->tail_len)
    return fail(BMX_E_INVALID, "bmx_k2b_decode: q/out/packed_len/tail_len must be non-NULL");
  if (a->max_packed_len > 0 && (!a->pages || !a->page_table || !a->basis))
    return fail(BMX_E_INVALID, "bmx_k2b_decode: pages/page_table/basis must be non-NULL");
  if (a->max_packed_len > 0 && a->n_pool_pages < 1)
    return fail(BMX_E_INVALID, "bmx_k2b_decode: n_pool_pages must be >= 1");
  if (a->tail_cap > 0 && (!a->k_tail || !a->v_tail))
    return fail(BMX_E_INVALID, "bmx_k2b_decode: k_tail/v_tail must be non-NULL when tail_cap > 0");
  if (a->tail_cap > 0 && (a->tail_stride_t % 8 != 0 || a->tail_stride_h % 8 != 0 ||
                          a->tail_stride_b % 8 != 0))
    return fail(BMX_E_INVALID, "bmx_k2b_decode: tail strides must be multiples of 8 elements");
  const int max_splits = choose_splits(a);
  const size_t need = ws_bytes(a, max_splits);
  if (max_splits + 1 > 8192)
    return fail(BMX_E_INVALID, "bmx_k2b_decode: more than 8191 splits; use a larger split_tokens");
  if (!a->workspace || a->workspace_bytes < need)
    return fail(BMX_E_WORKSPACE, "bmx_k2b_decode: workspace missing or smaller than "
                                 "bmx_k2b_decode_workspace_bytes()");
  hipStream_t st = (hipStream_t)stream;
  const size_t rows = (size_t)a->batch * (max_splits + 1) * g.h_kv * g.n_q_groups;
  float* ws_acc = (float*)a->workspace;
  float* ws_ml = ws_acc + rows * kD;
  const float qscale = a->sm_scale * 1.4426950408889634f;

  DecodeKArgs k{};
  k.h_kv = g.h_kv; k.G = g.n_q_groups; k.split_tokens = 0;
  k.max_splits = max_splits; k.max_pages = a->max_pages;
  k.max_packed_len = a->max_packed_len; k.n_pool = a->n_pool_pages > 0 ? a->n_pool_pages : 1;
  k.tail_cap = a->tail_cap;
  k.q = a->q; k.ws_acc = ws_acc; k.ws_ml = ws_ml;
  k.pages = a->pages; k.page_table = a->page_table; k.packed_len = a->packed_len;
  k.basis = a->basis; k.basis_stride = a->basis_stride;
  k.k_tail = a->k_tail; k.v_tail = a->v_tail;
  k.ts_b = a->tail_stride_b; k.ts_h = a->tail_stride_h; k.ts_t = a->tail_stride_t;
  k.tail_len = a->tail_len;
  k.L = PageLayout::make(g.h_kv, g.rank);
  k.qscale = qscale; k.rope_scaling = a->rope_scaling;
  for (int j = 0; j < 64; ++j) {
    k.inv_freq[j] = a->inv_freq[j];
    const double step = 64.0 * (double)a->inv_freq[j];  // exact: 64 * fp32
    k.step_c[j] = (float)cos(step);
    k.step_s[j] = (float)sin(step);
    k.step8_c[j] = (float)cos(step / 8.0);
    k.step8_s[j] = (float)sin(step / 8.0);
  }
  for (int j = 0; j < 4; ++j) { k.codebook[j] = a->codebook[j]; k.v_sign_bits[j] = a->v_sign_bits[j]; }
  const size_t smem = (size_t)2 * kGroupPages * k.L.bytes + kCsBytes;
  const size_t tail_smem = (size_t)kWaves * kTailSlice;
  const size_t smem_all = smem > tail_smem ? smem : tail_smem;
  dim3 grid(max_splits + 1, a->batch);
  hipError_t e = g.rank == 32 ? launch_split<32>(k, grid, smem_all, st)
                              : launch_split<16>(k, grid, smem_all, st);
  if (e != hipSuccess)
    return fail(BMX_E_HIP, std::string("bmx_k2b_decode: split kernel launch: ") + hipGetErrorString(e));
  if (a->split_end_event) {
    e = hipEventRecord((hipEvent_t)a->split_end_event, st);
    if (e != hipSuccess)
      return fail(BMX_E_HIP, std::string("bmx_k2b_decode: hipEventRecord: ") + hipGetErrorString(e));
  }
  CombineKArgs c{};
  c.h_kv = g.h_kv; c.G = g.n_q_groups;
  c.max_splits = max_splits; c.tail_cap = a->tail_cap;
  c.out = a->out; c.ws_acc = ws_acc; c.ws_ml = ws_ml;
  c.tail_len = a->tail_len;
  for (int j = 0; j < 4; ++j) c.v_sign_bits[j] = a->v_sign_bits[j];
  const size_t csmem = (size_t)(((max_splits + 4) & ~3) + kCombineStrides * 32 * 4 + 16) * sizeof(float);
  hipLaunchKernelGGL(k2b_combine_kernel, dim3(g.n_q_groups, g.h_kv, a->batch), dim3(kCombineThreads),
                     csmem, st, c);
  e = hipGetLastError();
  if (e != hipSuccess)
    return fail(BMX_E_HIP, std::string("bmx_k2b_decode: combine kernel launch: ") + hipGetErrorString(e));
  return BMX_OK;
}
