// Split-KV decode attention over packed k2b pages, gfx950.
//
// Work decomposition: one workgroup per (split, sequence) with one wave per KV
// head; every wave of the group walks the same 16-token pages, so the RoPE
// cos/sin of a page is computed once per workgroup (LDS) and shared by all
// heads.  Per page and head the wave
//   1. rebuilds K^T (128 ch x 16 tok) on MFMA: 8 x mfma_16x16x32(V_h tile, Us^T),
//   2. adds the 3-bit residual * group scale and applies RoPE in registers
//      (lane 16q+n owns token n, channels 16b+4q+i, so the RoPE pair (j, j+64)
//      is lane-local),
//   3. scores the G query heads on MFMA (keys in fp16 as the A operand); the
//      result layout (lane 16q+g: tokens 4q..4q+3 of query g) is exactly the
//      B-operand layout of the P.V product, so no transpose is needed,
//   4. runs the online softmax in base 2 (scores pre-scaled by log2 e),
//   5. accumulates P*norm against the raw codebook values on MFMA
//      (16x16x16), i.e. V stays in the Hadamard-rotated domain.
// The combine kernel merges the split partials with the fp16 recent window,
// applies the one inverse Hadamard per (head, query) and the V signs.
//
// Reference semantics: cache/triton_dequant_attention.py:863-1115 (kernel),
// 409-461 (merge), 324-360 (tail), 504-575 (finalize).

#include "k2b_common.h"

namespace bmx {

struct DecodeKArgs {
  int h_kv, G, split_tokens, max_splits, max_pages, max_packed_len, n_pool;
  const float* q;
  float* ws_acc;   // [B][max_splits][h_kv][G][128]
  float* ws_ml;    // [B][max_splits][h_kv][G][2]
  const uint8_t* pages;
  const int32_t* page_table;
  const int32_t* packed_len;
  const uint16_t* basis;
  int64_t basis_stride;
  PageLayout L;
  float qscale;        // sm_scale * log2(e)
  float rope_scaling;
  float inv_freq[64];
  float codebook[4];
};

constexpr int kCsStride = 66;  // float2 per token row of the cos/sin tile (padded)

template <int R, int MAXT>
__global__ __launch_bounds__(MAXT) void k2b_decode_split_kernel(const DecodeKArgs a) {
  const int h = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int n = lane & 15;   // token within page (K side) / query column (score side)
  const int q = lane >> 4;   // quarter
  const int split = blockIdx.x;
  const int b = blockIdx.y;
  const int len = min(a.packed_len[b], a.max_packed_len) & ~(kGroup - 1);
  const int t_begin = split * a.split_tokens;
  if (t_begin >= len) return;  // uniform over the workgroup, before any barrier
  const int t_end = min(len, t_begin + a.split_tokens);
  const int C = kD * a.h_kv;

  __shared__ float2 cs[kPT][kCsStride];

  // Frozen basis fragments (A operand of the K rebuild): tile bt = channels
  // 16bt..16bt+15 of head h, lane holds row n, ranks [kq*q, kq*q + kq).
  constexpr int KQ = R / 4;  // rank elements per lane per tile (8 or 4)
  const uint16_t* basis = a.basis + (int64_t)b * a.basis_stride;
  typedef _Float16 hvec_t __attribute__((ext_vector_type(KQ)));
  hvec_t vh[8];
#pragma unroll
  for (int bt = 0; bt < 8; ++bt) {
    const int row = h * kD + 16 * bt + n;
    vh[bt] = *reinterpret_cast<const hvec_t*>(basis + (int64_t)row * R + KQ * q);
  }

  // Query fragments (B operand of the scores): chunk kk covers channels
  // {32kk + 4q + i, 32kk + 16 + 4q + i}; column n is query n (zero if n >= G).
  half8_t qf[4];
  {
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

  // Codebook LUTs for v_perm: level k at bytes (2k, 2k+1) of {w1:w0}.  Each fp32
  // level is split into fp16 head + fp16 remainder (both multiplied by the same
  // P*norm in one K=32 MFMA), so the codebook keeps ~22 bits: a rounded level
  // would bias every rotated coordinate the same way and not average out.
  uint32_t cbh[2], cbl[2];
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    const _Float16 h0 = (_Float16)a.codebook[2 * w], h1 = (_Float16)a.codebook[2 * w + 1];
    const _Float16 l0 = (_Float16)(a.codebook[2 * w] - (float)h0);
    const _Float16 l1 = (_Float16)(a.codebook[2 * w + 1] - (float)h1);
    cbh[w] = half_bits(h0) | (half_bits(h1) << 16);
    cbl[w] = half_bits(l0) | (half_bits(l1) << 16);
  }

  float4_t acc[8];
#pragma unroll
  for (int bt = 0; bt < 8; ++bt) acc[bt] = float4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;
  float sc[32];
  int cur_group = -1;

  const int32_t* ptab = a.page_table + (int64_t)b * a.max_pages;
  const int nthreads = blockDim.x;

  for (int t0 = t_begin; t0 < t_end; t0 += kPT) {
    const int lp = t0 / kPT;
    const uint8_t* page = a.pages + clamp_page(ptab[lp], a.n_pool) * a.L.bytes;

    // ---- RoPE cos/sin of this page, shared by all heads ----
    __syncthreads();
    for (int idx = threadIdx.x; idx < kPT * 64; idx += nthreads) {
      const int tok = idx >> 6, j = idx & 63;
      const float ang = a.inv_freq[j] * (float)(t0 + tok);
      float s, c;
      sincosf(ang, &s, &c);
      cs[tok][j] = make_float2(c * a.rope_scaling, s * a.rope_scaling);
    }
    __syncthreads();

    // ---- key-residual scales of this 64-token group (8 runs of 4 channels) ----
    const int grp = t0 / kGroup;
    if (grp != cur_group) {
      cur_group = grp;
      const int quarter = C / 4;
#pragma unroll
      for (int bt = 0; bt < 8; ++bt) {
        const int c0 = h * kD + 16 * bt + 4 * q;
        const int slot = c0 / quarter, off = c0 % quarter;
        const uint8_t* sp = a.pages + clamp_page(ptab[grp * 4 + slot], a.n_pool) * a.L.bytes + a.L.kscale;
        const uint2 raw = *reinterpret_cast<const uint2*>(sp + 2 * off);
        sc[4 * bt + 0] = half_bits_to_float(raw.x & 0xffff);
        sc[4 * bt + 1] = half_bits_to_float(raw.x >> 16);
        sc[4 * bt + 2] = half_bits_to_float(raw.y & 0xffff);
        sc[4 * bt + 3] = half_bits_to_float(raw.y >> 16);
      }
    }

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
        kt[k >> 2][k & 3] += sc[k] * (float)kres_code(w0, w1, w2, k);
    }

    // ---- RoPE at read: channel j pairs with j+64 (tile bt with bt+4) ----
#pragma unroll
    for (int bt = 0; bt < 4; ++bt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float2 c = cs[n][16 * bt + 4 * q + i];
        const float k1 = kt[bt][i], k2 = kt[bt + 4][i];
        kt[bt][i] = k1 * c.x - k2 * c.y;
        kt[bt + 4][i] = k2 * c.x + k1 * c.y;
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
    // lane (g = n, q): s[i] = log2-domain score of token t0 + 4q + i for query g

    // ---- online softmax (base 2) ----
    float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    m_run = m_new;
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_exp2f(s[i] - m_new);
    l_run = l_run * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
#pragma unroll
    for (int bt = 0; bt < 8; ++bt) acc[bt] *= alpha;

    // ---- P*norm (B operand: tokens 4q..4q+3 of query g) ----
    const uint2 nr = *reinterpret_cast<const uint2*>(page + a.L.vnorm + h * 32 + q * 8);
    half8_t pb;
    pb[0] = (_Float16)(p[0] * half_bits_to_float(nr.x & 0xffff));
    pb[1] = (_Float16)(p[1] * half_bits_to_float(nr.x >> 16));
    pb[2] = (_Float16)(p[2] * half_bits_to_float(nr.y & 0xffff));
    pb[3] = (_Float16)(p[3] * half_bits_to_float(nr.y >> 16));
    pb[4] = pb[0]; pb[5] = pb[1]; pb[6] = pb[2]; pb[7] = pb[3];

    // ---- V codes -> codebook head/remainder (A operand), rotated-domain P.V:
    // K index 8q+i pairs level-head(token 4q+i) and 8q+4+i level-remainder(token
    // 4q+i) with the same P*norm ----
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
      acc[bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va.v, pb, acc[bt], 0, 0, 0);
    }
  }

  // ---- partials: lane (g = n, q) holds channels 16bt + 4q + i ----
  l_run += __shfl_xor(l_run, 16);
  l_run += __shfl_xor(l_run, 32);
  if (n < a.G) {
    const int64_t row = (((int64_t)b * a.max_splits + split) * a.h_kv + h) * a.G + n;
    float* dst = a.ws_acc + row * kD;
#pragma unroll
    for (int bt = 0; bt < 8; ++bt)
      *reinterpret_cast<float4_t*>(dst + 16 * bt + 4 * q) = acc[bt];
    if (q == 0) {
      a.ws_ml[row * 2 + 0] = m_run;
      a.ws_ml[row * 2 + 1] = l_run;
    }
  }
}

struct CombineKArgs {
  int h_kv, G, split_tokens, max_splits, tail_cap, max_packed_len;
  const float* q;
  float* out;
  const float* ws_acc;
  const float* ws_ml;
  const int32_t* packed_len;
  const uint16_t* k_tail;
  const uint16_t* v_tail;
  int64_t ts_b, ts_h, ts_t;
  const int32_t* tail_len;
  float qscale;
  uint32_t v_sign_bits[4];
};

// One workgroup (4 waves) per (head, sequence): fp16 tail partial, merge of the
// split partials (lanes run over splits, so the merge is not a serial chain),
// inverse Hadamard, signs, normalisation.
__global__ __launch_bounds__(256) void k2b_combine_kernel(const CombineKArgs a) {
  const int h = blockIdx.x, b = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int G = a.G;
  const int T = min(max(a.tail_len[b], 0), a.tail_cap);
  const int len = min(a.packed_len[b], a.max_packed_len) & ~(kGroup - 1);
  const int n_splits = (len + a.split_tokens - 1) / a.split_tokens;
  extern __shared__ float smem[];
  float* s_p = smem;                           // [G][tail_cap] tail scores -> weights
  float* s_w = s_p + G * a.tail_cap;           // [G][max_splits] split weights
  float* s_x = s_w + G * a.max_splits;         // [G][128] merged rotated accumulator
  float* s_lt = s_x + G * kD;                  // [16] total denominator

  const uint16_t* kt = a.k_tail + b * a.ts_b + h * a.ts_h;
  const uint16_t* vt = a.v_tail + b * a.ts_b + h * a.ts_h;
  const float* qh = a.q + ((int64_t)b * a.h_kv + h) * G * kD;
  const int64_t row0 = ((int64_t)b * a.max_splits * a.h_kv + h) * G;  // row of split 0, query 0
  const int64_t srow = (int64_t)a.h_kv * G;                          // row stride per split

  // (1) tail scores: wave per token, lanes over channel pairs
  for (int t = wave; t < T; t += 4) {
    const uint32_t kw = *reinterpret_cast<const uint32_t*>(kt + t * a.ts_t + 2 * lane);
    const float k0 = half_bits_to_float(kw & 0xffff), k1 = half_bits_to_float(kw >> 16);
    for (int g = 0; g < G; ++g) {
      float v = qh[g * kD + 2 * lane] * k0 + qh[g * kD + 2 * lane + 1] * k1;
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
      if (lane == 0) s_p[g * a.tail_cap + t] = v * a.qscale;
    }
  }
  __syncthreads();
  // (2) per query: tail statistics, split weights, denominator
  for (int g = wave; g < G; g += 4) {
    float mt = -INFINITY;
    for (int t = lane; t < T; t += 64) mt = fmaxf(mt, s_p[g * a.tail_cap + t]);
    float ms = -INFINITY;
    for (int s = lane; s < n_splits; s += 64) ms = fmaxf(ms, a.ws_ml[(row0 + s * srow + g) * 2]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      mt = fmaxf(mt, __shfl_xor(mt, o));
      ms = fmaxf(ms, __shfl_xor(ms, o));
    }
    const float m_star = fmaxf(mt, ms);
    float lt = 0.f;
    for (int t = lane; t < T; t += 64) {
      const float pv = __builtin_amdgcn_exp2f(s_p[g * a.tail_cap + t] - m_star);
      s_p[g * a.tail_cap + t] = pv;
      lt += pv;
    }
    float ls = 0.f;
    for (int s = lane; s < n_splits; s += 64) {
      const float2 ml = *reinterpret_cast<const float2*>(a.ws_ml + (row0 + s * srow + g) * 2);
      const float w = __builtin_amdgcn_exp2f(ml.x - m_star);
      s_w[g * a.max_splits + s] = w;
      ls += ml.y * w;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      lt += __shfl_xor(lt, o);
      ls += __shfl_xor(ls, o);
    }
    if (lane == 0) s_lt[g] = lt + ls;
  }
  __syncthreads();
  // (3) merged rotated accumulator: threads over (query, channel pair), four
  // independent partial sums over splits
  for (int e = tid; e < G * (kD / 2); e += 256) {
    const int g = e / (kD / 2), c = 2 * (e % (kD / 2));
    const float* base = a.ws_acc + (row0 + g) * kD + c;
    const float* w = s_w + g * a.max_splits;
    float2 x0 = make_float2(0.f, 0.f), x1 = x0, x2 = x0, x3 = x0;
    int s = 0;
    for (; s + 4 <= n_splits; s += 4) {
      const float2 v0 = *reinterpret_cast<const float2*>(base + (s + 0) * srow * kD);
      const float2 v1 = *reinterpret_cast<const float2*>(base + (s + 1) * srow * kD);
      const float2 v2 = *reinterpret_cast<const float2*>(base + (s + 2) * srow * kD);
      const float2 v3 = *reinterpret_cast<const float2*>(base + (s + 3) * srow * kD);
      x0.x += v0.x * w[s]; x0.y += v0.y * w[s];
      x1.x += v1.x * w[s + 1]; x1.y += v1.y * w[s + 1];
      x2.x += v2.x * w[s + 2]; x2.y += v2.y * w[s + 2];
      x3.x += v3.x * w[s + 3]; x3.y += v3.y * w[s + 3];
    }
    for (; s < n_splits; ++s) {
      const float2 v0 = *reinterpret_cast<const float2*>(base + s * srow * kD);
      x0.x += v0.x * w[s]; x0.y += v0.y * w[s];
    }
    s_x[g * kD + c] = (x0.x + x1.x) + (x2.x + x3.x);
    s_x[g * kD + c + 1] = (x0.y + x1.y) + (x2.y + x3.y);
  }
  __syncthreads();
  // (4) per query: inverse Hadamard, signs, tail values, normalise.  Lane holds
  // channels c0 = 2*lane, c1 = 2*lane + 1.
  for (int g = wave; g < G; g += 4) {
    float x0 = s_x[g * kD + 2 * lane], x1 = s_x[g * kD + 2 * lane + 1];
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
    float t0v = 0.f, t1v = 0.f;
    for (int t = 0; t < T; ++t) {
      const float pw = s_p[g * a.tail_cap + t];
      const uint32_t vw = *reinterpret_cast<const uint32_t*>(vt + t * a.ts_t + 2 * lane);
      t0v += pw * half_bits_to_float(vw & 0xffff);
      t1v += pw * half_bits_to_float(vw >> 16);
    }
    const int c0 = 2 * lane, c1 = 2 * lane + 1;
    const float inv_d = 1.0f / (float)kD;
    const float inv_l = 1.0f / s_lt[g];
    const float o0 = ((sign_neg(a.v_sign_bits, c0) ? -x0 : x0) * inv_d + t0v) * inv_l;
    const float o1 = ((sign_neg(a.v_sign_bits, c1) ? -x1 : x1) * inv_d + t1v) * inv_l;
    float* dst = a.out + (((int64_t)b * a.h_kv + h) * G + g) * kD;
    *reinterpret_cast<float2*>(dst + c0) = make_float2(o0, o1);
  }
}

}  // namespace bmx

using namespace bmx;

static int choose_split_tokens(const bmx_k2b_decode_args* a) {
  if (a->split_tokens > 0) return a->split_tokens;
  const int units = (a->max_packed_len + kGroup - 1) / kGroup;  // 64-token units per seq
  const long target_wgs = 512;
  long per = (long)units * a->batch / target_wgs;
  if (per < 2) per = 2;
  if (per > 32) per = 32;
  return (int)per * kGroup;
}

static size_t ws_bytes(const bmx_k2b_decode_args* a, int split_tokens, int* max_splits) {
  const int ms = (a->max_packed_len + split_tokens - 1) / split_tokens;
  if (max_splits) *max_splits = ms;
  const size_t rows = (size_t)a->batch * (ms > 0 ? ms : 1) * a->geom.h_kv * a->geom.n_q_groups;
  return rows * (kD + 2) * sizeof(float);
}

extern "C" size_t bmx_k2b_decode_workspace_bytes(const bmx_k2b_decode_args* a) {
  if (!a) return 0;
  return ws_bytes(a, choose_split_tokens(a), nullptr);
}

static int fail(int code, const std::string& msg) {
  bmx_set_error(msg);
  return code;
}

extern "C" int bmx_k2b_decode(const bmx_k2b_decode_args* a, void* stream) {
  if (!a) return fail(BMX_E_INVALID, "bmx_k2b_decode: args is NULL");
  const bmx_k2b_geom& g = a->geom;
  if (g.h_kv < 1 || g.h_kv > 16) return fail(BMX_E_INVALID, "bmx_k2b_decode: h_kv must be 1..16");
  if (g.rank != 16 && g.rank != 32) return fail(BMX_E_INVALID, "bmx_k2b_decode: rank must be 16 or 32");
  if (g.n_q_groups < 1 || g.n_q_groups > 16)
    return fail(BMX_E_INVALID, "bmx_k2b_decode: n_q_groups must be 1..16");
  if (a->batch < 1) return fail(BMX_E_INVALID, "bmx_k2b_decode: batch must be >= 1");
  if (a->max_packed_len < 0 || a->max_packed_len % kCodec != 0)
    return fail(BMX_E_INVALID, "bmx_k2b_decode: max_packed_len must be a multiple of 128");
  if (a->max_packed_len > 0 && a->max_pages * kPT < a->max_packed_len)
    return fail(BMX_E_INVALID, "bmx_k2b_decode: max_pages*16 < max_packed_len");
  if (a->tail_cap < 0 || a->tail_cap > 1024 || a->tail_cap * g.n_q_groups > 8192)
    return fail(BMX_E_INVALID, "bmx_k2b_decode: tail_cap must be <= 1024 and tail_cap*G <= 8192");
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
  const int split_tokens = choose_split_tokens(a);
  int max_splits = 0;
  const size_t need = ws_bytes(a, split_tokens, &max_splits);
  if ((size_t)g.n_q_groups * (a->tail_cap + max_splits + kD) + 64 > 16384)
    return fail(BMX_E_INVALID, "bmx_k2b_decode: G*(tail_cap + splits + 128) exceeds the "
                               "combine kernel's 64 KB of LDS; use a larger split_tokens");
  if (!a->workspace || a->workspace_bytes < need)
    return fail(BMX_E_WORKSPACE, "bmx_k2b_decode: workspace missing or smaller than "
                                 "bmx_k2b_decode_workspace_bytes()");
  hipStream_t st = (hipStream_t)stream;
  const size_t rows = (size_t)a->batch * (max_splits > 0 ? max_splits : 1) * g.h_kv * g.n_q_groups;
  float* ws_acc = (float*)a->workspace;
  float* ws_ml = ws_acc + rows * kD;
  const float qscale = a->sm_scale * 1.4426950408889634f;

  if (max_splits > 0) {
    DecodeKArgs k{};
    k.h_kv = g.h_kv; k.G = g.n_q_groups; k.split_tokens = split_tokens;
    k.max_splits = max_splits; k.max_pages = a->max_pages;
    k.max_packed_len = a->max_packed_len; k.n_pool = a->n_pool_pages;
    k.q = a->q; k.ws_acc = ws_acc; k.ws_ml = ws_ml;
    k.pages = a->pages; k.page_table = a->page_table; k.packed_len = a->packed_len;
    k.basis = a->basis; k.basis_stride = a->basis_stride;
    k.L = PageLayout::make(g.h_kv, g.rank);
    k.qscale = qscale; k.rope_scaling = a->rope_scaling;
    for (int j = 0; j < 64; ++j) k.inv_freq[j] = a->inv_freq[j];
    for (int j = 0; j < 4; ++j) k.codebook[j] = a->codebook[j];
    dim3 grid(max_splits, a->batch), block(64 * g.h_kv);
    // a workgroup of h_kv waves; <= 8 waves lets each wave hold 256 VGPRs
    if (g.rank == 32) {
      if (g.h_kv <= 8) hipLaunchKernelGGL((k2b_decode_split_kernel<32, 512>), grid, block, 0, st, k);
      else hipLaunchKernelGGL((k2b_decode_split_kernel<32, 1024>), grid, block, 0, st, k);
    } else {
      if (g.h_kv <= 8) hipLaunchKernelGGL((k2b_decode_split_kernel<16, 512>), grid, block, 0, st, k);
      else hipLaunchKernelGGL((k2b_decode_split_kernel<16, 1024>), grid, block, 0, st, k);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
      return fail(BMX_E_HIP, std::string("bmx_k2b_decode: split kernel launch: ") + hipGetErrorString(e));
  }
  if (a->split_end_event) {
    hipError_t e = hipEventRecord((hipEvent_t)a->split_end_event, st);
    if (e != hipSuccess)
      return fail(BMX_E_HIP, std::string("bmx_k2b_decode: hipEventRecord: ") + hipGetErrorString(e));
  }
  CombineKArgs c{};
  c.h_kv = g.h_kv; c.G = g.n_q_groups; c.split_tokens = split_tokens;
  c.max_splits = max_splits > 0 ? max_splits : 1; c.tail_cap = a->tail_cap > 0 ? a->tail_cap : 1;
  c.max_packed_len = a->max_packed_len;
  c.q = a->q; c.out = a->out; c.ws_acc = ws_acc; c.ws_ml = ws_ml;
  c.packed_len = a->packed_len; c.k_tail = a->k_tail; c.v_tail = a->v_tail;
  c.ts_b = a->tail_stride_b; c.ts_h = a->tail_stride_h; c.ts_t = a->tail_stride_t;
  c.tail_len = a->tail_len; c.qscale = qscale;
  for (int j = 0; j < 4; ++j) c.v_sign_bits[j] = a->v_sign_bits[j];
  const size_t smem = (size_t)(g.n_q_groups * (c.tail_cap + c.max_splits + kD) + 64) * sizeof(float);
  hipLaunchKernelGGL(k2b_combine_kernel, dim3(g.h_kv, a->batch), dim3(256), smem, st, c);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail(BMX_E_HIP, std::string("bmx_k2b_decode: combine kernel launch: ") + hipGetErrorString(e));
  return BMX_OK;
}
