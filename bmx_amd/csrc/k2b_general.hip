// The k2b path on the general page (include/bmx_k2b.h): head_dim 32, 64 or
// 128, rank 16..128, residual group 16..128 tokens, 2..4-bit keys, gfx950.
//
// Write (quantize-on-append), three launches per call as for the recipe's page:
//   gen_us_kernel    Us = M * basis32 (or the first codec page's SVD factor), fp16
//   gen_kres_kernel  R = M - Us16 * basis16^T, per-channel RTN over group tokens
//   gen_v_kernel     per (token, head): fp16 norm, sign flip, FWHT, Lloyd codes
// Read:
//   gen_split_kernel one workgroup per (split, head, sequence): every 16-token
//                    page of the split rebuilt on MFMA (K^T = basis * Us^T),
//                    residual and RoPE in registers (cos and sin of HF's fp32
//                    angle times rope_scaling, rounded to fp16: the
//                    reference's shared tables), scores K^T Q^T on MFMA,
//                    online softmax, P V on MFMA in the rotated value domain
//   gen_merge_kernel one workgroup per (query, head, sequence): the splits'
//                    partials, the inverse Hadamard, the recent window
//   gen_dequant_kernel  dense keys and values of committed pages (prefill)
// Reference semantics: cache/packed_streaming.py:475-580 and 957-1060,
// cache/codecs.py:616-649, 677-695, 786-796, quant/rtn.py:23-44,
// quant/hadamard.py:12-33, cache/triton_dequant_attention.py:1232-1368.
// Element-wise write steps follow the reference's operation order (divide,
// round-half-even, divide-then-multiply by sqrt(d)); this file is built without
// floating-point contraction.

#include <algorithm>
#include <string>

#include "decode_shared.h"
#include "k2b_general.h"

namespace bmx {

struct GenAppendArgs {
  GenLayout L;
  const uint16_t* k_pre;
  int64_t ksh, kst;
  const void* v;
  int64_t vsh, vst;
  int v_dtype;
  const float* basis32;
  const uint16_t* basis16;
  const float* us_first;
  float codebook[4];
  uint32_t v_sign_bits[4];
  uint8_t* pages;
  int32_t n_pool;
  const int32_t* page_ids;   // [n_codec_pages * 8]
};

__device__ __forceinline__ uint8_t* gen_page(const GenAppendArgs& a, int slot) {
  return a.pages + clamp_page(a.page_ids[slot], a.n_pool) * (int64_t)a.L.bytes;
}

// grid (n_codec_pages * 8), block 256 = 4 waves, one 16-token page each.
// Us[t][r] = sum_c M[t][c] basis32[c][r] in fp32 (the reference's M @ V): the
// page's 16 key rows staged in LDS, wave w sums channels [w C/4, (w+1) C/4) in
// order, lane (t = lane & 15, rq = lane >> 4) owns ranks rq R/4 .. + R/4, and
// the four partial sums are added in wave order.  The first codec page of a
// sequence takes its SVD factor instead.
template <int R>
__global__ __launch_bounds__(256) void gen_us_kernel(const GenAppendArgs a) {
  constexpr int RQ = R / 4;
  extern __shared__ uint16_t s_m[];          // [kPT][C + 2] fp16 key rows
  __shared__ float s_part[4][kPT][R + 1];
  const int pg = blockIdx.x, cp = pg / 8, pl = pg % 8;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int C = a.L.C, D = a.L.d, ld = C + 2;
  uint8_t* page = gen_page(a, pg);
  uint16_t* us = reinterpret_cast<uint16_t*>(page + a.L.us);
  if (a.us_first != nullptr && cp == 0) {
    for (int e = tid; e < kPT * R; e += 256) us[e] = float_to_half_bits(a.us_first[pl * kPT * R + e]);
    return;
  }
  for (int e = tid; e < kPT * C; e += 256) {
    const int t = e / C, c = e % C;
    s_m[t * ld + c] = a.k_pre[(c / D) * a.ksh + (int64_t)(pg * kPT + t) * a.kst + (c % D)];
  }
  __syncthreads();
  const int t = lane & 15, rq = lane >> 4;
  float acc[RQ];
#pragma unroll
  for (int k = 0; k < RQ; ++k) acc[k] = 0.f;
  const int c0 = wave * (C / 4), c1 = c0 + C / 4;
  for (int c = c0; c < c1; ++c) {
    const float m = half_bits_to_float(s_m[t * ld + c]);
    const float4* b = reinterpret_cast<const float4*>(a.basis32 + (int64_t)c * R + rq * RQ);
#pragma unroll
    for (int k4 = 0; k4 < RQ / 4; ++k4) {
      const float4 bv = b[k4];
      acc[4 * k4 + 0] = __builtin_fmaf(m, bv.x, acc[4 * k4 + 0]);
      acc[4 * k4 + 1] = __builtin_fmaf(m, bv.y, acc[4 * k4 + 1]);
      acc[4 * k4 + 2] = __builtin_fmaf(m, bv.z, acc[4 * k4 + 2]);
      acc[4 * k4 + 3] = __builtin_fmaf(m, bv.w, acc[4 * k4 + 3]);
    }
  }
#pragma unroll
  for (int k = 0; k < RQ; ++k) s_part[wave][t][rq * RQ + k] = acc[k];
  __syncthreads();
  for (int e = tid; e < kPT * R; e += 256) {
    const int tt = e / R, r = e % R;
    const float v = ((s_part[0][tt][r] + s_part[1][tt][r]) + s_part[2][tt][r]) + s_part[3][tt][r];
    us[e] = float_to_half_bits(v);
  }
}

// grid (residual groups of the call, h_kv), block 256: the group's tokens x
// the head's d channels.  Thread (channel j = tid % d, part tid / d) takes
// tokens part, part + 256/d, ...: L = sum_r Us16[t][r] basis16[c][r] (ranks in
// order), R = M - L; the channel's scale is max |R| over the group / qmax and
// its codes clamp(rint(R / scale), -qmax - 1, qmax).  Dynamic LDS: the
// group's Us16 rows and the head's basis16 rows (fp16, exact), then the codes.
__global__ __launch_bounds__(256) void gen_kres_kernel(const GenAppendArgs a) {
  const GenLayout& L = a.L;
  const int gi = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const int D = L.d, R = L.R, NG = L.group, C = L.C;
  const int gpp = kCodec / NG;                      // groups per codec page
  const int cp = gi / gpp, g_in = gi % gpp;
  const int slot0 = cp * 8 + g_in * (NG / kPT);     // first 16-token page slot of the group
  extern __shared__ uint16_t s_dyn[];
  uint16_t* s_us = s_dyn;                           // [NG][R]
  uint16_t* s_b = s_us + NG * R;                    // [D][R]
  int8_t* s_code = reinterpret_cast<int8_t*>(s_b + D * R);   // [NG][D]
  __shared__ float s_amax[8][128];
  for (int e = tid; e < NG * R; e += 256) {
    const int t = e / R, r = e % R;
    const uint8_t* page = gen_page(a, slot0 + t / kPT);
    s_us[e] = *reinterpret_cast<const uint16_t*>(page + L.us + ((t % kPT) * R + r) * 2);
  }
  for (int e = tid; e < D * R; e += 256) s_b[e] = a.basis16[(int64_t)(h * D) * R + e];
  __syncthreads();
  const int j = tid % D, part = tid / D, parts = 256 / D, per = NG / parts;
  const int qmax = (1 << (L.bits - 1)) - 1;
  float res[64];   // per <= 64 (d >= 32 and group <= 128): fixed bounds keep it in registers
  float amax = 0.f;
#pragma unroll
  for (int k = 0; k < 64; ++k) {
    if (k >= per) break;
    const int t = part + parts * k;
    const int tg = cp * kCodec + g_in * NG + t;     // token within the call
    float Lv = 0.f;
    for (int r = 0; r < R; ++r)
      Lv = __builtin_fmaf(half_bits_to_float(s_us[t * R + r]), half_bits_to_float(s_b[j * R + r]), Lv);
    const float m = half_bits_to_float(a.k_pre[h * a.ksh + (int64_t)tg * a.kst + j]);
    res[k] = m - Lv;
    amax = fmaxf(amax, fabsf(res[k]));
  }
  s_amax[part][j] = amax;
  __syncthreads();
  float mx = s_amax[0][j];
  for (int p = 1; p < parts; ++p) mx = fmaxf(mx, s_amax[p][j]);
  const float scale = fmaxf(mx, 1e-12f) / (float)qmax;
#pragma unroll
  for (int k = 0; k < 64; ++k) {
    if (k >= per) break;
    float cq = rintf(res[k] / scale);
    cq = fminf(fmaxf(cq, (float)(-qmax - 1)), (float)qmax);
    s_code[(part + parts * k) * D + j] = (int8_t)cq;
  }
  if (part == 0) {
    const int c = h * D + j, slot = c / L.per_slot, off = c % L.per_slot;
    *reinterpret_cast<uint16_t*>(gen_page(a, slot0 + slot) + L.kscale + off * 2) = float_to_half_bits(scale);
  }
  __syncthreads();
  // KRES: 8 channels (4 bytes) of one token per item, offset-binary nibbles
  const int off = 1 << (L.bits - 1);
  for (int e = tid; e < NG * (D / 8); e += 256) {
    const int t = e / (D / 8), j8 = e % (D / 8);
    uint32_t w = 0u;
#pragma unroll
    for (int i = 0; i < 8; ++i) w |= (uint32_t)(s_code[t * D + 8 * j8 + i] + off) << (4 * i);
    uint8_t* page = gen_page(a, slot0 + t / kPT);
    *reinterpret_cast<uint32_t*>(page + L.kres + (h * kPT + t % kPT) * (D / 2) + 4 * j8) = w;
  }
}

// grid (16-token pages of the call, h_kv), block 256: the page's 16 value rows
// of one head.
__global__ __launch_bounds__(256) void gen_v_kernel(const GenAppendArgs a) {
  const GenLayout& L = a.L;
  const int pg = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, D = L.d;
  __shared__ float x[kPT][128];
  __shared__ float s_norm[kPT];
  __shared__ uint8_t code[kPT][128];
  uint8_t* page = gen_page(a, pg);
  for (int e = tid; e < kPT * D; e += 256) {
    const int t = e / D, c = e % D;
    const int64_t i = h * a.vsh + (int64_t)(pg * kPT + t) * a.vst + c;
    float val;
    if (a.v_dtype == BMX_K2B_F32)
      val = static_cast<const float*>(a.v)[i];
    else if (a.v_dtype == BMX_K2B_BF16)
      val = __uint_as_float((uint32_t)static_cast<const uint16_t*>(a.v)[i] << 16);
    else
      val = half_bits_to_float(static_cast<const uint16_t*>(a.v)[i]);
    x[t][c] = val;
  }
  __syncthreads();
  // norms in the order torch's CPU 2-norm reduces a row (8 strided FMA
  // accumulators, a left-to-right sum of them, a correctly rounded sqrt)
  if (tid < kPT) {
    const int t = tid;
    float acc8[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) acc8[k] = 0.f;
    for (int i = 0; i < D; i += 8) {
#pragma unroll
      for (int k = 0; k < 8; ++k) acc8[k] = __builtin_fmaf(x[t][i + k], x[t][i + k], acc8[k]);
    }
    float ss = acc8[0];
#pragma unroll
    for (int k = 1; k < 8; ++k) ss = ss + acc8[k];
    const float nrm = fmaxf(__builtin_sqrtf(ss), 1e-12f);
    const uint16_t nb = float_to_half_bits(nrm);
    s_norm[t] = half_bits_to_float(nb);
    *reinterpret_cast<uint16_t*>(page + L.vnorm + (h * kPT + t) * 2) = nb;
  }
  __syncthreads();
  for (int e = tid; e < kPT * D; e += 256) {
    const int t = e / D, c = e % D;
    const float u = x[t][c] / s_norm[t];
    x[t][c] = sign_neg(a.v_sign_bits, c) ? -u : u;
  }
  __syncthreads();
  for (int hb = 1; hb < D; hb <<= 1) {   // FWHT stages as quant/hadamard.py:19-25
    for (int e = tid; e < kPT * D / 2; e += 256) {
      const int t = e / (D / 2), p = e % (D / 2);
      const int i0 = (p / hb) * 2 * hb + (p % hb);
      const float u = x[t][i0], w = x[t][i0 + hb];
      x[t][i0] = u + w;
      x[t][i0 + hb] = u - w;
    }
    __syncthreads();
  }
  const float sqrt_d = __builtin_sqrtf((float)D);   // fl32(sqrt(d)), applied as / then *
  const float mid0 = (a.codebook[0] + a.codebook[1]) / 2.0f;
  const float mid1 = (a.codebook[1] + a.codebook[2]) / 2.0f;
  const float mid2 = (a.codebook[2] + a.codebook[3]) / 2.0f;
  for (int e = tid; e < kPT * D; e += 256) {
    const int t = e / D, c = e % D;
    const float r = (x[t][c] / sqrt_d) * sqrt_d;
    code[t][c] = (uint8_t)((r > mid0) + (r > mid1) + (r > mid2));
  }
  __syncthreads();
  // VCODE [h][4][d]: byte (a, j) holds tokens 4a .. 4a + 3 of channel j; 4 channels per item
  for (int e = tid; e < D; e += 256) {
    const int aq = e / (D / 4), j4 = e % (D / 4);
    uint32_t w = 0u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = 4 * j4 + i;
      uint32_t byte = 0u;
#pragma unroll
      for (int t = 0; t < 4; ++t) byte |= (uint32_t)code[4 * aq + t][j] << (2 * t);
      w |= byte << (8 * i);
    }
    *reinterpret_cast<uint32_t*>(page + L.vcode + (h * 4 + aq) * D + 4 * j4) = w;
  }
}

// ---------------------------------------------------------------------------
// Read side.  MFMA 16x16x16 f16 fragments (lane l = 16 qd + n): A holds
// A[n][4qd .. 4qd+3], B holds B[4qd .. 4qd+3][n], the result D[4qd + e][n].
//   K^T tile rt (channels 16rt ..): A = basis rows 16rt + n, ranks 16ks + 4qd ..
//     (LDS), B = Us[token n][16ks + 4qd ..] -> lane: K[16rt + 4qd + e][token n]
//   S^T = K^T Q^T: A = that tile (token n, channels 16rt + 4qd + e), B = query
//     n's channels 16rt + 4qd + e, both as fp16 high and low parts
//     -> lane: score of token 4qd + e for query n
//   O = P V: A = those weights (query n, tokens 4qd + e), B = value level times
//     norm of token 4qd + e, channel n + 16ct (both high + low parts)
//     -> lane: O[query 4qd + e][n + 16ct]
// RoPE pairs channels j and j + d/2: tiles rt and rt + d/32 of the same lane.
// ---------------------------------------------------------------------------
struct GenReadArgs {
  GenLayout L;
  const uint8_t* pages;
  const int32_t* page_table;   // [B][max_pages] or NULL: page b * max_pages + i
  int max_pages, n_pool;
  const uint16_t* basis;       // [C][R] fp16 (+ b * basis_stride)
  int64_t basis_stride;
  float inv_freq[64];
  float rope_scaling;
  float level[4];
  uint32_t v_sign_bits[4];
};

struct GenDecodeArgs {
  GenReadArgs r;
  int G, n_split, pps;             // splits per sequence, 16-token pages per split
  const void* q;
  int io_dtype;
  const int32_t* packed_len;
  int max_packed_len;
  float qscale;                    // sm_scale * log2(e): scores in base 2
  float* ws_acc;                   // [B][h][G][n_split][d] unnormalised sums (rotated values)
  float* ws_ml;                    // [B][h][G][n_split][2] (max, sum)
  // the merge
  void* out;
  const uint16_t* k_tail;
  const uint16_t* v_tail;
  int64_t ts_b, ts_h, ts_t;
  int tail_cap, tail_bf16;
  const int32_t* tail_len;
  WinNew nw;
};

__device__ __forceinline__ half4_t gen_h4(float4_t v) {
  return half4_t{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
}

__device__ __forceinline__ const uint8_t* gen_read_page(const GenReadArgs& a, int b, int p) {
  const int32_t pid = a.page_table ? a.page_table[(int64_t)b * a.max_pages + p] : b * a.max_pages + p;
  return a.pages + clamp_page(pid, a.n_pool) * (int64_t)a.L.bytes;
}

// The lane's rebuilt keys of one page (before RoPE): kt[rt][e] = channel
// 16rt + 4qd + e of token n (head h).
template <int D, int R>
__device__ __forceinline__ void gen_keys(const GenReadArgs& a, const uint8_t* pg, const uint16_t* s_B, int b,
                                         int p, int h, int n, int qd, float4_t kt[D / 16]) {
  constexpr int NT = D / 16, NK = R / 16, LDB = R + 4;
  const GenLayout& L = a.L;
  half4_t us[NK];
#pragma unroll
  for (int ks = 0; ks < NK; ++ks)
    us[ks] = *reinterpret_cast<const half4_t*>(pg + L.us + (n * R + 16 * ks + 4 * qd) * 2);
  uint32_t kr[NT];
  half4_t sc[NT];
  const int p0 = p - p % L.slots;   // first page of the residual group
#pragma unroll
  for (int rt = 0; rt < NT; ++rt) {
    kr[rt] = *reinterpret_cast<const uint16_t*>(pg + L.kres + (h * kPT + n) * (D / 2) + (16 * rt + 4 * qd) / 2);
    const int c0 = h * D + 16 * rt + 4 * qd, slot = c0 / L.per_slot;
    const uint8_t* spg = slot == p - p0 ? pg : gen_read_page(a, b, p0 + slot);
    sc[rt] = *reinterpret_cast<const half4_t*>(spg + L.kscale + (c0 % L.per_slot) * 2);
  }
  const int off = 1 << (L.bits - 1);
#pragma unroll
  for (int rt = 0; rt < NT; ++rt) {
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < NK; ++ks) {
      const half4_t bw = *reinterpret_cast<const half4_t*>(s_B + (16 * rt + n) * LDB + 16 * ks + 4 * qd);
      acc = __builtin_amdgcn_mfma_f32_16x16x16f16(bw, us[ks], acc, 0, 0, 0);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e)
      acc[e] = __builtin_fmaf((float)sc[rt][e], (float)((int)((kr[rt] >> (4 * e)) & 15u) - off), acc[e]);
    kt[rt] = acc;
  }
}

// RoPE of the lane's keys at position pos: mode 1 exact fp32 cos/sin, mode 2
// the fp16-rounded tables (cos and sin times rope_scaling, then fp16).
// kFast: cos/sin of HF's fp32 angle fl(pos * inv_freq) from its fraction of a
// revolution (the product scaled by 1/2pi in double, its fraction rounded to
// fp32) and the hardware sin/cos of revolutions, ~1e-6 absolute: the decode's
// tables are rounded to fp16 after it (the library's sincosf takes the long
// argument reduction for the angles of long contexts and was the decode's
// bound).  Without kFast, sincosf of the fp32 angle.
template <int D, bool kFast>
__device__ __forceinline__ void gen_rope(const GenReadArgs& a, float4_t kt[D / 16], int pos, int qd, int mode) {
  constexpr int NP = D / 32;
#pragma unroll
  for (int rt = 0; rt < NP; ++rt)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float ang = (float)pos * a.inv_freq[16 * rt + 4 * qd + e];
      float sn, cs;
      if constexpr (kFast) {
        const double rev = (double)ang * 0.15915494309189535;
        const float fr = (float)(rev - floor(rev));
        cs = __builtin_amdgcn_cosf(fr);
        sn = __builtin_amdgcn_sinf(fr);
      } else {
        sincosf(ang, &sn, &cs);
      }
      cs = cs * a.rope_scaling;
      sn = sn * a.rope_scaling;
      if (mode == 2) {
        cs = (float)(_Float16)cs;
        sn = (float)(_Float16)sn;
      }
      const float x = kt[rt][e], y = kt[rt + NP][e];
      kt[rt][e] = x * cs - y * sn;
      kt[rt + NP][e] = y * cs + x * sn;
    }
}

template <int D, int R>
__global__ __launch_bounds__(256) void gen_split_kernel(const GenDecodeArgs a) {
  constexpr int NT = D / 16, LDB = R + 4;
  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, n = lane & 15, qd = lane >> 4;
  const int H = a.r.L.h, G = a.G;
  // the basis rows during the page loop, the waves' partial sums after it
  constexpr int kBBytes = D * LDB * 2, kOBytes = 4 * 16 * (D + 1) * 4;
  __shared__ __align__(16) uint8_t s_buf[kBBytes > kOBytes ? kBBytes : kOBytes];
  __shared__ float s_m[4][16], s_l[4][16];
  uint16_t* s_B = reinterpret_cast<uint16_t*>(s_buf);
  float (*s_o)[16][D + 1] = reinterpret_cast<float (*)[16][D + 1]>(s_buf);
  const uint16_t* basis = a.r.basis + (int64_t)b * a.r.basis_stride + (int64_t)(h * D) * R;
  for (int e = tid; e < D * R; e += 256) s_B[(e / R) * LDB + e % R] = basis[e];
  // query n's channels 16ks + 4qd .. as fp16 high and low parts (scaled to base 2)
  half4_t qh[NT], ql[NT];
  {
    const float sc = n < G ? a.qscale : 0.f;
    const int64_t qrow = (((int64_t)b * H + h) * G + (n < G ? n : 0)) * D;
#pragma unroll
    for (int ks = 0; ks < NT; ++ks) {
      const float4_t x = load_q4(a.q, qrow + 16 * ks + 4 * qd, a.io_dtype) * sc;
      qh[ks] = gen_h4(x);
      ql[ks] = gen_h4(x - float4_t{(float)qh[ks][0], (float)qh[ks][1], (float)qh[ks][2], (float)qh[ks][3]});
    }
  }
  const int n_tok = min(max(a.packed_len[b], 0), a.max_packed_len);
  const int n_pages = n_tok / kPT;
  const int p_begin = split * a.pps, p_end = min(p_begin + a.pps, n_pages);
  __syncthreads();
  float m_run = -INFINITY, l_part = 0.f;
  float4_t o[NT];
#pragma unroll
  for (int ct = 0; ct < NT; ++ct) o[ct] = float4_t{0.f, 0.f, 0.f, 0.f};
  for (int p = p_begin + wave; p < p_end; p += 4) {
    const uint8_t* pg = gen_read_page(a.r, b, p);
    const GenLayout& L = a.r.L;
    const half4_t vn = *reinterpret_cast<const half4_t*>(pg + L.vnorm + (h * kPT + 4 * qd) * 2);
    uint32_t vc[NT];
#pragma unroll
    for (int ct = 0; ct < NT; ++ct) vc[ct] = pg[L.vcode + (h * 4 + qd) * D + n + 16 * ct];
    float4_t kt[NT];
    gen_keys<D, R>(a.r, pg, s_B, b, p, h, n, qd, kt);
    gen_rope<D, true>(a.r, kt, p * kPT + n, qd, 2);   // the reference's shared fp16 tables
    // keys and queries as fp16 high + low parts: the three products that
    // matter carry both to about 2^-22
    float4_t st = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < NT; ++ks) {
      const half4_t kh = gen_h4(kt[ks]);
      const half4_t kl = gen_h4(kt[ks] - float4_t{(float)kh[0], (float)kh[1], (float)kh[2], (float)kh[3]});
      st = __builtin_amdgcn_mfma_f32_16x16x16f16(kh, qh[ks], st, 0, 0, 0);
      st = __builtin_amdgcn_mfma_f32_16x16x16f16(kh, ql[ks], st, 0, 0, 0);
      st = __builtin_amdgcn_mfma_f32_16x16x16f16(kl, qh[ks], st, 0, 0, 0);
    }
    // online softmax of query n over the page's 16 tokens (4 per lane)
    float mloc = fmaxf(fmaxf(st[0], st[1]), fmaxf(st[2], st[3]));
    mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
    const float m_new = fmaxf(m_run, mloc);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    float4_t pw;
#pragma unroll
    for (int e = 0; e < 4; ++e) pw[e] = __builtin_amdgcn_exp2f(st[e] - m_new);
    l_part = l_part * alpha + ((pw[0] + pw[1]) + (pw[2] + pw[3]));
    m_run = m_new;
    // the output rows are queries 4qd + e: their rescale factors from lanes 4qd + e
    float4_t al;
#pragma unroll
    for (int e = 0; e < 4; ++e) al[e] = __shfl(alpha, 4 * qd + e);
    const half4_t ph = gen_h4(pw);
    const half4_t pl = gen_h4(pw - float4_t{(float)ph[0], (float)ph[1], (float)ph[2], (float)ph[3]});
#pragma unroll
    for (int ct = 0; ct < NT; ++ct) {
      half4_t vh, vl;   // norm times level, fp16 high + low parts
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = (float)vn[e] * a.r.level[(vc[ct] >> (2 * e)) & 3u];
        vh[e] = (_Float16)x;
        vl[e] = (_Float16)(x - (float)vh[e]);
      }
      o[ct] *= al;
      o[ct] = __builtin_amdgcn_mfma_f32_16x16x16f16(ph, vh, o[ct], 0, 0, 0);
      o[ct] = __builtin_amdgcn_mfma_f32_16x16x16f16(pl, vh, o[ct], 0, 0, 0);
      o[ct] = __builtin_amdgcn_mfma_f32_16x16x16f16(ph, vl, o[ct], 0, 0, 0);
    }
  }
  l_part += __shfl_xor(l_part, 16);
  l_part += __shfl_xor(l_part, 32);
  __syncthreads();   // every wave is done with the basis rows
  if (qd == 0) {
    s_m[wave][n] = m_run;
    s_l[wave][n] = l_part;
  }
#pragma unroll
  for (int ct = 0; ct < NT; ++ct)
#pragma unroll
    for (int e = 0; e < 4; ++e) s_o[wave][4 * qd + e][n + 16 * ct] = o[ct][e];
  __syncthreads();
  const int64_t rows = ((int64_t)b * H + h) * G;
  for (int it = tid; it < G * D; it += 256) {
    const int g = it / D, c = it % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, s_m[w][g]);
    float acc = 0.f, l = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float wt = s_m[w][g] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s_m[w][g] - M);
      acc += wt * s_o[w][g][c];
      l += wt * s_l[w][g];
    }
    const int64_t slot = (rows + g) * a.n_split + split;
    a.ws_acc[slot * D + c] = acc;
    if (c == 0) {
      a.ws_ml[2 * slot] = M;
      a.ws_ml[2 * slot + 1] = l;
    }
  }
}

__device__ __forceinline__ void gen_store_io(void* base, int64_t idx, float v, int io) {
  if (io == kIoF32) {
    reinterpret_cast<float*>(base)[idx] = v;
  } else if (io == kIoF16) {
    reinterpret_cast<uint16_t*>(base)[idx] = float_to_half_bits(v);
  } else {
    reinterpret_cast<uint16_t*>(base)[idx] = (uint16_t)bf16_bits(v);
  }
}

// Sum over the 128 threads of v (every thread gets the result); s_red holds 2.
__device__ __forceinline__ float gen_block_sum(float v, float* s_red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = v;
  __syncthreads();
  return s_red[0] + s_red[1];
}

__device__ __forceinline__ float gen_block_max(float v, float* s_red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = v;
  __syncthreads();
  return fmaxf(s_red[0], s_red[1]);
}

// grid (G, h_kv, B), block 128: output row (b, h, g).  The splits' partials
// merge by the split softmax's weights, the inverse value rotation (H_d, the
// codec's signs, 1/d) turns the sum into values, and the recent window
// (scored here; rows given apart read from there and copied into the window
// buffer by query 0's workgroup) joins with its own weight.  Thread (part,
// c4) takes 4 channels of splits / window rows part, part + P, ...  Every
// first-pass load of the four phases (the split maxima and sums, the
// thread's splits' partial sums, its window row's key, its window value rows)
// is issued before any of them is used, so the phases share one memory round
// trip; splits and window rows beyond the first pass are loaded in later
// passes.
template <int D>
__global__ __launch_bounds__(128) void gen_merge_kernel(const GenDecodeArgs a) {
  constexpr int NC4 = D / 4, P = 128 / NC4;   // channel quads, row parts
  constexpr int kMS = 64 / P;                 // first-pass splits per thread: 64 splits
  constexpr int kMV = (D == 128 ? 64 : 128) / P;   // first-pass window value rows per thread
  const int g = blockIdx.x, h = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  const int H = a.r.L.h, G = a.G, S = a.n_split;
  const int c4 = tid % NC4, part = tid / NC4;
  __shared__ float s_x[D], s_q[D], s_red[2];
  __shared__ float4_t s_part[P][NC4];
  __shared__ float s_s[4096];
  const int64_t row = ((int64_t)b * H + h) * G + g;
  const float2* ml = reinterpret_cast<const float2*>(a.ws_ml) + row * S;
  const float* accr = a.ws_acc + row * S * D + 4 * c4;
  const bool wbf = __builtin_amdgcn_readfirstlane(a.tail_bf16) != 0;
  const int64_t tb = (int64_t)b * a.ts_b + (int64_t)h * a.ts_h;
  const int64_t nb = (int64_t)b * a.nw.sb + (int64_t)h * a.nw.sh;
  auto wrow = [&](const uint16_t* fresh, const uint16_t* buf, int t) {
    const int i = fresh_row(a.nw, t);
    return i >= 0 ? fresh + nb + (int64_t)i * a.nw.st : buf + tb + (int64_t)t * a.ts_t;
  };
  auto cvt4 = [&](uint2 r) {   // 4 window elements as fp32
    return wbf ? float4_t{__uint_as_float(r.x << 16), __uint_as_float(r.x & 0xffff0000u),
                          __uint_as_float(r.y << 16), __uint_as_float(r.y & 0xffff0000u)}
               : float4_t{half_bits_to_float(r.x & 0xffff), half_bits_to_float(r.x >> 16),
                          half_bits_to_float(r.y & 0xffff), half_bits_to_float(r.y >> 16)};
  };
  const int Tc = a.tail_cap;   // the host's bound of the window
  // ---- every first-pass load at once
  float4_t qx = {0.f, 0.f, 0.f, 0.f};
  if (tid < D) qx = load_q4(a.q, row * D + (tid & ~3), a.io_dtype);
  const float2 mlv = ml[min(tid, S - 1)];
  float msp[kMS];
  float4_t accv[kMS];
#pragma unroll
  for (int k = 0; k < kMS; ++k) {
    const int sc = min(part + P * k, S - 1);
    msp[k] = ml[sc].x;
    accv[k] = *reinterpret_cast<const float4_t*>(accr + (int64_t)sc * D);
  }
  uint2 kv[NC4], vv[kMV];
  if (Tc > 0) {
    const uint16_t* kr = wrow(a.nw.k, a.k_tail, min(tid, Tc - 1));
#pragma unroll
    for (int c = 0; c < NC4; ++c) kv[c] = *reinterpret_cast<const uint2*>(kr + 4 * c);
#pragma unroll
    for (int k = 0; k < kMV; ++k)
      vv[k] = *reinterpret_cast<const uint2*>(wrow(a.nw.v, a.v_tail, min(part + P * k, Tc - 1)) + 4 * c4);
  }
  const int T = a.tail_len ? min(max(a.tail_len[b], 0), Tc) : a.nw.T;
  if (tid < D) s_q[tid] = qx[tid & 3] * a.qscale;   // published by the block max's barriers

  // ---- packed partials: the max, then weighted sums
  float mx = tid < S ? mlv.x : -INFINITY;
  for (int s2 = tid + 128; s2 < S; s2 += 128) mx = fmaxf(mx, ml[s2].x);
  const float Mp = gen_block_max(mx, s_red);
  float lp = 0.f;
  float4_t acc = {0.f, 0.f, 0.f, 0.f};
  if (Mp != -INFINITY) {
    if (tid < S && mlv.x != -INFINITY) lp = __builtin_amdgcn_exp2f(mlv.x - Mp) * mlv.y;
    for (int s2 = tid + 128; s2 < S; s2 += 128) {
      const float2 v = ml[s2];
      lp += v.x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(v.x - Mp) * v.y;
    }
#pragma unroll
    for (int k = 0; k < kMS; ++k) {
      const bool ok = part + P * k < S && msp[k] != -INFINITY;
      const float w = ok ? __builtin_amdgcn_exp2f(msp[k] - Mp) : 0.f;
      acc += ok ? w * accv[k] : float4_t{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll 4
    for (int s2 = part + P * kMS; s2 < S; s2 += P) {
      const float m = ml[s2].x;
      const float w = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - Mp);
      acc += w * *reinterpret_cast<const float4_t*>(accr + (int64_t)s2 * D);
    }
  }
  const float Lp = gen_block_sum(lp, s_red);
  s_part[part][c4] = acc;
  __syncthreads();
  if (tid < NC4) {
    float4_t t = s_part[0][tid];
    for (int q = 1; q < P; ++q) t += s_part[q][tid];
    *reinterpret_cast<float4_t*>(&s_x[4 * tid]) = t;
  }
  __syncthreads();
  for (int hb = 1; hb < D; hb <<= 1) {   // unnormalised H_d, Sylvester order
    float u = 0.f, v = 0.f;
    int i0 = 0;
    if (tid < D / 2) {
      i0 = (tid / hb) * 2 * hb + (tid % hb);
      u = s_x[i0];
      v = s_x[i0 + hb];
    }
    __syncthreads();
    if (tid < D / 2) {
      s_x[i0] = u + v;
      s_x[i0 + hb] = u - v;
    }
    __syncthreads();
  }
  float op = 0.f;
  if (tid < D) {
    op = s_x[tid] / (float)D;
    if (sign_neg(a.r.v_sign_bits, tid)) op = -op;
  }
  // ---- the recent window: scores, one row per thread (its first from kv)
  auto score = [&](const uint2 (&k4)[NC4]) {
    float sc = 0.f;
#pragma unroll
    for (int c = 0; c < NC4; ++c) {
      const float4_t x = cvt4(k4[c]);
#pragma unroll
      for (int e = 0; e < 4; ++e) sc = __builtin_fmaf(s_q[4 * c + e], x[e], sc);
    }
    return sc;
  };
  float mw = -INFINITY;
  if (tid < T) {
    const float sc = score(kv);
    s_s[tid] = sc;
    mw = sc;
  }
  for (int t = tid + 128; t < T; t += 128) {
    const uint16_t* kr = wrow(a.nw.k, a.k_tail, t);
    uint2 k4[NC4];
#pragma unroll
    for (int c = 0; c < NC4; ++c) k4[c] = *reinterpret_cast<const uint2*>(kr + 4 * c);
    const float sc = score(k4);
    s_s[t] = sc;
    mw = fmaxf(mw, sc);
  }
  mw = gen_block_max(mw, s_red);   // its barriers also publish s_s
  float lw = 0.f;
  for (int t = tid; t < T; t += 128) lw += __builtin_amdgcn_exp2f(s_s[t] - mw);
  float4_t ow = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < kMV; ++k) {
    const int t = part + P * k;
    if (t < T) ow += __builtin_amdgcn_exp2f(s_s[t] - mw) * cvt4(vv[k]);
  }
#pragma unroll 4
  for (int t = part + P * kMV; t < T; t += P)
    ow += __builtin_amdgcn_exp2f(s_s[t] - mw) * cvt4(*reinterpret_cast<const uint2*>(wrow(a.nw.v, a.v_tail, t) + 4 * c4));
  const float Lw = gen_block_sum(lw, s_red);
  s_part[part][c4] = ow;
  if (g == 0 && a.nw.n > 0) {   // rows given apart into the window buffer
    for (int e = tid; e < a.nw.n * D; e += 128) {
      const int t = a.nw.T - a.nw.n + e / D, c = e % D;
      const int64_t src = nb + (int64_t)(e / D) * a.nw.st + c, dst = tb + (int64_t)t * a.ts_t + c;
      a.nw.k_dst[dst] = a.nw.k[src];
      a.nw.v_dst[dst] = a.nw.v[src];
    }
  }
  __syncthreads();
  if (tid < D) {
    float owc = 0.f;
    for (int q = 0; q < P; ++q) owc += s_part[q][tid / 4][tid % 4];
    const float M = fmaxf(Mp, mw);
    const float wp = Mp == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(Mp - M);
    const float ww = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M);
    const float den = wp * Lp + ww * Lw;
    gen_store_io(a.out, row * D + tid, den > 0.f ? (wp * op + ww * owc) / den : 0.f, a.io_dtype);
  }
}

// Dense keys and values of committed pages: grid (pages, h_kv), block 64.
struct GenDequantArgs {
  GenReadArgs r;
  int apply_rope, pos0, out_dtype;
  int64_t out_rows;
  void* k_out;
  void* v_out;
};

template <int D, int R>
__global__ __launch_bounds__(64) void gen_dequant_kernel(const GenDequantArgs a) {
  constexpr int NT = D / 16, LDB = R + 4;
  const int p = blockIdx.x, h = blockIdx.y, lane = threadIdx.x, n = lane & 15, qd = lane >> 4;
  const GenLayout& L = a.r.L;
  __shared__ __align__(16) uint16_t s_B[D * LDB];
  __shared__ float s_v[kPT][D + 1];
  const uint16_t* basis = a.r.basis + (int64_t)(h * D) * R;
  for (int e = lane; e < D * R; e += 64) s_B[(e / R) * LDB + e % R] = basis[e];
  __syncthreads();
  const uint8_t* pg = gen_read_page(a.r, 0, p);
  float4_t kt[NT];
  gen_keys<D, R>(a.r, pg, s_B, 0, p, h, n, qd, kt);
  if (a.apply_rope) gen_rope<D, false>(a.r, kt, a.pos0 + p * kPT + n, qd, a.apply_rope);
  const int64_t krow = ((int64_t)h * a.out_rows + p * kPT + n) * D;
#pragma unroll
  for (int rt = 0; rt < NT; ++rt)
#pragma unroll
    for (int e = 0; e < 4; ++e) store_elem(a.k_out, krow + 16 * rt + 4 * qd + e, kt[rt][e], a.out_dtype);
  // values: fwht(level / sqrt(d)) * signs * norm, per token
  const float sqrt_d = __builtin_sqrtf((float)D);
  for (int e = lane; e < kPT * D; e += 64) {
    const int t = e / D, c = e % D;
    const uint32_t code = (pg[L.vcode + (h * 4 + t / 4) * D + c] >> (2 * (t % 4))) & 3u;
    s_v[t][c] = a.r.level[code] / sqrt_d;
  }
  __syncthreads();
  for (int hb = 1; hb < D; hb <<= 1) {
    for (int e = lane; e < kPT * D / 2; e += 64) {
      const int t = e / (D / 2), i = e % (D / 2), i0 = (i / hb) * 2 * hb + (i % hb);
      const float u = s_v[t][i0], v = s_v[t][i0 + hb];
      s_v[t][i0] = u + v;
      s_v[t][i0 + hb] = u - v;
    }
    __syncthreads();
  }
  for (int e = lane; e < kPT * D; e += 64) {
    const int t = e / D, c = e % D;
    float v = s_v[t][c] / sqrt_d;
    if (sign_neg(a.r.v_sign_bits, c)) v = -v;
    v = v * half_bits_to_float(*reinterpret_cast<const uint16_t*>(pg + L.vnorm + (h * kPT + t) * 2));
    store_elem(a.v_out, ((int64_t)h * a.out_rows + p * kPT + t) * D + c, v, a.out_dtype);
  }
}

}  // namespace bmx

// ---------------------------------------------------------------------------
// Host side: argument checks, launches.
// ---------------------------------------------------------------------------
using namespace bmx;

static int gfail(int code, const std::string& msg) {
  bmx_set_error(msg);
  return code;
}

namespace {

// the (d, R) instance of a kernel template: d in {32, 64, 128}, R in {16, 32, 64, 128}
#define BMX_GEN_DISPATCH(D_, R_, CALL)                                    \
  switch ((D_) * 1000 + (R_)) {                                          \
    case 32016: CALL(32, 16); break;  case 32032: CALL(32, 32); break;    \
    case 32064: CALL(32, 64); break;  case 32128: CALL(32, 128); break;   \
    case 64016: CALL(64, 16); break;  case 64032: CALL(64, 32); break;    \
    case 64064: CALL(64, 64); break;  case 64128: CALL(64, 128); break;   \
    case 128016: CALL(128, 16); break; case 128032: CALL(128, 32); break; \
    case 128064: CALL(128, 64); break; case 128128: CALL(128, 128); break; \
    default: break;                                                      \
  }

void fill_read(GenReadArgs& r, const Geo& g) {
  r.L = GenLayout::of(g);
}

// splits per sequence and 16-token pages per split
void gen_plan(const bmx_k2b_decode_args* a, const Geo& g, int* n_split, int* pps) {
  const int pages = a->max_packed_len / kPT;
  if (pages == 0) {
    *n_split = 1;
    *pps = 1;
    return;
  }
  int per = a->split_tokens > 0 ? a->split_tokens / kPT : 0;
  if (per == 0) {
    const int target = 2 * bmx_device_cu_count();
    const int per_seq = std::max(1, (target + a->batch * g.h - 1) / (a->batch * g.h));
    per = std::max(4, (pages + per_seq - 1) / per_seq);
  }
  *pps = per;
  *n_split = (pages + per - 1) / per;
}

}  // namespace

namespace bmx {

int gen_append(const bmx_k2b_append_args* a, hipStream_t st) {
  const Geo g = Geo::from(a->geom);
  const std::string why = g.check();
  if (!why.empty()) return gfail(BMX_E_INVALID, "bmx_k2b_append: " + why);
  GenAppendArgs k{};
  k.L = GenLayout::of(g);
  k.k_pre = a->k_pre; k.ksh = a->k_stride_h; k.kst = a->k_stride_t;
  k.v = a->v; k.vsh = a->v_stride_h; k.vst = a->v_stride_t; k.v_dtype = a->v_dtype;
  k.basis32 = a->basis32; k.basis16 = a->basis16; k.us_first = a->us_first;
  for (int i = 0; i < 4; ++i) { k.codebook[i] = a->codebook[i]; k.v_sign_bits[i] = a->v_sign_bits[i]; }
  k.pages = a->pages; k.n_pool = a->n_pool_pages; k.page_ids = a->page_ids;
  const int np = a->n_codec_pages * 8;
  const size_t us_lds = (size_t)kPT * (g.C() + 2) * 2;
  hipError_t e = hipSuccess;
#define BMX_GEN_US(R_)                                                                          \
  if (g.R == R_) {                                                                              \
    if (us_lds > 65536) e = bmx_ensure_dynamic_lds((const void*)gen_us_kernel<R_>, us_lds);      \
    if (e == hipSuccess) hipLaunchKernelGGL(gen_us_kernel<R_>, dim3(np), dim3(256), us_lds, st, k); \
  }
  BMX_GEN_US(16) BMX_GEN_US(32) BMX_GEN_US(64) BMX_GEN_US(128)
#undef BMX_GEN_US
  if (e != hipSuccess) return gfail(BMX_E_HIP, std::string("bmx_k2b_append: LDS limit: ") + hipGetErrorString(e));
  const size_t kres_lds = (size_t)(g.group * g.R + g.d * g.R) * 2 + (size_t)g.group * g.d;
  if (kres_lds > 65536) {
    e = bmx_ensure_dynamic_lds((const void*)gen_kres_kernel, kres_lds);
    if (e != hipSuccess) return gfail(BMX_E_HIP, std::string("bmx_k2b_append: LDS limit: ") + hipGetErrorString(e));
  }
  hipLaunchKernelGGL(gen_kres_kernel, dim3(a->n_codec_pages * (kCodec / g.group), g.h), dim3(256), kres_lds, st, k);
  hipLaunchKernelGGL(gen_v_kernel, dim3(np, g.h), dim3(256), 0, st, k);
  e = hipGetLastError();
  if (e != hipSuccess) return gfail(BMX_E_HIP, std::string("bmx_k2b_append: launch: ") + hipGetErrorString(e));
  return BMX_OK;
}

size_t gen_decode_workspace(const bmx_k2b_decode_args* a) {
  const Geo g = Geo::from(a->geom);
  int n_split, pps;
  gen_plan(a, g, &n_split, &pps);
  return (size_t)a->batch * g.h * g.G * n_split * (g.d + 2) * sizeof(float);
}

std::string gen_decode_check(const bmx_k2b_decode_args* a) {
  const Geo g = Geo::from(a->geom);
  const std::string why = g.check();
  if (!why.empty()) return why;
  if (g.G < 1 || g.G > 16) return "n_q_groups must be 1..16";
  if (a->max_packed_len % g.group != 0) return "max_packed_len must be a multiple of k_group";
  return "";
}

int gen_decode(const bmx_k2b_decode_args* a, hipStream_t st, void* ws, size_t ws_cap, const std::string& name) {
  const Geo g = Geo::from(a->geom);
  int n_split, pps;
  gen_plan(a, g, &n_split, &pps);
  const size_t need = gen_decode_workspace(a);
  if (!ws || ws_cap < need)
    return gfail(BMX_E_WORKSPACE, name + ": workspace missing or smaller than bmx_k2b_decode_workspace_bytes()");
  GenDecodeArgs k{};
  fill_read(k.r, g);
  k.r.pages = a->pages; k.r.page_table = a->page_table; k.r.max_pages = a->max_pages;
  k.r.n_pool = a->n_pool_pages > 0 ? a->n_pool_pages : 1;
  k.r.basis = a->basis; k.r.basis_stride = a->basis_stride;
  for (int j = 0; j < 64; ++j) k.r.inv_freq[j] = a->inv_freq[j];
  k.r.rope_scaling = a->rope_scaling;
  for (int j = 0; j < 4; ++j) { k.r.level[j] = a->codebook[j]; k.r.v_sign_bits[j] = a->v_sign_bits[j]; }
  k.G = g.G; k.n_split = n_split; k.pps = pps;
  k.q = a->q; k.io_dtype = a->io_dtype;
  k.packed_len = a->packed_len; k.max_packed_len = a->max_packed_len;
  k.qscale = a->sm_scale * 1.4426950408889634f;
  const size_t rows = (size_t)a->batch * g.h * g.G * n_split;
  k.ws_acc = (float*)ws;
  k.ws_ml = k.ws_acc + rows * g.d;
  k.out = a->out;
  k.k_tail = a->k_tail; k.v_tail = a->v_tail;
  k.ts_b = a->tail_stride_b; k.ts_h = a->tail_stride_h; k.ts_t = a->tail_stride_t;
  k.tail_cap = a->tail_cap; k.tail_bf16 = a->tail_dtype == BMX_K2B_TAIL_BF16;
  k.tail_len = a->tail_len;
  k.nw.k = a->new_k; k.nw.v = a->new_v;
  k.nw.sb = a->new_stride_b; k.nw.sh = a->new_stride_h; k.nw.st = a->new_stride_t;
  k.nw.n = a->n_new;
  k.nw.T = a->tail_len ? -1 : a->tail_len_value;
  k.nw.k_dst = const_cast<uint16_t*>(a->k_tail);
  k.nw.v_dst = const_cast<uint16_t*>(a->v_tail);
  const dim3 grid(n_split, g.h, a->batch);
#define BMX_GEN_SPLIT(D_, R_) hipLaunchKernelGGL((gen_split_kernel<D_, R_>), grid, dim3(256), 0, st, k)
  BMX_GEN_DISPATCH(g.d, g.R, BMX_GEN_SPLIT)
#undef BMX_GEN_SPLIT
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return gfail(BMX_E_HIP, name + ": split kernel launch: " + hipGetErrorString(e));
  if (a->split_end_event) {
    e = hipEventRecord((hipEvent_t)a->split_end_event, st);
    if (e != hipSuccess) return gfail(BMX_E_HIP, name + ": hipEventRecord: " + hipGetErrorString(e));
  }
  const dim3 mgrid(g.G, g.h, a->batch);
  if (g.d == 32) hipLaunchKernelGGL(gen_merge_kernel<32>, mgrid, dim3(128), 0, st, k);
  else if (g.d == 64) hipLaunchKernelGGL(gen_merge_kernel<64>, mgrid, dim3(128), 0, st, k);
  else hipLaunchKernelGGL(gen_merge_kernel<128>, mgrid, dim3(128), 0, st, k);
  e = hipGetLastError();
  if (e != hipSuccess) return gfail(BMX_E_HIP, name + ": merge kernel launch: " + hipGetErrorString(e));
  return BMX_OK;
}

int gen_dequant(const bmx_k2b_dequant_args* a, hipStream_t st) {
  const Geo g = Geo::from(a->geom);
  const std::string why = g.check();
  if (!why.empty()) return gfail(BMX_E_INVALID, "bmx_k2b_dequant: " + why);
  if (a->n_tokens % g.group != 0)
    return gfail(BMX_E_INVALID, "bmx_k2b_dequant: n_tokens must be a multiple of k_group");
  GenDequantArgs k{};
  fill_read(k.r, g);
  k.r.pages = a->pages; k.r.page_table = a->page_table; k.r.max_pages = 0; k.r.n_pool = a->n_pool_pages;
  k.r.basis = a->basis; k.r.basis_stride = 0;
  for (int j = 0; j < 64; ++j) k.r.inv_freq[j] = a->inv_freq[j];
  k.r.rope_scaling = a->rope_scaling;
  for (int j = 0; j < 4; ++j) { k.r.level[j] = a->codebook[j]; k.r.v_sign_bits[j] = a->v_sign_bits[j]; }
  k.apply_rope = a->apply_rope; k.pos0 = a->pos0; k.out_dtype = a->out_dtype;
  k.out_rows = a->out_rows ? a->out_rows : a->n_tokens;
  k.k_out = a->k_out; k.v_out = a->v_out;
  const dim3 grid(a->n_tokens / kPT, g.h);
#define BMX_GEN_DQ(D_, R_) hipLaunchKernelGGL((gen_dequant_kernel<D_, R_>), grid, dim3(64), 0, st, k)
  BMX_GEN_DISPATCH(g.d, g.R, BMX_GEN_DQ)
#undef BMX_GEN_DQ
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return gfail(BMX_E_HIP, std::string("bmx_k2b_dequant: launch: ") + hipGetErrorString(e));
  return BMX_OK;
}

}  // namespace bmx
