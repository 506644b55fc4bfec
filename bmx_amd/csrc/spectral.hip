// Spectral (K4) key path on gfx950: the write kernel (encode, MSE-refined RTN
// per direction, page packing) and the dense dequantization (tier codes ->
// Y_hat, Y_hat dec^T on MFMA, RoPE), with the k2b value codec in value-only
// pages.  Reference semantics: cache/spectral.py:763-841, quant/rtn.py:10-53,
// cache/chunked_attention.py:52-194; the page format is in
// include/bmx_spectral.h.  Built without floating-point contraction: every
// product and sum of the write kernel is rounded on its own, in a fixed order.

#include "bmx_spectral.h"
#include "k2b_common.h"

namespace bmx {

constexpr int kSpCh = 64;                          // key channels staged per pass
constexpr int kSpMaxSlices = BMX_SPECTRAL_MAX_CPAD / 8;

__device__ __forceinline__ int sp_width(int b) { return b == 2 ? 2 : (b <= 4 ? 4 : 8); }

__device__ __forceinline__ float sp_load(const void* base, int64_t i, int dtype) {
  if (dtype == BMX_K2B_F32) return static_cast<const float*>(base)[i];
  const uint16_t u = static_cast<const uint16_t*>(base)[i];
  if (dtype == BMX_K2B_BF16) return __uint_as_float((uint32_t)u << 16);
  return half_bits_to_float(u);
}

struct SpEncodeKArgs {
  int C, c_pad, n_pool, k_dtype, page_bytes;
  const void* k;
  int64_t ksh, kst;
  const float* encp;
  const int32_t* slice_tab;
  uint8_t* pages;
  const int32_t* page_ids;
};

// grid (ceil(c_pad / 64), n_groups), block 64: thread j of block x codes page
// column 64x + j of group y.  Y[t][j] for the group's 64 tokens accumulates in
// registers over the C channels, staged 64 at a time through LDS (every lane
// reads the same key element: a broadcast); then the column's step (max|Y| /
// qmax and 10 rounds of <Y, Q> / <Q, Q>), its codes, and the block's 8 slices
// assembled in LDS and written with dword stores.
__global__ __launch_bounds__(64) void spectral_encode_kernel(const SpEncodeKArgs a) {
  __shared__ float s_m[kGroup][kSpCh + 1];
  __shared__ uint32_t s_code[8 * kGroup * 8 / 4];   // 8 slices of at most 512 bytes
  const int lane = threadIdx.x, j = blockIdx.x * 64 + lane, g = blockIdx.y;
  const bool active = j < a.c_pad;
  float y[kGroup];
#pragma unroll
  for (int t = 0; t < kGroup; ++t) y[t] = 0.f;
  for (int c0 = 0; c0 < a.C; c0 += kSpCh) {
    __syncthreads();
    const int c = c0 + lane, h = c >> 7, d = c & (kD - 1);
    for (int t = 0; t < kGroup; ++t)
      s_m[t][lane] = sp_load(a.k, h * a.ksh + (int64_t)(g * kGroup + t) * a.kst + d, a.k_dtype);
    __syncthreads();
    if (active) {
      for (int cc = 0; cc < kSpCh; ++cc) {
        const float e = a.encp[(int64_t)(c0 + cc) * a.c_pad + j];
#pragma unroll
        for (int t = 0; t < kGroup; ++t) y[t] = __fadd_rn(y[t], __fmul_rn(s_m[t][cc], e));
      }
    }
  }
  const int s = j >> 3, k = j & 7;
  const uint32_t tab = active ? (uint32_t)a.slice_tab[s] : 0u;
  const int b = active ? (int)(tab >> 24) : 2, w = sp_width(b);
  const float qmax = (float)((1 << (b - 1)) - 1);
  float scale = 1e-12f;
  if (active) {
    float amax = 0.f;
#pragma unroll
    for (int t = 0; t < kGroup; ++t) amax = fmaxf(amax, fabsf(y[t]));
    scale = fmaxf(amax, 1e-12f) / qmax;
    for (int it = 0; it < 10; ++it) {
      float num = 0.f, den = 0.f;
#pragma unroll
      for (int t = 0; t < kGroup; ++t) {
        const float qv = fminf(fmaxf(rintf(y[t] / scale), -qmax - 1.f), qmax);
        num = __fadd_rn(num, __fmul_rn(y[t], qv));
        den = __fadd_rn(den, __fmul_rn(qv, qv));
      }
      scale = fmaxf(num / fmaxf(den, 1e-12f), 1e-12f);
    }
  }
  // the block's slices are contiguous in the page: [base, end)
  const int n_sl = a.c_pad >> 3, s_first = blockIdx.x * 8, s_last = min(s_first + 8, n_sl) - 1;
  const uint32_t tab0 = (uint32_t)a.slice_tab[s_first], tabl = (uint32_t)a.slice_tab[s_last];
  const int base = (int)(tab0 & 0xFFFFFFu);
  const int n_words = ((int)(tabl & 0xFFFFFFu) + kGroup * sp_width((int)(tabl >> 24)) - base) >> 2;
  for (int i = lane; i < n_words; i += 64) s_code[i] = 0u;
  __syncthreads();
  if (active) {
    const int bit0 = ((int)(tab & 0xFFFFFFu) - base) * 8 + k * w;
    const uint32_t bias = 1u << (b - 1);
#pragma unroll
    for (int t = 0; t < kGroup; ++t) {
      const float qv = fminf(fmaxf(rintf(y[t] / scale), -qmax - 1.f), qmax);
      const uint32_t stored = (uint32_t)((int)qv + (int)bias);
      const int bit = bit0 + t * w * 8;
      atomicOr(&s_code[bit >> 5], stored << (bit & 31));
    }
  }
  __syncthreads();
  uint8_t* page = a.pages + clamp_page(a.page_ids[g], a.n_pool) * (int64_t)a.page_bytes;
  uint32_t* dst = reinterpret_cast<uint32_t*>(page + base);
  for (int i = lane; i < n_words; i += 64) dst[i] = s_code[i];
  if (active) reinterpret_cast<uint16_t*>(page)[j] = float_to_half_bits(scale);
}

struct SpDequantKArgs {
  int h_kv, c_pad, c_pad32, n_tokens, apply_rope, n_k_pool, n_v_pool, out_dtype, k_page_bytes;
  const uint8_t* k_pages;
  const int32_t* k_table;
  const uint8_t* v_pages;
  const int32_t* v_table;
  const int32_t* slice_tab;
  const uint16_t* dec;
  PageLayout VL;
  float rope_scaling;
  float inv_freq[64];
  float codebook[4];
  uint32_t v_sign_bits[4];
  void* k_out;
  void* v_out;
};

// grid (n_tokens / 64, h_kv), block 256: the group's keys and values of one
// head.  Wave w computes K^T rows 16w .. 16w + 15 and their RoPE partners
// 64 + 16w .. (two 16-row tiles) for the group's 4 token tiles: per 32-column
// step, A = dec rows (fp16, lane 16q + n: row n, columns 8q .. 8q + 7) and
// B = Y_hat^T (lane 16q + n: token n of the tile, the 8 columns of slice
// 4 step + q, code times step rounded to fp16), accumulated in fp32.  Then
// RoPE on the lane's pairs (j, j + 64) and LDS-staged dense rows; the wave
// then dequantizes value page 4 group + w.
__global__ __launch_bounds__(256) void spectral_dequant_kernel(const SpDequantKArgs a) {
  const int g = blockIdx.x, h = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, n = lane & 15, q = lane >> 4;
  __shared__ uint32_t s_tab[kSpMaxSlices];
  __shared__ DqTile s_tile[4];
  const int n_sl = a.c_pad >> 3;
  for (int i = tid; i < n_sl; i += 256) s_tab[i] = (uint32_t)a.slice_tab[i];
  const uint8_t* page = a.k_pages + clamp_page(a.k_table[g], a.n_k_pool) * (int64_t)a.k_page_bytes;
  const uint8_t* vpage = a.v_pages + clamp_page(a.v_table[4 * g + wave], a.n_v_pool) * (int64_t)a.VL.bytes;
  const uint2 vcd = *reinterpret_cast<const uint2*>(vpage + a.VL.vcode + h * 512 + lane * 8);
  const uint2 nrm = *reinterpret_cast<const uint2*>(vpage + a.VL.vnorm + (h * kPT + 4 * q) * 2);
  __syncthreads();

  const uint16_t* dec0 = a.dec + ((int64_t)h * kD + 16 * wave + n) * a.c_pad32 + 8 * q;
  const uint16_t* dec1 = dec0 + (int64_t)64 * a.c_pad32;
  float4_t acc[2][4];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) acc[r][tt] = (float4_t){0.f, 0.f, 0.f, 0.f};
  const int n_steps = a.c_pad32 / 32;
  for (int ks = 0; ks < n_steps; ++ks) {
    const half8_t A0 = *reinterpret_cast<const half8_t*>(dec0 + 32 * ks);
    const half8_t A1 = *reinterpret_cast<const half8_t*>(dec1 + 32 * ks);
    const int s = 4 * ks + q;
    half8_t B[4];
    if (s < n_sl) {
      const uint32_t tab = s_tab[s];
      const int b = (int)(tab >> 24), off = (int)(tab & 0xFFFFFFu), w = sp_width(b);
      const uint4 sc = *reinterpret_cast<const uint4*>(page + 16 * s);
      const uint32_t sw[4] = {sc.x, sc.y, sc.z, sc.w};
      float scl[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        scl[2 * e] = half_bits_to_float(sw[e] & 0xffffu);
        scl[2 * e + 1] = half_bits_to_float(sw[e] >> 16);
      }
      const float bias = (float)(1 << (b - 1));
      const uint32_t mask = (1u << w) - 1u;
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const uint8_t* p = page + off + (16 * tt + n) * w;
        uint32_t lo, hi = 0u;
        if (w == 8) {
          const uint2 v = *reinterpret_cast<const uint2*>(p);
          lo = v.x;
          hi = v.y;
        } else if (w == 4) {
          lo = *reinterpret_cast<const uint32_t*>(p);
        } else {
          lo = *reinterpret_cast<const uint16_t*>(p);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          uint32_t code;
          if (w == 8)
            code = ((e < 4 ? lo : hi) >> (8 * (e & 3))) & 0xFFu;
          else
            code = (lo >> (e * w)) & mask;
          B[tt][e] = (_Float16)(((float)code - bias) * scl[e]);
        }
      }
    } else {
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int e = 0; e < 8; ++e) B[tt][e] = (_Float16)0.f;
    }
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      acc[0][tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, B[tt], acc[0][tt], 0, 0, 0);
      acc[1][tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, B[tt], acc[1][tt], 0, 0, 0);
    }
  }

  // RoPE of the lane's pairs: channel j = 16w + 4q + i and j + 64, token
  // 16tt + n, HF's fp32 angle fl(inv_freq_j * pos)
  const int pos0 = g * kGroup;
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = 16 * wave + 4 * q + i;
      float k0 = acc[0][tt][i], k1 = acc[1][tt][i];
      if (a.apply_rope) {
        float sn, cn;
        sincosf(a.inv_freq[j] * (float)(pos0 + 16 * tt + n), &sn, &cn);
        cn *= a.rope_scaling;
        sn *= a.rope_scaling;
        if (a.apply_rope == 2) {
          cn = half_bits_to_float(float_to_half_bits(cn));
          sn = half_bits_to_float(float_to_half_bits(sn));
        }
        const float r0 = __fmul_rn(k0, cn) - __fmul_rn(k1, sn);
        k1 = __fmul_rn(k1, cn) + __fmul_rn(k0, sn);
        k0 = r0;
      }
      s_tile[tt].v[n][j] = k0;
      s_tile[tt].v[n][j + 64] = k1;
    }
  }
  __syncthreads();
  const int64_t row0 = (int64_t)h * a.n_tokens + pos0 + 16 * wave;
  dq_store_tile(s_tile[wave], a.k_out, row0, a.out_dtype);
  __syncthreads();   // the staging tiles are reused for the values
  dq_value_tile(vcd, nrm, a.codebook, a.v_sign_bits, n, q, s_tile[wave]);
  __syncthreads();
  dq_store_tile(s_tile[wave], a.v_out, row0, a.out_dtype);
}

static PageLayout value_layout(int h_kv) {
  PageLayout L{};
  L.vnorm = 0;
  L.vcode = h_kv * kPT * 2;
  L.bytes = L.vcode + h_kv * 64 * 8;
  return L;
}

static int sp_fail(const char* fn, const std::string& msg) {
  bmx_set_error(std::string(fn) + ": " + msg);
  return BMX_E_INVALID;
}

static bool sp_layout_ok(const bmx_spectral_layout& L, std::string& why) {
  if (L.h_kv < 1 || L.h_kv > 8) { why = "h_kv must be 1..8"; return false; }
  const int C = kD * L.h_kv;
  if (L.c_pad < 8 || L.c_pad % 8 != 0 || L.c_pad > C + 48 || L.c_pad > BMX_SPECTRAL_MAX_CPAD) {
    why = "c_pad must be a multiple of 8 in 8..C + 48";
    return false;
  }
  const int64_t min_bytes = 2 * (int64_t)L.c_pad + (int64_t)(L.c_pad / 8) * kGroup * 2 + 16;
  if (L.k_page_bytes < min_bytes || L.k_page_bytes % 16 != 0) {
    why = "k_page_bytes too small for c_pad, or not a multiple of 16";
    return false;
  }
  if (!L.slice_tab) { why = "slice_tab is NULL"; return false; }
  return true;
}

static bool dtype_ok(int d) { return d == BMX_K2B_F16 || d == BMX_K2B_F32 || d == BMX_K2B_BF16; }

}  // namespace bmx

using namespace bmx;

extern "C" int64_t bmx_spectral_v_page_bytes(int32_t h_kv) {
  return (h_kv < 1 || h_kv > 8) ? -1 : (int64_t)value_layout(h_kv).bytes;
}

extern "C" int32_t bmx_spectral_append(const bmx_spectral_append_args* a, void* stream) {
  const char* fn = "bmx_spectral_append";
  if (!a) return sp_fail(fn, "args is NULL");
  std::string why;
  if (!sp_layout_ok(a->L, why)) return sp_fail(fn, why);
  if (a->n_groups < 0) return sp_fail(fn, "n_groups must be >= 0");
  if (a->n_groups == 0) return BMX_OK;
  if (!dtype_ok(a->k_dtype) || !dtype_ok(a->v_dtype)) return sp_fail(fn, "k_dtype / v_dtype must be BMX_K2B_F16, _F32 or _BF16");
  if (!a->k_pre || !a->v || !a->enc_perm || !a->k_pages || !a->k_page_ids || !a->v_pages || !a->v_page_ids ||
      a->n_k_pool < 1 || a->n_v_pool < 1)
    return sp_fail(fn, "null pointer argument or empty pool");
  hipStream_t st = (hipStream_t)stream;
  SpEncodeKArgs k{};
  k.C = kD * a->L.h_kv; k.c_pad = a->L.c_pad; k.n_pool = a->n_k_pool; k.k_dtype = a->k_dtype;
  k.page_bytes = a->L.k_page_bytes;
  k.k = a->k_pre; k.ksh = a->k_sh; k.kst = a->k_st;
  k.encp = a->enc_perm; k.slice_tab = a->L.slice_tab; k.pages = a->k_pages; k.page_ids = a->k_page_ids;
  hipLaunchKernelGGL(spectral_encode_kernel, dim3((a->L.c_pad + 63) / 64, a->n_groups), dim3(64), 0, st, k);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) {
    AppendKArgs v{};
    v.h_kv = a->L.h_kv; v.n_pool = a->n_v_pool;
    v.v = a->v; v.vsh = a->v_sh; v.vst = a->v_st; v.v_dtype = a->v_dtype;
    v.pages = a->v_pages; v.page_ids = a->v_page_ids; v.L = value_layout(a->L.h_kv);
    for (int i = 0; i < 4; ++i) { v.codebook[i] = a->v_codebook[i]; v.v_sign_bits[i] = a->v_sign_bits[i]; }
    e = launch_k2b_values(v, 4 * a->n_groups, a->L.h_kv, st);
  }
  if (e != hipSuccess) {
    bmx_set_error(std::string(fn) + ": launch: " + hipGetErrorString(e));
    return BMX_E_HIP;
  }
  return BMX_OK;
}

extern "C" int32_t bmx_spectral_dequant(const bmx_spectral_dequant_args* a, void* stream) {
  const char* fn = "bmx_spectral_dequant";
  if (!a) return sp_fail(fn, "args is NULL");
  std::string why;
  if (!sp_layout_ok(a->L, why)) return sp_fail(fn, why);
  if (a->n_tokens < 0 || a->n_tokens % kGroup != 0) return sp_fail(fn, "n_tokens must be a non-negative multiple of 64");
  if (a->n_tokens == 0) return BMX_OK;
  if (a->apply_rope < 0 || a->apply_rope > 2) return sp_fail(fn, "apply_rope must be 0, 1 or 2");
  if (!dtype_ok(a->out_dtype)) return sp_fail(fn, "out_dtype must be BMX_K2B_F16, _F32 or _BF16");
  if (!a->k_pages || !a->k_page_table || !a->v_pages || !a->v_page_table || !a->dec_perm || !a->k_out ||
      !a->v_out || a->n_k_pool < 1 || a->n_v_pool < 1)
    return sp_fail(fn, "null pointer argument or empty pool");
  SpDequantKArgs k{};
  k.h_kv = a->L.h_kv; k.c_pad = a->L.c_pad; k.c_pad32 = (a->L.c_pad + 31) / 32 * 32;
  k.n_tokens = a->n_tokens; k.apply_rope = a->apply_rope; k.n_k_pool = a->n_k_pool; k.n_v_pool = a->n_v_pool;
  k.out_dtype = a->out_dtype; k.k_page_bytes = a->L.k_page_bytes;
  k.k_pages = a->k_pages; k.k_table = a->k_page_table; k.v_pages = a->v_pages; k.v_table = a->v_page_table;
  k.slice_tab = a->L.slice_tab; k.dec = a->dec_perm; k.VL = value_layout(a->L.h_kv);
  k.rope_scaling = a->rope_scaling;
  for (int j = 0; j < 64; ++j) k.inv_freq[j] = a->inv_freq[j];
  for (int i = 0; i < 4; ++i) { k.codebook[i] = a->v_codebook[i]; k.v_sign_bits[i] = a->v_sign_bits[i]; }
  k.k_out = a->k_out; k.v_out = a->v_out;
  hipLaunchKernelGGL(spectral_dequant_kernel, dim3(a->n_tokens / kGroup, a->L.h_kv), dim3(256), 0,
                     (hipStream_t)stream, k);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    bmx_set_error(std::string(fn) + ": launch: " + hipGetErrorString(e));
    return BMX_E_HIP;
  }
  return BMX_OK;
}
