// Dense dequantization of committed k2b pages (prefill path and checks), gfx950.
// Reference semantics: cache/chunked_attention.py:52-194 (_dequant_block,
// _dense_kv), cache/codecs.py:639-649, 839-842 (dequant_packed).

#include "k2b_common.h"

namespace bmx {

struct DequantKArgs {
  int h_kv, R, n_tokens, apply_rope, n_pool, out_dtype;
  const uint8_t* pages;
  const int32_t* page_table;
  const uint16_t* basis;
  PageLayout L;
  float rope_scaling;
  float inv_freq[64];
  float codebook[4];
  uint32_t v_sign_bits[4];
  void* k_out;
  void* v_out;
};

// grid (n_tokens/16, h_kv), block 256
__global__ __launch_bounds__(256) void k2b_dequant_kernel(const DequantKArgs a) {
  const int lp = blockIdx.x, h = blockIdx.y;
  const int tid = threadIdx.x;
  const int C = kD * a.h_kv;
  const int R = a.R;
  const uint8_t* page = a.pages + clamp_page(a.page_table[lp], a.n_pool) * a.L.bytes;
  __shared__ float s_us[kPT][33];
  __shared__ float x[kPT][kD];
  for (int e = tid; e < kPT * R; e += 256)
    s_us[e / R][e % R] = half_bits_to_float(
        *reinterpret_cast<const uint16_t*>(page + a.L.us + us_half(R, e / R, e % R) * 2));
  __syncthreads();

  // keys: thread handles (token t, channel pair j, j+64) for 4 pairs
  const int grp = lp / 4;
  for (int e = tid; e < kPT * 64; e += 256) {
    const int t = e / 64, j0 = e % 64;
    float kv[2];
    for (int s = 0; s < 2; ++s) {
      const int j = j0 + 64 * s;
      const int c = h * kD + j;
      float acc = 0.f;
      for (int r = 0; r < R; ++r)
        acc = __builtin_fmaf(s_us[t][r], half_bits_to_float(a.basis[(int64_t)c * R + r]), acc);
      const int f = kscale_flat(c), quarter = C / 4, slot = f / quarter, off = f % quarter;
      const uint8_t* sp = a.pages + clamp_page(a.page_table[grp * 4 + slot], a.n_pool) * a.L.bytes + a.L.kscale;
      const float scale = half_bits_to_float(*reinterpret_cast<const uint16_t*>(sp + off * 2));
      const int b = j0 / 16, q = (j0 % 16) / 4, i = j0 % 4;
      const uint32_t* kr = reinterpret_cast<const uint32_t*>(page + a.L.kres + h * 768 + (16 * q + t) * 12);
      const int code = kres_pair_code(kr[0], kr[1], kr[2], 4 * b + i, s);
      kv[s] = acc + scale * (float)code;
    }
    const int64_t base = ((int64_t)h * a.n_tokens + lp * kPT + t) * kD;
    float k0 = kv[0], k1 = kv[1];
    if (a.apply_rope) {
      const float ang = a.inv_freq[j0] * (float)(lp * kPT + t);   // HF's fp32 angle
      float sn, cn;
      sincosf(ang, &sn, &cn);
      cn *= a.rope_scaling;
      sn *= a.rope_scaling;
      if (a.apply_rope == 2) {   // the reference's fp16 tables
        cn = half_bits_to_float(float_to_half_bits(cn));
        sn = half_bits_to_float(float_to_half_bits(sn));
      }
      // x*cos + rotate_half(x)*sin, rounded per operation as torch does
      k0 = __fmul_rn(kv[0], cn) - __fmul_rn(kv[1], sn);
      k1 = __fmul_rn(kv[1], cn) + __fmul_rn(kv[0], sn);
    }
    store_elem(a.k_out, base + j0, k0, a.out_dtype);
    store_elem(a.k_out, base + j0 + 64, k1, a.out_dtype);
  }

  // values: codebook level per (token, channel), FWHT, signs, norm
  for (int e = tid; e < kPT * kD; e += 256) {
    const int t = e / kD, c = e % kD;
    const int b = c / 16, m = c % 16, q = t / 4, tt = t % 4;
    const uint32_t* vc = reinterpret_cast<const uint32_t*>(page + a.L.vcode + h * 512 + (16 * q + m) * 8);
    const uint32_t D = vc[b / 4];
    const int idx = (D >> (8 * (b % 4) + 2 * tt)) & 3;
    x[t][c] = a.codebook[idx];
  }
  __syncthreads();
  for (int hb = 1; hb < kD; hb <<= 1) {
    for (int e = tid; e < kPT * kD / 2; e += 256) {
      const int t = e / (kD / 2), pidx = e % (kD / 2);
      const int i0 = (pidx / hb) * 2 * hb + (pidx % hb);
      const float u = x[t][i0], w = x[t][i0 + hb];
      x[t][i0] = u + w;
      x[t][i0 + hb] = u - w;
    }
    __syncthreads();
  }
  for (int e = tid; e < kPT * kD; e += 256) {
    const int t = e / kD, c = e % kD;
    const float nrm = half_bits_to_float(*reinterpret_cast<const uint16_t*>(page + a.L.vnorm + (h * kPT + t) * 2));
    const float v = x[t][c] / (float)kD;
    store_elem(a.v_out, ((int64_t)h * a.n_tokens + lp * kPT + t) * kD + c, (sign_neg(a.v_sign_bits, c) ? -v : v) * nrm,
               a.out_dtype);
  }
}

}  // namespace bmx

using namespace bmx;

extern "C" int bmx_k2b_dequant(const bmx_k2b_dequant_args* a, void* stream) {
  if (!a) { bmx_set_error("bmx_k2b_dequant: args is NULL"); return BMX_E_INVALID; }
  const bmx_k2b_geom& g = a->geom;
  if (g.h_kv < 1 || g.h_kv > 16 || (g.rank != 16 && g.rank != 32)) {
    bmx_set_error("bmx_k2b_dequant: unsupported geometry (h_kv 1..16, rank 16|32)");
    return BMX_E_INVALID;
  }
  if (a->n_tokens < 0 || a->n_tokens % kGroup != 0) {
    bmx_set_error("bmx_k2b_dequant: n_tokens must be a non-negative multiple of 64");
    return BMX_E_INVALID;
  }
  if (a->n_tokens == 0) return BMX_OK;
  if (!a->pages || !a->page_table || !a->basis || !a->k_out || !a->v_out || a->n_pool_pages < 1) {
    bmx_set_error("bmx_k2b_dequant: null pointer argument");
    return BMX_E_INVALID;
  }
  DequantKArgs k{};
  if (a->apply_rope < 0 || a->apply_rope > 2) {
    bmx_set_error("bmx_k2b_dequant: apply_rope must be 0, 1 or 2");
    return BMX_E_INVALID;
  }
  if (a->out_dtype < BMX_K2B_F16 || a->out_dtype > BMX_K2B_BF16) {
    bmx_set_error("bmx_k2b_dequant: out_dtype must be BMX_K2B_F16, _F32 or _BF16");
    return BMX_E_INVALID;
  }
  k.h_kv = g.h_kv; k.R = g.rank; k.n_tokens = a->n_tokens; k.apply_rope = a->apply_rope;
  k.out_dtype = a->out_dtype;
  k.pages = a->pages; k.page_table = a->page_table; k.basis = a->basis; k.n_pool = a->n_pool_pages;
  k.L = PageLayout::make(g.h_kv, g.rank);
  k.rope_scaling = a->rope_scaling;
  for (int j = 0; j < 64; ++j) k.inv_freq[j] = a->inv_freq[j];
  for (int j = 0; j < 4; ++j) { k.codebook[j] = a->codebook[j]; k.v_sign_bits[j] = a->v_sign_bits[j]; }
  k.k_out = a->k_out; k.v_out = a->v_out;
  hipLaunchKernelGGL(k2b_dequant_kernel, dim3(a->n_tokens / kPT, g.h_kv), dim3(256), 0,
                     (hipStream_t)stream, k);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    bmx_set_error(std::string("bmx_k2b_dequant: launch: ") + hipGetErrorString(e));
    return BMX_E_HIP;
  }
  return BMX_OK;
}
