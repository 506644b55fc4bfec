// Quantize-on-append: encode 128-token codec pages of pre-RoPE keys and values
// straight into 16-token physical pages, gfx950.
//
// Three launches per call (all codec pages of the call in each):
//   k2b_us_kernel    Us = M * basis32 (or the first page's SVD factor), fp16
//   k2b_kres_kernel  R = M - Us16 * basis16^T, per-channel 64-token RTN at 3 bits
//   k2b_v_kernel     per (token, head): fp16 norm, sign flip, FWHT, Lloyd codes
// Reference semantics: cache/packed_streaming.py:475-580 (page commit),
// cache/codecs.py:616-636, 677-695, 786-796 (codecs), quant/rtn.py:23-44 (RTN),
// quant/hadamard.py:12-33 (FWHT).  Element-wise steps follow the reference's
// operation order (divide, round-half-even, divide-then-multiply by sqrt(d)) and
// this file is built without floating-point contraction, so codes are identical
// to the reference's whenever the reduction results (Us, the norm) agree.

#include "k2b_common.h"
#include "k2b_general.h"

namespace bmx {

// grid (n_codec_pages * 8), block 256 = 4 waves, one 16-token page slot each.
// Us[t][r] = sum_c M[t][c] basis32[c][r] in fp32 (the reference's M @ V).  The
// page's 16 key rows are staged in LDS (rows padded by one bank); wave w sums
// channels [w C/4, (w+1) C/4) in order, lane (t = lane & 15, quad rq = lane >> 4)
// owns ranks rq R/4 .. + R/4; the four partial sums are then added in wave
// order.  The first codec page of a sequence takes its SVD factor instead.
template <int R>
__global__ __launch_bounds__(256) void k2b_us_kernel(const AppendKArgs a) {
  constexpr int RQ = R / 4;
  extern __shared__ uint16_t s_m[];          // [kPT][C + 2] fp16 key rows
  __shared__ float s_part[4][kPT][R + 1];
  const int pg = blockIdx.x;                  // physical page slot (16 tokens)
  const int cp = pg / 8, pl = pg % 8;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int C = kD * a.h_kv, ld = C + 2;
  uint8_t* page = a.pages + clamp_page(a.page_ids[pg], a.n_pool) * a.L.bytes;
  if (a.us_first != nullptr && cp == 0) {
    for (int e = tid; e < kPT * R; e += 256) {
      const int t = e / R, r = e % R;
      *reinterpret_cast<uint16_t*>(page + a.L.us + us_half(R, t, r) * 2) =
          float_to_half_bits(a.us_first[(pl * kPT + t) * R + r]);
    }
    return;
  }
  for (int e = tid; e < kPT * C; e += 256) {
    const int t = e / C, c = e % C;
    s_m[t * ld + c] = a.k_pre[(c / kD) * a.ksh + (int64_t)(pg * kPT + t) * a.kst + (c % kD)];
  }
  __syncthreads();
  const int t = lane & 15, rq = lane >> 4;
  float acc[RQ];
#pragma unroll
  for (int k = 0; k < RQ; ++k) acc[k] = 0.f;
  const int c0 = wave * (C / 4), c1 = c0 + C / 4;
#pragma unroll 4
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
    const float us = ((s_part[0][tt][r] + s_part[1][tt][r]) + s_part[2][tt][r]) + s_part[3][tt][r];
    *reinterpret_cast<uint16_t*>(page + a.L.us + us_half(R, tt, r) * 2) = float_to_half_bits(us);
  }
}

// grid (n_codec_pages * 2 groups, h_kv), block 256: 64 tokens x 128 channels.
__global__ __launch_bounds__(256) void k2b_kres_kernel(const AppendKArgs a) {
  const int gi = blockIdx.x;        // 64-token group index within the call
  const int h = blockIdx.y;
  const int cp = gi / 2, grp_in = gi % 2;
  const int C = kD * a.h_kv;
  const int R = a.R;
  __shared__ float s_us[kGroup][33];
  __shared__ float s_b[kD][33];
  __shared__ float s_amax[2][kD];
  __shared__ int8_t s_code[kGroup][kD + 4];

  const int tid = threadIdx.x;
  // Us16 of the group's 64 tokens (already written to the 4 pages)
  for (int e = tid; e < kGroup * R; e += 256) {
    const int t = e / R, r = e % R;
    const int pslot = cp * 8 + grp_in * 4 + t / kPT;
    const uint8_t* page = a.pages + clamp_page(a.page_ids[pslot], a.n_pool) * a.L.bytes;
    s_us[t][r] = half_bits_to_float(*reinterpret_cast<const uint16_t*>(page + a.L.us + us_half(R, t % kPT, r) * 2));
  }
  for (int e = tid; e < kD * R; e += 256) {
    const int j = e / R, r = e % R;
    s_b[j][r] = half_bits_to_float(a.basis16[(int64_t)(h * kD + j) * R + r]);
  }
  __syncthreads();

  const int j = tid & 127, half = tid >> 7;
  float res[32];
  float amax = 0.f;
#pragma unroll
  for (int tt = 0; tt < 32; ++tt) {
    const int t = half * 32 + tt;                                  // token within group
    const int tg = cp * kCodec + grp_in * kGroup + t;             // token within call
    float L = 0.f;
    for (int r = 0; r < R; ++r) L = __builtin_fmaf(s_us[t][r], s_b[j][r], L);
    const float m = half_bits_to_float(a.k_pre[h * a.ksh + (int64_t)tg * a.kst + j]);
    res[tt] = m - L;
    amax = fmaxf(amax, fabsf(res[tt]));
  }
  s_amax[half][j] = amax;
  __syncthreads();
  const float scale = fmaxf(fmaxf(s_amax[0][j], s_amax[1][j]), 1e-12f) / 3.0f;
#pragma unroll
  for (int tt = 0; tt < 32; ++tt) {
    float cq = rintf(res[tt] / scale);
    cq = fminf(fmaxf(cq, -4.0f), 3.0f);
    s_code[half * 32 + tt][j] = (int8_t)cq;
  }
  if (half == 0) {
    const int f = kscale_flat(h * kD + j), quarter = C / 4;
    const int slot = f / quarter, off = f % quarter;
    uint8_t* page = a.pages + clamp_page(a.page_ids[cp * 8 + grp_in * 4 + slot], a.n_pool) * a.L.bytes;
    *reinterpret_cast<uint16_t*>(page + a.L.kscale + off * 2) = float_to_half_bits(scale);
  }
  __syncthreads();
  // pack: thread -> (page pl, lane 16q+n); pair p = 4b+i is channels (j, j+64),
  // j = 16b + 4q + i, stored offset-binary
  {
    const int pl = tid >> 6, lane = tid & 63, q = lane >> 4, n = lane & 15;
    const int t = pl * kPT + n;
    uint32_t w[3] = {0u, 0u, 0u};
#pragma unroll
    for (int p = 0; p < 16; ++p) {
      const int jj = 16 * (p >> 2) + 4 * q + (p & 3);
      const uint32_t lo = (uint32_t)(s_code[t][jj] + 4), hi = (uint32_t)(s_code[t][jj + 64] + 4);
      if (p < 15) {
        w[p / 5] |= (lo << (3 * (p % 5))) | (hi << (16 + 3 * (p % 5)));
      } else {
#pragma unroll
        for (int k = 0; k < 3; ++k) w[k] |= (((lo >> k) & 1u) << 15) | (((hi >> k) & 1u) << 31);
      }
    }
    uint8_t* page = a.pages + clamp_page(a.page_ids[cp * 8 + grp_in * 4 + pl], a.n_pool) * a.L.bytes;
    uint32_t* dst = reinterpret_cast<uint32_t*>(page + a.L.kres + h * 768 + lane * 12);
    dst[0] = w[0]; dst[1] = w[1]; dst[2] = w[2];
  }
}

// grid (n_codec_pages * 8, h_kv), block 256: 16 tokens x 128 channels.
__global__ __launch_bounds__(256) void k2b_v_kernel(const AppendKArgs a) {
  const int pg = blockIdx.x, h = blockIdx.y;
  const int tid = threadIdx.x;
  __shared__ float x[kPT][kD];
  __shared__ float s_norm[kPT];
  __shared__ uint8_t code[kPT][kD];
  uint8_t* page = a.pages + clamp_page(a.page_ids[pg], a.n_pool) * a.L.bytes;

  for (int e = tid; e < kPT * kD; e += 256) {
    const int t = e / kD, c = e % kD;
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
  // norms: one thread per token, in the order torch's CPU 2-norm reduces a
  // 128-float row (8 strided FMA accumulators, then a left-to-right sum, then a
  // correctly rounded sqrt), so the fp16 norm is identical to the reference's
  if (tid < kPT) {
    const int t = tid;
    float acc8[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc8[j] = 0.f;
    for (int i = 0; i < kD; i += 8) {
#pragma unroll
      for (int j = 0; j < 8; ++j) acc8[j] = __builtin_fmaf(x[t][i + j], x[t][i + j], acc8[j]);
    }
    float ss = acc8[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) ss = ss + acc8[j];
    {
      const float nrm = fmaxf(__builtin_sqrtf(ss), 1e-12f);
      const uint16_t nb = float_to_half_bits(nrm);
      s_norm[t] = half_bits_to_float(nb);
      *reinterpret_cast<uint16_t*>(page + a.L.vnorm + (h * kPT + t) * 2) = nb;
    }
  }
  __syncthreads();
  for (int e = tid; e < kPT * kD; e += 256) {
    const int t = e / kD, c = e % kD;
    const float u = x[t][c] / s_norm[t];
    x[t][c] = sign_neg(a.v_sign_bits, c) ? -u : u;
  }
  __syncthreads();
  // FWHT stages (i, i+hb) inside blocks of 2hb, as quant/hadamard.py:19-25
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
  const float sqrt_d = 11.313708498984761f;  // fl32(sqrt(128)), applied as / then *
  const float mid0 = (a.codebook[0] + a.codebook[1]) / 2.0f;
  const float mid1 = (a.codebook[1] + a.codebook[2]) / 2.0f;
  const float mid2 = (a.codebook[2] + a.codebook[3]) / 2.0f;
  for (int e = tid; e < kPT * kD; e += 256) {
    const int t = e / kD, c = e % kD;
    const float r = (x[t][c] / sqrt_d) * sqrt_d;
    code[t][c] = (uint8_t)((r > mid0) + (r > mid1) + (r > mid2));
  }
  __syncthreads();
  if (tid < 128) {  // lane 16q+m, dword w: channel 16b + m (b = 4w + bb), token 4q + t at bit 8bb + 2t
    const int lane = tid >> 1, w = tid & 1, q = lane >> 4, m = lane & 15;
    uint32_t dword = 0;
    for (int bb = 0; bb < 4; ++bb) {
      const int c = 16 * (4 * w + bb) + m;
      for (int t = 0; t < 4; ++t) dword |= (uint32_t)code[4 * q + t][c] << (8 * bb + 2 * t);
    }
    *reinterpret_cast<uint32_t*>(page + a.L.vcode + h * 512 + lane * 8 + w * 4) = dword;
  }
}

// The value kernel alone, for pages whose layout has value sections only
// (the spectral key path keeps its keys in pages of its own).
hipError_t launch_k2b_values(const AppendKArgs& a, int n_pages16, int h_kv, hipStream_t st) {
  hipLaunchKernelGGL(k2b_v_kernel, dim3(n_pages16, h_kv), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace bmx

using namespace bmx;

static int afail(int code, const std::string& msg) {
  bmx_set_error(msg);
  return code;
}

// The Us kernel stages 16 key rows of C channels in LDS: above 64 KB (h_kv 16)
// the launch needs the larger dynamic-LDS limit set once.
template <int R>
static hipError_t launch_us(const AppendKArgs& k, dim3 grid, size_t lds, hipStream_t st) {
  if (lds > 65536) {
    const hipError_t e = bmx_ensure_dynamic_lds((const void*)k2b_us_kernel<R>, lds);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(k2b_us_kernel<R>, grid, dim3(256), lds, st, k);
  return hipGetLastError();
}

extern "C" int bmx_k2b_append(const bmx_k2b_append_args* a, void* stream) {
  if (!a) return afail(BMX_E_INVALID, "bmx_k2b_append: args is NULL");
  const bmx_k2b_geom& g = a->geom;
  const Geo geo = Geo::from(g);
  if (g.h_kv < 1 || g.h_kv > 16) return afail(BMX_E_INVALID, "bmx_k2b_append: h_kv must be 1..16");
  if (!geo.general && g.rank != 16 && g.rank != 32)
    return afail(BMX_E_INVALID, "bmx_k2b_append: rank must be 16 or 32");
  if (geo.general && !geo.check().empty()) return afail(BMX_E_INVALID, "bmx_k2b_append: " + geo.check());
  if (a->n_codec_pages < 0) return afail(BMX_E_INVALID, "bmx_k2b_append: n_codec_pages < 0");
  if (a->n_codec_pages == 0) return BMX_OK;
  if (!a->k_pre || !a->v || !a->basis32 || !a->basis16 || !a->pages || !a->page_ids)
    return afail(BMX_E_INVALID, "bmx_k2b_append: null pointer argument");
  if (a->n_pool_pages < 1) return afail(BMX_E_INVALID, "bmx_k2b_append: n_pool_pages must be >= 1");
  if (reinterpret_cast<uintptr_t>(a->basis32) % 16 != 0)
    return afail(BMX_E_INVALID, "bmx_k2b_append: basis32 must be 16-byte aligned");
  if (a->v_dtype != BMX_K2B_F16 && a->v_dtype != BMX_K2B_F32 && a->v_dtype != BMX_K2B_BF16)
    return afail(BMX_E_INVALID, "bmx_k2b_append: v_dtype must be BMX_K2B_F16, _F32 or _BF16");
  if (geo.general) return gen_append(a, (hipStream_t)stream);
  AppendKArgs k{};
  k.h_kv = g.h_kv; k.R = g.rank; k.n_codec_pages = a->n_codec_pages;
  k.k_pre = a->k_pre; k.ksh = a->k_stride_h; k.kst = a->k_stride_t;
  k.v = a->v; k.vsh = a->v_stride_h; k.vst = a->v_stride_t; k.v_dtype = a->v_dtype;
  k.basis32 = a->basis32; k.basis16 = a->basis16; k.us_first = a->us_first;
  k.pages = a->pages; k.page_ids = a->page_ids; k.n_pool = a->n_pool_pages;
  k.L = PageLayout::make(g.h_kv, g.rank);
  for (int i = 0; i < 4; ++i) { k.codebook[i] = a->codebook[i]; k.v_sign_bits[i] = a->v_sign_bits[i]; }
  hipStream_t st = (hipStream_t)stream;
  const size_t us_lds = (size_t)kPT * (kD * g.h_kv + 2) * 2;
  hipError_t le = g.rank == 32 ? launch_us<32>(k, dim3(a->n_codec_pages * 8), us_lds, st)
                               : launch_us<16>(k, dim3(a->n_codec_pages * 8), us_lds, st);
  if (le != hipSuccess) return afail(BMX_E_HIP, std::string("bmx_k2b_append: launch: ") + hipGetErrorString(le));
  hipLaunchKernelGGL(k2b_kres_kernel, dim3(a->n_codec_pages * 2, g.h_kv), dim3(256), 0, st, k);
  hipLaunchKernelGGL(k2b_v_kernel, dim3(a->n_codec_pages * 8, g.h_kv), dim3(256), 0, st, k);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return afail(BMX_E_HIP, std::string("bmx_k2b_append: launch: ") + hipGetErrorString(e));
  return BMX_OK;
}
