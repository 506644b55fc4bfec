// Dense dequantization of committed k2b pages (prefill path and checks), gfx950.
// Reference semantics: cache/chunked_attention.py:52-194 (_dequant_block,
// _dense_kv), cache/codecs.py:639-649, 839-842 (dequant_packed).

#include "k2b_common.h"
#include "k2b_general.h"

namespace bmx {

struct DequantKArgs {
  int h_kv, R, n_tokens, apply_rope, n_pool, out_dtype;
  int pos0;          // position of the first listed token
  int64_t out_rows;  // rows between consecutive heads in k_out / v_out
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

// One wave per (16-token page, head), four heads per workgroup; grid
// (n_tokens / 16, ceil(h_kv / 4)), block 256.  The wave does a decode
// kernel's page work once, in fp32:
//   keys: K^T = basis_h * Us^T on MFMA (lane 16q + n: token n, channels
//   j = 16bb + 4q + i and j + 64), plus code * scale (the 3-bit codes as exact
//   fp16 integers), then RoPE from the page's cos/sin table, shared by the
//   workgroup's heads;
//   values: the lane's code bytes (channel 16b + n, tokens 4q .. 4q + 3) give
//   codebook levels, H8 over b in registers and H16 over n across the row's
//   lanes make the 128-point Hadamard, then 1/128, signs and the norm;
// each tile goes through a per-wave LDS staging tile (the output's 16-bit
// bits for fp16 / bf16, else fp32: 26 or 43 KB a workgroup with the table)
// so that the dense rows are written with 16-byte coalesced stores, rounded
// once to the output type.  At 16-bit tiles and 5 waves per SIMD (at most
// 102 VGPRs) an 8k-token prefill's 1,072 workgroups are all resident at once.
// The codebook levels and the first H8 stage come from a 16-entry pair table
// (dq_value_tile_lut), the key's code * scale + low-rank part is one fma.
// Only the cos/sin table is shared between waves; a wave's own tile is
// ordered by its own LDS waits.
constexpr int kDqWaves = 4;

template <int R, class Tile>
__global__ __launch_bounds__(64 * kDqWaves) __attribute__((amdgpu_waves_per_eu(5)))
void k2b_dequant_kernel(const DequantKArgs a) {
  constexpr int KQ = R / 4;
  typedef _Float16 hvec_t __attribute__((ext_vector_type(KQ)));
  const int lp = blockIdx.x;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, n = lane & 15, q = lane >> 4;
  const int h_raw = blockIdx.y * kDqWaves + wave;
  const bool active = h_raw < a.h_kv;
  const int h = active ? h_raw : 0;
  const int C = kD * a.h_kv, quarter = C / 4;
  __shared__ __align__(16) float s_cs[2][kPT][kCsPad];   // rows padded: conflict-free 16-byte reads
  __shared__ Tile s_tile[kDqWaves];
  __shared__ DqPairLut s_lut;

  // ---- every load first ----
  const uint8_t* page = a.pages + clamp_page(a.page_table[lp], a.n_pool) * a.L.bytes;
  const hvec_t us = *reinterpret_cast<const hvec_t*>(page + a.L.us + lane * (2 * KQ));
  const uint3 kres = *reinterpret_cast<const uint3*>(page + a.L.kres + h * 768 + lane * 12);
  const uint2 vcd = *reinterpret_cast<const uint2*>(page + a.L.vcode + h * 512 + lane * 8);
  const uint2 nrm = *reinterpret_cast<const uint2*>(page + a.L.vnorm + (h * kPT + 4 * q) * 2);
  uint4 scl[4];   // key-scale pairs (s_j, s_{j+64}), j = 16bb + 4q + i, in the group's pages
#pragma unroll
  for (int bb = 0; bb < 4; ++bb) {
    const int f = h * kD + 2 * (16 * bb + 4 * q);
    const int slot = f / quarter, off = f - slot * quarter;
    const uint8_t* sp = a.pages + clamp_page(a.page_table[(lp & ~3) + slot], a.n_pool) * a.L.bytes;
    scl[bb] = *reinterpret_cast<const uint4*>(sp + a.L.kscale + 2 * off);
  }
  hvec_t vh[8];
#pragma unroll
  for (int bt = 0; bt < 8; ++bt)
    vh[bt] = *reinterpret_cast<const hvec_t*>(a.basis + (int64_t)(h * kD + 16 * bt + n) * R + KQ * q);

  // ---- the page's cos/sin: HF's fp32 angle fl(inv_freq_j * pos) ----
  if (a.apply_rope) {
#pragma unroll
    for (int k = 0; k < kPT * 64 / (64 * kDqWaves); ++k) {
      const int e = tid + 64 * kDqWaves * k, t = e >> 6, j = e & 63;
      float sn, cn;
      sincosf(a.inv_freq[j] * (float)(a.pos0 + lp * kPT + t), &sn, &cn);
      cn *= a.rope_scaling;
      sn *= a.rope_scaling;
      if (a.apply_rope == 2) {   // the reference's fp16 tables
        cn = half_bits_to_float(float_to_half_bits(fp32_rounded(cn)));
        sn = half_bits_to_float(float_to_half_bits(fp32_rounded(sn)));
      }
      s_cs[0][t][j] = cn;
      s_cs[1][t][j] = sn;
    }
  }

  // ---- keys ----
  float4_t kt[8];
#pragma unroll
  for (int bt = 0; bt < 8; ++bt) {
    const float4_t z = {0.f, 0.f, 0.f, 0.f};
    if constexpr (R == 32)
      kt[bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh[bt], us, z, 0, 0, 0);
    else
      kt[bt] = __builtin_amdgcn_mfma_f32_16x16x16f16(vh[bt], us, z, 0, 0, 0);
  }
  dq_pair_lut_build(s_lut, a.codebook);
  KresMasks km;
  km.init();
  half2_t cp[16];
  kres_pairs(km, kres.x, kres.y, kres.z, cp);
  __syncthreads();   // s_cs
  Tile& tl = s_tile[wave];
#pragma unroll
  for (int bb = 0; bb < 4; ++bb) {
    const uint32_t sv[4] = {scl[bb].x, scl[bb].y, scl[bb].z, scl[bb].w};
    const float4_t c4 = *reinterpret_cast<const float4_t*>(&s_cs[0][n][16 * bb + 4 * q]);
    const float4_t s4 = *reinterpret_cast<const float4_t*>(&s_cs[1][n][16 * bb + 4 * q]);
    float o0[4], o1[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const half2_t s2 = as_h2(sv[i]);
      // L + code * scale in fp32: the product is exact, so the fma rounds as the sum does
      float k0 = __builtin_fmaf((float)cp[4 * bb + i][0], (float)s2[0], kt[bb][i]);
      float k1 = __builtin_fmaf((float)cp[4 * bb + i][1], (float)s2[1], kt[bb + 4][i]);
      if (a.apply_rope) {
        const float c = c4[i], sn = s4[i];
        // x*cos + rotate_half(x)*sin, rounded per operation as torch does
        const float r0 = __fmul_rn(k0, c) - __fmul_rn(k1, sn);
        k1 = __fmul_rn(k1, c) + __fmul_rn(k0, sn);
        k0 = r0;
      }
      o0[i] = k0;
      o1[i] = k1;
    }
    tile_put4(tl, n, 16 * bb + 4 * q, o0, a.out_dtype);
    tile_put4(tl, n, 16 * bb + 4 * q + 64, o1, a.out_dtype);
  }
  wave_lds_order();
  const int64_t row0 = (int64_t)h * a.out_rows + (int64_t)lp * kPT;
  if (active) dq_store_tile(tl, a.k_out, row0, a.out_dtype);
  wave_lds_order();   // the staging tile is reused for the values

  dq_value_tile_lut(vcd, nrm, s_lut, a.v_sign_bits, n, q, tl, a.out_dtype);
  wave_lds_order();
  if (active) dq_store_tile(tl, a.v_out, row0, a.out_dtype);
}

}  // namespace bmx

using namespace bmx;

extern "C" int bmx_k2b_dequant(const bmx_k2b_dequant_args* a, void* stream) {
  if (!a) { bmx_set_error("bmx_k2b_dequant: args is NULL"); return BMX_E_INVALID; }
  const bmx_k2b_geom& g = a->geom;
  const Geo geo = Geo::from(g);
  if (g.h_kv < 1 || g.h_kv > 16 || (!geo.general && g.rank != 16 && g.rank != 32)) {
    bmx_set_error("bmx_k2b_dequant: unsupported geometry (h_kv 1..16, rank 16|32)");
    return BMX_E_INVALID;
  }
  if (geo.general && !geo.check().empty()) {
    bmx_set_error("bmx_k2b_dequant: " + geo.check());
    return BMX_E_INVALID;
  }
  if (a->n_tokens < 0 || a->n_tokens % geo.group != 0) {
    bmx_set_error("bmx_k2b_dequant: n_tokens must be a non-negative multiple of the residual group");
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
  if (a->pos0 < 0 || (a->out_rows != 0 && a->out_rows < a->n_tokens)) {
    bmx_set_error("bmx_k2b_dequant: pos0 must be >= 0 and out_rows 0 or >= n_tokens");
    return BMX_E_INVALID;
  }
  if (geo.general) return gen_dequant(a, (hipStream_t)stream);
  k.h_kv = g.h_kv; k.R = g.rank; k.n_tokens = a->n_tokens; k.apply_rope = a->apply_rope;
  k.out_dtype = a->out_dtype;
  k.pages = a->pages; k.page_table = a->page_table; k.basis = a->basis; k.n_pool = a->n_pool_pages;
  k.L = PageLayout::make(g.h_kv, g.rank);
  k.rope_scaling = a->rope_scaling;
  for (int j = 0; j < 64; ++j) k.inv_freq[j] = a->inv_freq[j];
  for (int j = 0; j < 4; ++j) { k.codebook[j] = a->codebook[j]; k.v_sign_bits[j] = a->v_sign_bits[j]; }
  k.k_out = a->k_out; k.v_out = a->v_out;
  k.pos0 = a->pos0;
  k.out_rows = a->out_rows ? a->out_rows : a->n_tokens;
  const dim3 grid(a->n_tokens / kPT, (g.h_kv + kDqWaves - 1) / kDqWaves);
  const hipStream_t st = (hipStream_t)stream;
  const dim3 block(64 * kDqWaves);
  switch (a->out_dtype * 2 + (g.rank == 32)) {
    case BMX_K2B_F16 * 2 + 1: hipLaunchKernelGGL((k2b_dequant_kernel<32, DqTile16<BMX_K2B_F16>>), grid, block, 0, st, k); break;
    case BMX_K2B_F16 * 2: hipLaunchKernelGGL((k2b_dequant_kernel<16, DqTile16<BMX_K2B_F16>>), grid, block, 0, st, k); break;
    case BMX_K2B_BF16 * 2 + 1: hipLaunchKernelGGL((k2b_dequant_kernel<32, DqTile16<BMX_K2B_BF16>>), grid, block, 0, st, k); break;
    case BMX_K2B_BF16 * 2: hipLaunchKernelGGL((k2b_dequant_kernel<16, DqTile16<BMX_K2B_BF16>>), grid, block, 0, st, k); break;
    case BMX_K2B_F32 * 2 + 1: hipLaunchKernelGGL((k2b_dequant_kernel<32, DqTile>), grid, block, 0, st, k); break;
    default: hipLaunchKernelGGL((k2b_dequant_kernel<16, DqTile>), grid, block, 0, st, k); break;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    bmx_set_error(std::string("bmx_k2b_dequant: launch: ") + hipGetErrorString(e));
    return BMX_E_HIP;
  }
  return BMX_OK;
}
