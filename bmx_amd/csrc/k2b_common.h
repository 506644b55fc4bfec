// Shared definitions of the gfx950 k2b kernels: page geometry, fp16 helpers,
// MFMA fragment types and the error channel of the C-ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "bmx_k2b.h"

namespace bmx {

constexpr int kPT = 16;      // tokens per physical page
constexpr int kD = 128;      // head_dim
constexpr int kGroup = 64;   // tokens per key-scale group
constexpr int kCodec = 128;  // tokens per codec page

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// Byte offsets of the five page sections (see include/bmx_k2b.h).
struct PageLayout {
  int32_t us, vnorm, kscale, kres, vcode, bytes;
  __host__ __device__ static PageLayout make(int h_kv, int rank) {
    PageLayout L;
    const int C = kD * h_kv;
    L.us = 0;
    L.vnorm = L.us + kPT * rank * 2;
    L.kscale = L.vnorm + h_kv * kPT * 2;
    L.kres = L.kscale + (C / 4) * 2;
    L.vcode = L.kres + h_kv * 64 * 12;
    L.bytes = L.vcode + h_kv * 64 * 8;
    return L;
  }
};

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
  _Float16 v;
  __builtin_memcpy(&v, &h, 2);
  return (float)v;
}

__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
  _Float16 v = (_Float16)f;  // round to nearest even
  uint16_t h;
  __builtin_memcpy(&h, &v, 2);
  return h;
}

__device__ __forceinline__ uint32_t half_bits(_Float16 v) {
  uint16_t h;
  __builtin_memcpy(&h, &v, 2);
  return h;
}

// Element idx of a dense output in dtype BMX_K2B_F32 / _F16 / _BF16 (fp16 and
// bf16 round to nearest even, as torch's casts do).
__device__ __forceinline__ void store_elem(void* base, int64_t idx, float v, int dtype) {
  if (dtype == 1) {   // BMX_K2B_F32
    reinterpret_cast<float*>(base)[idx] = v;
  } else if (dtype == 2) {   // BMX_K2B_BF16
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    u = (u & 0x7fffffffu) > 0x7f800000u ? (u | 0x00400000u) : u + 0x7fffu + ((u >> 16) & 1u);
    reinterpret_cast<uint16_t*>(base)[idx] = (uint16_t)(u >> 16);
  } else {
    reinterpret_cast<uint16_t*>(base)[idx] = float_to_half_bits(v);
  }
}

// v as computed in fp32, opaque to the compiler: a product that made v is not
// fused with a later conversion to 16 bits (v_fma_mix*, one rounding), so the
// conversion rounds the fp32 value, as a stored fp32 tensor converted later.
__device__ __forceinline__ float fp32_rounded(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

__device__ __forceinline__ half2_t as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t as_u32(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

// The masks arrive in VGPRs (KresMasks) so each half pair is one v_and_or_b32.
struct KresMasks {
  uint32_t m0, m1, m2;   // code bits of slots 0, 3, 6 (both halves)
  uint32_t e0, e1, e2;   // exponent fields 25, 22, 19 (both halves)
  __device__ __forceinline__ void init() {
    m0 = 0x00070007u; m1 = 0x00380038u; m2 = 0x01C001C0u;
    e0 = 0x64006400u; e1 = 0x58005800u; e2 = 0x4C004C00u;
    // opaque to the optimiser: keeps them in registers, out of literal operands
    asm volatile("" : "+v"(m0), "+v"(m1), "+v"(m2));
    asm volatile("" : "+s"(e0), "+s"(e1), "+s"(e2));
  }
};

// The lane's 16 key-residual pairs (channels j, j+64) as exact fp16 integers.
// An offset-binary 3-bit code c' at mantissa bits [s, s+3) under exponent field
// 25 - s reads as 2^(10-s) + c'; one AND-OR builds two such halves and one
// packed add removes 2^(10-s) + 4, leaving code = c' - 4.
__device__ __forceinline__ void kres_pairs(const KresMasks& km, uint32_t w0, uint32_t w1, uint32_t w2,
                                           half2_t c[16]) {
  const half2_t b0 = {(_Float16)-1028.0f, (_Float16)-1028.0f};
  const half2_t b1 = {(_Float16)-132.0f, (_Float16)-132.0f};
  const half2_t b2 = {(_Float16)-20.0f, (_Float16)-20.0f};
  const uint32_t w[3] = {w0, w1, w2};
#pragma unroll
  for (int d = 0; d < 3; ++d) {
    const uint32_t x = w[d], y = x >> 9;
    c[5 * d + 0] = as_h2((x & km.m0) | km.e0) + b0;
    c[5 * d + 1] = as_h2((x & km.m1) | km.e1) + b1;
    c[5 * d + 2] = as_h2((x & km.m2) | km.e2) + b2;
    c[5 * d + 3] = as_h2((y & km.m0) | km.e0) + b0;
    c[5 * d + 4] = as_h2((y & km.m1) | km.e1) + b1;
  }
  c[15] = as_h2(((w0 >> 15) & 0x00010001u) | ((w1 >> 14) & 0x00020002u) |
                ((w2 >> 13) & 0x00040004u) | km.e0) + b0;
}

// Pair P (0..15) of kres_pairs alone, for a caller that decodes the pairs
// just before it uses them.
template <int P>
__device__ __forceinline__ half2_t kres_pair(const KresMasks& km, uint32_t w0, uint32_t w1, uint32_t w2) {
  const half2_t b0 = {(_Float16)-1028.0f, (_Float16)-1028.0f};
  const half2_t b1 = {(_Float16)-132.0f, (_Float16)-132.0f};
  const half2_t b2 = {(_Float16)-20.0f, (_Float16)-20.0f};
  if constexpr (P == 15) {
    return as_h2(((w0 >> 15) & 0x00010001u) | ((w1 >> 14) & 0x00020002u) | ((w2 >> 13) & 0x00040004u) | km.e0) + b0;
  } else {
    constexpr int d = P / 5, k = P % 5;
    const uint32_t x = d == 0 ? w0 : d == 1 ? w1 : w2;
    if constexpr (k == 0) return as_h2((x & km.m0) | km.e0) + b0;
    if constexpr (k == 1) return as_h2((x & km.m1) | km.e1) + b1;
    if constexpr (k == 2) return as_h2((x & km.m2) | km.e2) + b2;
    if constexpr (k == 3) return as_h2(((x >> 9) & km.m0) | km.e0) + b0;
    return as_h2(((x >> 9) & km.m1) | km.e1) + b1;
  }
}

// Physical page id clamped into the pool: a corrupt table entry cannot fault.
__device__ __forceinline__ int64_t clamp_page(int32_t pid, int32_t n_pool) {
  return (int64_t)min(max(pid, 0), n_pool - 1);
}

// V-codec sign of channel c (true -> -1).
__device__ __forceinline__ bool sign_neg(const uint32_t bits[4], int c) {
  return (bits[c >> 5] >> (c & 31)) & 1u;
}

// US: half index of (token t, rank r); lane 16q+n of an MFMA reads R/4 halfs
// Us[n][(R/4)q ..] contiguously.
__host__ __device__ __forceinline__ int us_half(int R, int t, int r) {
  const int kpl = R / 4;
  return ((r / kpl) * kPT + t) * kpl + r % kpl;
}

// KSCALE: position of channel c (0..C-1) in the group's pair-ordered scale
// array F (F[128h + 2j + e] = scale of channel 128h + j + 64e).
__host__ __device__ __forceinline__ int kscale_flat(int c) {
  const int j = c & (kD - 1);
  return (c - j) + 2 * (j & 63) + (j >> 6);
}

// KRES: signed residual code of pair p (0..15), half e (0: channel j, 1: j+64)
// from the lane's three dwords (offset-binary 3-bit codes).
__device__ __forceinline__ int kres_pair_code(uint32_t w0, uint32_t w1, uint32_t w2, int p, int e) {
  uint32_t v;
  if (p < 15) {
    const uint32_t w = p < 5 ? w0 : (p < 10 ? w1 : w2);
    v = (w >> (3 * (p % 5) + 16 * e)) & 7u;
  } else {
    const int sh = 15 + 16 * e;
    v = ((w0 >> sh) & 1u) | (((w1 >> sh) & 1u) << 1) | (((w2 >> sh) & 1u) << 2);
  }
  return (int)v - 4;
}

constexpr int kDqPad = kD + 4;   // staging row stride (floats)
constexpr int kDqPad16 = kD + 8; // staging row stride (16-bit elements): 272-byte rows, 16-byte aligned
constexpr int kCsPad = 68;       // cos/sin table row stride (floats): 16-byte reads of 16 rows hit distinct banks

// A wave's 16-token staging tile: fp32 (fp32 output) or the output's 16-bit
// bits (DT = BMX_K2B_F16 or BMX_K2B_BF16 output: each value rounded once,
// when it is put).
struct DqTile {
  float v[kPT][kDqPad];
};
template <int DT>
struct DqTile16 {
  uint16_t v[kPT][kDqPad16];
};

// Order a wave's LDS writes before its later LDS reads (of other lanes'
// data): no compiler motion across it, every LDS operation of the wave done.
__device__ __forceinline__ void wave_lds_order() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ uint16_t to_bits16(float v, int dtype) {
  if (dtype == 2) {   // BMX_K2B_BF16
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    u = (u & 0x7fffffffu) > 0x7f800000u ? (u | 0x00400000u) : u + 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
  }
  return float_to_half_bits(v);
}

__device__ __forceinline__ void tile_put(DqTile& tl, int t, int c, float v, int) { tl.v[t][c] = v; }
// the value rounded to fp32, then to 16 bits (as an fp32 tile stored and
// converted later)
template <int DT>
__device__ __forceinline__ void tile_put(DqTile16<DT>& tl, int t, int c, float v, int) {
  tl.v[t][c] = to_bits16(fp32_rounded(v), DT);
}

// channels c .. c + 3 (c a multiple of 4) of row t
__device__ __forceinline__ void tile_put4(DqTile& tl, int t, int c, const float (&v)[4], int) {
  *reinterpret_cast<float4_t*>(&tl.v[t][c]) = float4_t{v[0], v[1], v[2], v[3]};
}
template <int DT>
__device__ __forceinline__ void tile_put4(DqTile16<DT>& tl, int t, int c, const float (&v)[4], int) {
  uint16_t b[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) b[i] = to_bits16(fp32_rounded(v[i]), DT);
  *reinterpret_cast<uint2*>(&tl.v[t][c]) = make_uint2(b[0] | (uint32_t)b[1] << 16, b[2] | (uint32_t)b[3] << 16);
}

// row t = lane / 4, columns 32 (lane % 4) .. + 31 of the wave's staging tile
// to out rows base + t (elements of dtype)
__device__ __forceinline__ void dq_store_tile(const DqTile& tl, void* out, int64_t row0, int dtype) {
  const int lane = threadIdx.x & 63, t = lane >> 2, c0 = 32 * (lane & 3);
  const float* src = &tl.v[t][c0];
  const int64_t e0 = (row0 + t) * kD + c0;
  if (dtype == 1) {   // BMX_K2B_F32
    float4_t* dst = reinterpret_cast<float4_t*>(reinterpret_cast<float*>(out) + e0);
#pragma unroll
    for (int u = 0; u < 8; ++u) dst[u] = *reinterpret_cast<const float4_t*>(src + 4 * u);
  } else {
    uint4* dst = reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(out) + e0);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      uint16_t hbits[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) hbits[e] = to_bits16(src[8 * u + e], dtype);
      dst[u] = make_uint4(hbits[0] | (uint32_t)hbits[1] << 16, hbits[2] | (uint32_t)hbits[3] << 16,
                          hbits[4] | (uint32_t)hbits[5] << 16, hbits[6] | (uint32_t)hbits[7] << 16);
    }
  }
}
template <int DT>
__device__ __forceinline__ void dq_store_tile(const DqTile16<DT>& tl, void* out, int64_t row0, int) {
  const int lane = threadIdx.x & 63, t = lane >> 2, c0 = 32 * (lane & 3);
  const uint4* src = reinterpret_cast<const uint4*>(&tl.v[t][c0]);
  uint4* dst = reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(out) + (row0 + t) * kD + c0);
#pragma unroll
  for (int u = 0; u < 4; ++u) dst[u] = src[u];
}

// Arguments of the k2b write kernels (k2b_append.hip).
struct AppendKArgs {
  int h_kv, R, n_codec_pages, n_pool;
  const uint16_t* k_pre;
  int64_t ksh, kst;
  const void* v;
  int64_t vsh, vst;
  int v_dtype;         // BMX_K2B_F16 / F32 / BF16
  const float* basis32;
  const uint16_t* basis16;
  const float* us_first;
  uint8_t* pages;
  const int32_t* page_ids;
  PageLayout L;
  float codebook[4];
  uint32_t v_sign_bits[4];
};

// k2b_v_kernel over n_pages16 16-token pages of h_kv heads: norms and codes
// into the VNORM and VCODE sections of a.L (k2b_append.hip).
hipError_t launch_k2b_values(const AppendKArgs& a, int n_pages16, int h_kv, hipStream_t st);

// Values of one 16-token page of one head into the wave's staging tile: the
// lane's code bytes (channel 16b + n, tokens 4q .. 4q + 3) give codebook
// levels, H8 over b in registers and H16 over n across the row's lanes make
// the 128-point Hadamard, then 1/128, the signs and the token's norm.
// level c (0..3) of four held in registers: a select chain, no indexed load
// (an array indexed by a lane-varying code would be read from memory)
__device__ __forceinline__ float level4(uint32_t c, float l0, float l1, float l2, float l3) {
  const float lo = (c & 1u) ? l1 : l0, hi = (c & 1u) ? l3 : l2;
  return (c & 2u) ? hi : lo;
}

// x of lane n ^ HB of the lane's 16-lane row (HB 1, 2, 4 or 8), by DPP:
// quad_perm [1,0,3,2] and [2,3,0,1] for bits 0 and 1; bit 2 as the half-row
// mirror (n ^ 7) followed by quad_perm [3,2,1,0] (^ 3); bit 3 as a row
// rotation by 8.
template <int HB>
__device__ __forceinline__ float xor_row16(float x) {
  const int v = __builtin_bit_cast(int, x);
  if constexpr (HB == 1) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true));
  if constexpr (HB == 2) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, true));
  if constexpr (HB == 4)
    return __builtin_bit_cast(
        float, __builtin_amdgcn_mov_dpp(__builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, true), 0x1B, 0xF, 0xF, true));
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(v, 0x128, 0xF, 0xF, true));
}

// one stage of H16 over n across the row: (y, partner o) -> y + o on the
// lanes with bit HB of n clear, o - y on the others, as o + s y with s = +-1
// (s y exact: the same one rounding as either sum)
template <int HB>
__device__ __forceinline__ void h16_stage(float (&y)[4][8], int n) {
  const float s = (n & HB) ? -1.f : 1.f;
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int b = 0; b < 8; ++b) y[tt][b] = xor_row16<HB>(y[tt][b]) + s * y[tt][b];
}

// The rotated-domain values y of one 16-token value tile back to channels:
// lane 16q + n holds y[tt][b] of token 4q + tt, rotated channel 16b + n; H128
// (H8 over b, H16 over n across the row), times inv_d and the signs, times
// the token norms, into the staging tile at [token][channel].
// (kFirstHb 2: the H8 stage over bit 0 of b is already applied)
template <class Tile, int kFirstHb = 1>
__device__ __forceinline__ void dq_value_tile_rot(float (&y)[4][8], uint2 nrm, const uint32_t sign_bits[4],
                                                  float inv_d, int n, int q, Tile& tl, int dtype) {
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
#pragma unroll
    for (int hb = kFirstHb; hb < 8; hb <<= 1)   // H8 over b
#pragma unroll
      for (int b = 0; b < 8; ++b)
        if (!(b & hb)) {
          const float u = y[tt][b], w = y[tt][b | hb];
          y[tt][b] = u + w;
          y[tt][b | hb] = u - w;
        }
  }
  h16_stage<1>(y, n);   // H16 over n, across the row
  h16_stage<2>(y, n);
  h16_stage<4>(y, n);
  h16_stage<8>(y, n);
  const float nv[4] = {half_bits_to_float(nrm.x & 0xffff), half_bits_to_float(nrm.x >> 16),
                       half_bits_to_float(nrm.y & 0xffff), half_bits_to_float(nrm.y >> 16)};
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    const int c = 16 * b + n;
    const bool neg = sign_neg(sign_bits, c);
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const float v = y[tt][b] * inv_d;   // inv_d a power of two: exact
      tile_put(tl, 4 * q + tt, c, (neg ? -v : v) * nv[tt], dtype);
    }
  }
}

template <class Tile>
__device__ __forceinline__ void dq_value_tile(uint2 vcd, uint2 nrm, const float codebook[4],
                                              const uint32_t sign_bits[4], int n, int q, Tile& tl, int dtype) {
  const float l0 = codebook[0], l1 = codebook[1], l2 = codebook[2], l3 = codebook[3];
  float y[4][8];
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    const uint32_t D = b < 4 ? vcd.x : vcd.y;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) y[tt][b] = level4((D >> (8 * (b & 3) + 2 * tt)) & 3u, l0, l1, l2, l3);
  }
  dq_value_tile_rot(y, nrm, sign_bits, 1.0f / (float)kD, n, q, tl, dtype);
}

// Level pair table of a 2-bit codebook: entry a + 4 b (codes a, b) holds
// (l[a] + l[b], l[a] - l[b]), the first H8 stage of channel blocks 2k, 2k + 1
// (codes a, b of one token).  Built by the first 16 threads.
struct DqPairLut {
  float2 e[16];
};
__device__ __forceinline__ void dq_pair_lut_build(DqPairLut& t, const float codebook[4]) {
  const int i = threadIdx.x;
  if (i < 16) {
    const float la = codebook[i & 3], lb = codebook[i >> 2];
    t.e[i] = make_float2(la + lb, la - lb);
  }
}

// dq_value_tile with the codebook levels and the first H8 stage from the
// pair table (same values, same operations as the select chain and the
// in-register stage)
template <class Tile>
__device__ __forceinline__ void dq_value_tile_lut(uint2 vcd, uint2 nrm, const DqPairLut& lut,
                                                  const uint32_t sign_bits[4], int n, int q, Tile& tl, int dtype) {
  float y[4][8];
#pragma unroll
  for (int bp = 0; bp < 4; ++bp) {   // blocks 2 bp, 2 bp + 1: bytes (2 bp) & 3 and (2 bp + 1) & 3 of a word
    const uint32_t D = bp < 2 ? vcd.x : vcd.y;
    const uint32_t x = D >> (16 * (bp & 1));
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const uint32_t idx = ((x >> (2 * tt)) & 3u) | (((x >> (8 + 2 * tt)) & 3u) << 2);
      const float2 e = lut.e[idx];
      y[tt][2 * bp] = e.x;
      y[tt][2 * bp + 1] = e.y;
    }
  }
  dq_value_tile_rot<Tile, 2>(y, nrm, sign_bits, 1.0f / (float)kD, n, q, tl, dtype);
}

}  // namespace bmx

// Error channel shared by every C-ABI entry point (defined in k2b_api.hip).
void bmx_set_error(const std::string& msg);

// Per-device host state of the launchers (k2b_api.hip; thread-safe): the
// current device's CU count (cached per device; 256, MI355X's, if the query
// fails), and the dynamic-LDS limit of a kernel raised to at least bytes on
// the current device (hipFuncSetAttribute once per device, kernel and size).
int bmx_device_cu_count();
hipError_t bmx_ensure_dynamic_lds(const void* kernel, size_t bytes);
