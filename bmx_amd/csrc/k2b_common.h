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
typedef float float4_t __attribute__((ext_vector_type(4)));

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

}  // namespace bmx

// Error channel shared by every C-ABI entry point (defined in k2b_api.cpp).
void bmx_set_error(const std::string& msg);
