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

// Physical page id clamped into the pool: a corrupt table entry cannot fault.
__device__ __forceinline__ int64_t clamp_page(int32_t pid, int32_t n_pool) {
  return (int64_t)min(max(pid, 0), n_pool - 1);
}

// V-codec sign of channel c (true -> -1).
__device__ __forceinline__ bool sign_neg(const uint32_t bits[4], int c) {
  return (bits[c >> 5] >> (c & 31)) & 1u;
}

// 3-bit two's-complement residual code k (0..31) of a 96-bit lane string.
__device__ __forceinline__ int kres_code(uint32_t w0, uint32_t w1, uint32_t w2, int k) {
  const int bit = 3 * k;
  uint32_t word;
  int sh;
  if (bit + 3 <= 32) {
    word = w0; sh = bit;
  } else if (bit < 32) {
    word = __builtin_amdgcn_alignbit(w1, w0, 30); sh = 0;   // bits 30..61
  } else if (bit + 3 <= 64) {
    word = w1; sh = bit - 32;
  } else if (bit < 64) {
    word = __builtin_amdgcn_alignbit(w2, w1, 31); sh = 0;   // bits 63..94
  } else {
    word = w2; sh = bit - 64;
  }
  return ((int)(word << (29 - sh))) >> 29;
}

}  // namespace bmx

// Error channel shared by every C-ABI entry point (defined in k2b_api.cpp).
void bmx_set_error(const std::string& msg);
