// Packed-KV RTN path on gfx950: rtn_token keys (post-RoPE) and values, 2..4-bit
// codes times a per-(token, channel group) fp16 scale, in 16-token pages.
//
// rtn_append_kernel   quantize-on-append: codes and scales of committed pages
// rtn_decode_split_kernel<SW>
//                     split-KV decode: one workgroup of 8 waves per (split,
//                     sequence), wave w = KV head w, walking 64-token groups
//                     (4 pages) of the split's balanced share:
//   * each lane streams its 16-byte key-code and value-code slices of every
//     page straight into VGPRs, a whole group ahead; the scale sections of the
//     group's pages are staged cooperatively two groups ahead in a three-slot
//     LDS ring that the waves hand on with LDS counters (no barrier per
//     group), so a wave may run a group ahead of the slowest;
//   * keys: the lane's 8 channels of a word become 4 fp16 pairs of exact
//     integer codes with one and-or each (code + 8 in the mantissa of 1024)
//     and a packed subtract; the G query heads are scored on MFMA against the
//     query split into fp16 high and low parts, one product per 32-channel
//     block (inside one scale group), scaled by the (token, group) scale in
//     fp32;
//   * the 4 pages' score tiles are compacted (DPP) and the online softmax runs
//     once per group, as in the k2b kernel;
//   * values: P.V on MFMA, two pages per product (K index 8q + 2t + e is token
//     4q + t of page e of the pair); the A operand is the exact integer codes,
//     the value scales multiply P in the B operand (one B per channel group);
//   * the window's 16-token score tiles and the merge are the shared ones
//     (decode_shared.h); the partials are plain channel sums.
// rtn_dequant_kernel  pages -> dense keys and values in fp32, fp16 or bf16 (prefill)
//
// Reference semantics: cache/triton_dequant_attention.py:580-728 (kernel),
// 731-832 (launcher), 1390-1451 (stacks: fp16 scales), 504-575 / 409-461 /
// 324-360 (finalize, merge, tail); cache/codecs.py:720-722 and
// quant/rtn.py:23-53 (codec).

#include "k2b_common.h"
#include "decode_shared.h"
#include "bmx_rtn.h"

#include <algorithm>
#include <cmath>

namespace bmx {

constexpr int kRWaves = 8;
constexpr int kRThreads = 64 * kRWaves;
constexpr int kRGroupPages = 4;                  // 64-token groups, as for k2b
constexpr int kRGroup = kRGroupPages * kPT;
constexpr int kRPidWindow = 64;
constexpr int kRMaxPrefix = 8 * (2 * kD + kPT * 4) * 2;  // scale bytes of a page at most: h_kv 8,
                                                     // channel-arm keys, value groups of 32

// Byte offsets of the four page sections (see include/bmx_rtn.h).
struct RtnLayout {
  int32_t kscale, vscale, kcode, vcode, bytes;
  int32_t ngk, ngv;   // scale groups per head and token (ngk: token-arm keys)
  __host__ __device__ static RtnLayout make(int h_kv, int karm, int gk, int gv) {
    RtnLayout L;
    L.ngk = kD / gk;
    L.ngv = kD / gv;
    L.kscale = 0;
    // channel-arm keys: the fp32 scale as an fp16 pair, hi for every head, then lo
    L.vscale = L.kscale + h_kv * (karm == BMX_RTN_CHANNEL ? 2 * kD : kPT * L.ngk) * 2;
    L.kcode = L.vscale + h_kv * kPT * L.ngv * 2;
    L.vcode = L.kcode + h_kv * 1024;
    L.bytes = L.vcode + h_kv * 1024;
    return L;
  }
};

__device__ __forceinline__ float load_elem(const void* base, int64_t idx, int dtype) {
  if (dtype == BMX_K2B_F32) return reinterpret_cast<const float*>(base)[idx];
  const uint16_t u = reinterpret_cast<const uint16_t*>(base)[idx];
  if (dtype == BMX_K2B_BF16) return __uint_as_float((uint32_t)u << 16);
  return half_bits_to_float(u);
}

// ---------------------------------------------------------------------------
// Quantize-on-append.  grid (8 * n_codec_pages, h_kv), block 256: thread
// (token tt = tid / 16, slice l = tid % 16) owns channels 8l .. 8l + 7 of one
// token; a channel group of g spans g / 8 threads, reduced by shuffles.  The
// element-wise steps follow rtn.py:23-44 in fp32 (max, divide, round half to
// even, clamp); this file is built without floating-point contraction.
// ---------------------------------------------------------------------------
struct RtnAppendKArgs {
  int h_kv, kbits, vbits, gk, gv, n_pool, karm;
  const void* k;
  int64_t ksh, kst;
  int kdt;
  const void* v;
  int64_t vsh, vst;
  int vdt;
  uint8_t* pages;
  const int32_t* page_ids;
  RtnLayout L;
};

// scale and codes of one thread's 8 values in a group of g channels
__device__ __forceinline__ float rtn_codes(const float x[8], int g, int bits, int code[8]) {
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(x[j]));
  for (int o = 1; o < g / 8; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  const int qmax = (1 << (bits - 1)) - 1;
  const float scale = fmaxf(amax, 1e-12f) / (float)qmax;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float r = __builtin_rintf(x[j] / scale);
    code[j] = (int)fminf(fmaxf(r, (float)(-qmax - 1)), (float)qmax);
  }
  return scale;
}

__global__ __launch_bounds__(256) void rtn_append_kernel(const RtnAppendKArgs a) {
  const int pg = blockIdx.x, h = blockIdx.y;
  const int tid = threadIdx.x, tt = tid >> 4, l = tid & 15;
  const int64_t T = (int64_t)pg * kPT + tt;   // token within the call
  uint8_t* page = a.pages + clamp_page(a.page_ids[pg], a.n_pool) * a.L.bytes;
  __shared__ int8_t s_v[kPT][kD];
  float x[8];
  int code[8];
  float s;
  if (a.karm == BMX_RTN_TOKEN) {   // channel-arm keys: rtn_append_kchan_kernel
    // keys: word w = l / 4 of quarter q = l % 4 holds channels 32w + 8q .. +7 = 8l .. 8l + 7
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = load_elem(a.k, h * a.ksh + T * a.kst + 8 * l + j, a.kdt);
    s = rtn_codes(x, a.gk, a.kbits, code);
    uint32_t w = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) w |= (uint32_t)(code[j] + 8) << (4 * j);
    reinterpret_cast<uint32_t*>(page + a.L.kcode + h * 1024)[((l & 3) * kPT + tt) * 4 + (l >> 2)] = w;
    if ((l & (a.gk / 8 - 1)) == 0)
      reinterpret_cast<uint16_t*>(page + a.L.kscale)[(h * kPT + tt) * a.L.ngk + (8 * l) / a.gk] =
          float_to_half_bits(s);
  }
  // values: codes to LDS, then one 16-bit cell (4 tokens of a channel) per write
#pragma unroll
  for (int j = 0; j < 8; ++j) x[j] = load_elem(a.v, h * a.vsh + T * a.vst + 8 * l + j, a.vdt);
  s = rtn_codes(x, a.gv, a.vbits, code);
#pragma unroll
  for (int j = 0; j < 8; ++j) s_v[tt][8 * l + j] = (int8_t)code[j];
  if ((l & (a.gv / 8 - 1)) == 0)
    reinterpret_cast<uint16_t*>(page + a.L.vscale)[((h * 4 + (tt >> 2)) * a.L.ngv + (8 * l) / a.gv) * 4 +
                                                   (tt & 3)] = float_to_half_bits(s);
  __syncthreads();
  uint16_t* vcode = reinterpret_cast<uint16_t*>(page + a.L.vcode + h * 1024);
  for (int e = tid; e < 4 * 16 * 8; e += 256) {   // cell (q, c, b): channel 16b + c, tokens 4q ..
    const int q = e >> 7, c = (e >> 3) & 15, bt = e & 7;
    uint32_t cell = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) cell |= (uint32_t)(s_v[4 * q + j][16 * bt + c] + 8) << (4 * j);
    vcode[e] = (uint16_t)cell;
  }
}

// position of channel c in a channel-arm KSCALE row: [4 b][4 q][8 j'], channel
// 32b + 8q + p(j'), p = 0 4 1 5 2 6 3 7 (the pair order of nibble_pairs)
__host__ __device__ __forceinline__ int kchan_slot(int c) {
  const int j = c & 7;
  return (c & ~7) + 2 * (j & 3) + (j >> 2);
}

// Channel-arm keys (quantize_packed("rtn_channel"), codecs.py:723-725: the
// token axis grouped per channel).  grid (n_codec_pages * 128 / gk, h_kv),
// block 128: thread c owns channel c of one gk-token group, spanning gk / 16
// pages; codes go through LDS to be packed into the pages' code words, and
// the group's fp16 scales are written into each of its pages.
__global__ __launch_bounds__(128) void rtn_append_kchan_kernel(const RtnAppendKArgs a) {
  const int grp = blockIdx.x, h = blockIdx.y, c = threadIdx.x;
  const int64_t T0 = (int64_t)grp * a.gk;   // first token of the group within the call
  __shared__ int8_t s_k[kCodec][kD];
  float amax = 0.f;
  for (int t = 0; t < a.gk; ++t) amax = fmaxf(amax, fabsf(load_elem(a.k, h * a.ksh + (T0 + t) * a.kst + c, a.kdt)));
  const int qmax = (1 << (a.kbits - 1)) - 1;
  const float scale = fmaxf(amax, 1e-12f) / (float)qmax;
  for (int t = 0; t < a.gk; ++t) {
    const float r = __builtin_rintf(load_elem(a.k, h * a.ksh + (T0 + t) * a.kst + c, a.kdt) / scale);
    s_k[t][c] = (int8_t)fminf(fmaxf(r, (float)(-qmax - 1)), (float)qmax);
  }
  const int n_pg = a.gk / kPT;
  const int pg0 = (int)(T0 / kPT);
  // the fp32 scale as hi = fp16(scale) and lo = fp16(scale - hi): hi + lo is
  // the scale to 2^-22 relative (the reference dequantizes with the fp32 scale)
  const uint16_t s_hi = float_to_half_bits(scale);
  const uint16_t s_lo = float_to_half_bits(scale - half_bits_to_float(s_hi));
  for (int p = 0; p < n_pg; ++p) {
    uint8_t* page = a.pages + clamp_page(a.page_ids[pg0 + p], a.n_pool) * a.L.bytes;
    uint16_t* ks = reinterpret_cast<uint16_t*>(page + a.L.kscale);
    ks[h * kD + kchan_slot(c)] = s_hi;
    ks[(a.h_kv + h) * kD + kchan_slot(c)] = s_lo;
  }
  __syncthreads();
  for (int e = c; e < n_pg * 256; e += 128) {   // word (q, n, w): token n, channels 32w + 8q ..
    const int p = e >> 8, qq = (e >> 6) & 3, n = (e >> 2) & 15, w = e & 3;
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) word |= (uint32_t)(s_k[p * kPT + n][32 * w + 8 * qq + j] + 8) << (4 * j);
    uint8_t* page = a.pages + clamp_page(a.page_ids[pg0 + p], a.n_pool) * a.L.bytes;
    reinterpret_cast<uint32_t*>(page + a.L.kcode + h * 1024)[e & 255] = word;
  }
}

// ---------------------------------------------------------------------------
// Dequantize: grid (n_pages, h_kv), block 256, thread (token tt, slice l).
// ---------------------------------------------------------------------------
struct RtnDequantKArgs {
  int h_kv, n_pool, karm;
  const uint8_t* pages;
  const int32_t* page_ids;
  int64_t n_tok;       // rows between consecutive heads in k_out / v_out
  void* k_out;
  void* v_out;
  int out_dtype;
  int gk, gv;
  RtnLayout L;
};

__global__ __launch_bounds__(256) void rtn_dequant_kernel(const RtnDequantKArgs a) {
  const int p = blockIdx.x, h = blockIdx.y;
  const int tid = threadIdx.x, tt = tid >> 4, l = tid & 15;
  const uint8_t* page = a.pages + clamp_page(a.page_ids[p], a.n_pool) * a.L.bytes;
  const int64_t row = ((int64_t)h * a.n_tok + (int64_t)p * kPT + tt) * kD;
  const uint32_t w = reinterpret_cast<const uint32_t*>(page + a.L.kcode + h * 1024)[((l & 3) * kPT + tt) * 4 + (l >> 2)];
  const uint16_t* ksc = reinterpret_cast<const uint16_t*>(page + a.L.kscale);
  const float sk = a.karm == BMX_RTN_TOKEN ? half_bits_to_float(ksc[(h * kPT + tt) * a.L.ngk + (8 * l) / a.gk]) : 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float s = a.karm == BMX_RTN_TOKEN
                        ? sk
                        : half_bits_to_float(ksc[h * kD + kchan_slot(8 * l + j)]) +
                              half_bits_to_float(ksc[(a.h_kv + h) * kD + kchan_slot(8 * l + j)]);
    store_elem(a.k_out, row + 8 * l + j, (float)((int)((w >> (4 * j)) & 15u) - 8) * s, a.out_dtype);
  }
  const uint16_t* vcode = reinterpret_cast<const uint16_t*>(page + a.L.vcode + h * 1024);
  const float sv = half_bits_to_float(reinterpret_cast<const uint16_t*>(page + a.L.vscale)
                                          [((h * 4 + (tt >> 2)) * a.L.ngv + (8 * l) / a.gv) * 4 + (tt & 3)]);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int c = 8 * l + j;
    const uint32_t cell = vcode[((tt >> 2) * 16 + (c & 15)) * 8 + (c >> 4)];
    store_elem(a.v_out, row + c, (float)((int)((cell >> (4 * (tt & 3))) & 15u) - 8) * sv, a.out_dtype);
  }
}

// ---------------------------------------------------------------------------
// Decode.
// ---------------------------------------------------------------------------
struct RtnDecodeKArgs {
  int h_kv, G, max_splits, max_pages, max_packed_len, n_pool;
  int gk, gv;
  int prefix_bytes;    // scale bytes of one page (KSCALE + VSCALE), multiple of 16
  const void* q;       // [B][h_kv][G][128] in io_dtype
  int io_dtype;
  uint16_t* ws_acc;    // [B][h_kv][G][8][max_splits][16] partial records of the channel sums (decode_shared.h)
  float* ws_ml;        // [B][h_kv][G][max_splits][2] (running max, sum), base 2
  const uint8_t* pages;
  const int32_t* page_table;
  const int32_t* packed_len;
  RtnLayout L;
  float qscale;        // sm_scale * log2(e)
  // recent window (decode_shared.h), fp16 or bf16 (tail_bf16)
  const uint16_t* k_tail;
  int64_t ts_b, ts_h, ts_t;
  int tail_bf16;
  WinNew nw;           // the window's newest rows given apart (decode_shared.h)
  int tail_cap;
  float win_rescale;   // 1: the window keys are scored with qscale
  float* ws_win;
};

__device__ __forceinline__ half2_t as_h2r(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t as_u32r(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

template <int CTRL, int BANK = 0xF>
__device__ __forceinline__ float dpp_r(float old, float src) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old),
                                                               __builtin_bit_cast(int, src), CTRL, 0xF,
                                                               BANK, false));
}
template <int CTRL>
__device__ __forceinline__ float dpp_all_r(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}
constexpr int kRRowShr = 0x110;
constexpr int kRRowRor = 0x120;

constexpr int kRBufWord3 = 0x00020000;   // buffer descriptor word 3: raw 32-bit data

// 8 nibbles (offset binary) -> fp16 pairs (n_p, n_{p+4}) - 8, exact.  A
// nibble at mantissa bits [0, 4) under exponent field 25 reads as 1024 + n,
// at bits [4, 8) under exponent field 21 as 64 + n: nibbles 0, 1 (and 4, 5)
// in place, 2, 3 (6, 7) after one shift by 8, each pair one AND-OR (masks in
// registers: a VOP3 takes no two literals) and one packed add.
struct NibMasks {
  uint32_t m0, m1;   // nibble bits of slots 0 and 1 (both halves)
  uint32_t e0, e1;   // exponent fields 25 and 21 (both halves)
  __device__ __forceinline__ void init() {
    m0 = 0x000F000Fu; m1 = 0x00F000F0u;
    e0 = 0x64006400u; e1 = 0x54005400u;
    asm volatile("" : "+v"(m0), "+v"(m1));
    asm volatile("" : "+s"(e0), "+s"(e1));
  }
};
__device__ __forceinline__ void nibble_pairs(const NibMasks& nm, uint32_t x, uint32_t out[4]) {
  const half2_t b0 = {(_Float16)-1032.0f, (_Float16)-1032.0f};   // 1024 + 8
  const half2_t b1 = {(_Float16)-72.0f, (_Float16)-72.0f};       // 64 + 8
  const uint32_t y = x >> 8;
  out[0] = as_u32r(as_h2r((x & nm.m0) | nm.e0) + b0);
  out[1] = as_u32r(as_h2r((x & nm.m1) | nm.e1) + b1);
  out[2] = as_u32r(as_h2r((y & nm.m0) | nm.e0) + b0);
  out[3] = as_u32r(as_h2r((y & nm.m1) | nm.e1) + b1);
}

// The partial of one (sequence, head, split): plain channel sums.
__device__ __forceinline__ void rtn_store_partial(const RtnDecodeKArgs& a, int b, int split, int h, int n,
                                                  int q, const float4_t acc[8], float m_run, float l_run) {
  l_run += __shfl_xor(l_run, 16);
  l_run += __shfl_xor(l_run, 32);
  if (n < a.G)
    store_partial_record(a.ws_acc, a.ws_ml, ((int64_t)b * a.h_kv + h) * a.G + n, a.max_splits, split, q, acc,
                         m_run, l_run);
}

// the lane's query in the RoPE pair order of the window tiles (decode_shared.h)
__device__ __forceinline__ void rtn_window_fragments(const RtnDecodeKArgs& a, int b, int h, int n, int q,
                                                     half8_t qh[4], half8_t ql[4]) {
  const int64_t qrow = (((int64_t)b * a.h_kv + h) * a.G + (n < a.G ? n : 0)) * kD;
  float4_t qraw[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) qraw[u] = load_q4(a.q, qrow + 16 * (u & 3) + 4 * q + 64 * (u >> 2), a.io_dtype);
  window_fragments(qraw, n < a.G ? a.qscale : 0.0f, a.tail_bf16, qh, ql);
}

// A workgroup with no packed tokens: its window tiles and an empty partial.
__device__ __noinline__ void rtn_empty_range(const RtnDecodeKArgs& a, int b, int split, int h, int n, int q) {
  const int n_tiles = (a.tail_cap + 15) >> 4;
  if (split < n_tiles) {
    half8_t qh[4], ql[4];
    rtn_window_fragments(a, b, h, n, q, qh, ql);
    const int64_t tail_base = (int64_t)b * a.ts_b + (int64_t)h * a.ts_h;
    for (int j = split; j < n_tiles; j += a.max_splits) {
      uint2 kw[8];
      load_win_tile(a, tail_base, j, n, q, kw, (int64_t)b * a.nw.sb + (int64_t)h * a.nw.sh);
      score_win_tile(a, b, h, j, n, q, kw, qh, ql, tail_base);
    }
  }
  float4_t zero[8];
#pragma unroll
  for (int bt = 0; bt < 8; ++bt) zero[bt] = float4_t{0.f, 0.f, 0.f, 0.f};
  rtn_store_partial(a, b, split, h, n, q, zero, -INFINITY, 0.f);
}

// SW: query slot width (G rounded up to 4, 8 or 16); the 16 score columns of a
// page hold 16 / SW pages after compaction.  NGK: key scale groups per token
// (128 / k_group) of token-arm keys, 0 for channel-arm keys.
// kNT: page loads non-temporal (calls whose pages stream from HBM)
template <int SW, int NGK, bool kNT>
__global__ __launch_bounds__(kRThreads) void rtn_decode_split_kernel(const RtnDecodeKArgs a) {
  constexpr int NSLOT = 16 / SW;
  constexpr int NCR = kRGroupPages / NSLOT;
  constexpr int kSlots = 3;   // group g's scales in ring slot g % 3
  __shared__ __attribute__((aligned(16))) uint8_t ring[kSlots][kRGroupPages][kRMaxPrefix];
  // s_sync[s]: waves that have stored a group's scales into slot s;
  // s_sync[kSlots + s]: waves done reading a group from slot s (monotonic)
  __shared__ uint32_t s_sync[2 * kSlots];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int n = lane & 15, q = lane >> 4;
  const int split = blockIdx.x, b = blockIdx.y;
  const bool active = wave < a.h_kv;
  const int h = active ? wave : 0;
  const int S = a.max_splits;
  const int len_spec = a.max_packed_len & ~(kRGroup - 1);
  auto range = [&](int L, int& r0, int& r1) {
    const int NG = L / kRGroup;
    r0 = (int)(((int64_t)split * NG) / S);
    r1 = (int)(((int64_t)(split + 1) * NG) / S);
  };
  int g0, g1;
  range(len_spec, g0, g1);
  const int32_t* ptab_row = a.page_table + (int64_t)b * a.max_pages;
  auto load_ids_raw = [&](int first, int count) {
    const int32_t* src = count > 0 ? ptab_row + g0 * kRGroupPages + min(first + lane, count - 1)
                                   : a.packed_len + b;
    return (int)*src;
  };
  const int pid_raw = load_ids_raw(0, (g1 - g0) * kRGroupPages);
  const int len_raw = a.packed_len[b];
  // the lane's query: channels 32bb + 8q + j (bb < 4, j < 8) of query n
  float4_t qraw[8];
  {
    const int64_t qrow = (((int64_t)b * a.h_kv + h) * a.G + (n < a.G ? n : 0)) * kD;
#pragma unroll
    for (int u = 0; u < 8; ++u) qraw[u] = load_q4(a.q, qrow + 32 * (u >> 1) + 8 * q + 4 * (u & 1), a.io_dtype);
  }
  const int n_win_tiles = (a.tail_cap + 15) >> 4;
  const int64_t tail_base = (int64_t)b * a.ts_b + (int64_t)h * a.ts_h;

  int pidv = (int)clamp_page(pid_raw, a.n_pool);
  // uniform values in scalar registers: the group loop's bookkeeping is scalar work
  const int len = __builtin_amdgcn_readfirstlane(min(len_raw, a.max_packed_len) & ~(kRGroup - 1));
  if (len != len_spec) {
    range(len, g0, g1);
    pidv = (int)clamp_page(load_ids_raw(0, (g1 - g0) * kRGroupPages), a.n_pool);
  }
  g0 = __builtin_amdgcn_readfirstlane(g0);
  g1 = __builtin_amdgcn_readfirstlane(g1);
  const int n_groups = g1 - g0;
  if (n_groups == 0) {
    if (active)
      rtn_empty_range(*(const RtnDecodeKArgs*)__builtin_amdgcn_kernarg_segment_ptr(), b, split, h, n, q);
    return;
  }
  auto load_ids = [&](int first, int count) { return (int)clamp_page(load_ids_raw(first, count), a.n_pool); };
  const int pb = a.L.bytes;
  const int PB = a.prefix_bytes;
  const int chunks_pp = PB / 16;
  const int pre_chunks = kRGroupPages * chunks_pp;
  const int n_pages = n_groups * kRGroupPages;
  int pid_base = 0;
  auto page_ptr = [&](int gi, int pp) -> const uint8_t* {
    const int id = __builtin_amdgcn_readlane(pidv, gi * kRGroupPages + pp - pid_base);
    return a.pages + (int64_t)id * pb;
  };
  // the 4 pages' scale sections, 16-byte chunk c (tid, tid + 512 and tid +
  // 1024: the channel-arm key scales, hi and lo, make them up to 1280 chunks)
  struct Pre { uint4 c0, c1, c2; };
  auto load_chunk = [&](int gi, int c) -> uint4 {
    c = min(c, pre_chunks - 1);
    const int pp = c / chunks_pp;
    const int id = __shfl(pidv, gi * kRGroupPages + pp - pid_base);
    const uint8_t* src = a.pages + (int64_t)id * pb + (c - pp * chunks_pp) * 16;
    if constexpr (kNT) {
      typedef uint32_t p_u32x4_t __attribute__((ext_vector_type(4)));
      const p_u32x4_t w = __builtin_nontemporal_load(reinterpret_cast<const p_u32x4_t*>(src));
      return make_uint4(w[0], w[1], w[2], w[3]);
    } else {
      return *reinterpret_cast<const uint4*>(src);
    }
  };
  auto load_prefix = [&](int gi) -> Pre {
    Pre r;
    r.c0 = load_chunk(gi, tid);
    r.c1 = pre_chunks > kRThreads ? load_chunk(gi, tid + kRThreads) : r.c0;
    r.c2 = pre_chunks > 2 * kRThreads ? load_chunk(gi, tid + 2 * kRThreads) : r.c0;
    return r;
  };
  auto store_prefix = [&](const Pre& v, int slot) {
    if (tid < pre_chunks) {
      const int pp = tid / chunks_pp;
      *reinterpret_cast<uint4*>(&ring[slot][pp][(tid - pp * chunks_pp) * 16]) = v.c0;
    }
    const int c1 = tid + kRThreads;
    if (c1 < pre_chunks) {
      const int pp = c1 / chunks_pp;
      *reinterpret_cast<uint4*>(&ring[slot][pp][(c1 - pp * chunks_pp) * 16]) = v.c1;
    }
    const int c2 = tid + 2 * kRThreads;
    if (c2 < pre_chunks) {
      const int pp = c2 / chunks_pp;
      *reinterpret_cast<uint4*>(&ring[slot][pp][(c2 - pp * chunks_pp) * 16]) = v.c2;
    }
  };
  const uint32_t kc_off = (uint32_t)(a.L.kcode + h * 1024 + lane * 16);
  const uint32_t vc_off = (uint32_t)(a.L.vcode + h * 1024 + lane * 16);
  // a page's code sections through a buffer descriptor on its (uniform) base:
  // the address is scalar work, the lane offset a constant register, and the
  // load is non-temporal (aux 2: the codes are read once)
  typedef uint32_t r_u32x4_t __attribute__((ext_vector_type(4)));
  auto load_code = [&](int gi, int pp, uint32_t off) -> uint4 {
    const r_u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(page_ptr(gi, pp)), (short)0, pb, kRBufWord3), (int)off,
        0, kNT ? 2 : 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
  };
  auto load_kc = [&](int gi, int pp) { return load_code(gi, pp, kc_off); };
  auto load_vc = [&](int gi, int pp) { return load_code(gi, pp, vc_off); };

  Pre pre = load_prefix(0);
  const Pre pre1 = load_prefix(min(1, n_groups - 1));
  uint4 kc[kRGroupPages], vc[kRGroupPages];
#pragma unroll
  for (int pp = 0; pp < kRGroupPages; ++pp) {
    kc[pp] = load_kc(0, pp);
    vc[pp] = load_vc(0, pp);
  }
  // query fragments: B[8q + j'][n] = x_n[32bb + 8q + perm(j')], perm = 0 4 1 5 2 6 3 7
  // (the order in which a code word leaves nibble_pairs), x = q * qscale, hi + lo
  half8_t qh[4], ql[4];
  {
    const float sc = n < a.G ? a.qscale : 0.0f;
#pragma unroll
    for (int bb = 0; bb < 4; ++bb)
#pragma unroll
      for (int jp = 0; jp < 8; ++jp) {
        const int j = (jp >> 1) + 4 * (jp & 1);
        const float x = qraw[2 * bb + (j >> 2)][j & 3] * sc;
        const _Float16 xh = (_Float16)x;
        qh[bb][jp] = xh;
        ql[bb][jp] = (_Float16)(x - (float)xh);
      }
  }
  // the window tiles of this workgroup (their rows after the first group's pages)
  if (active && split < n_win_tiles) {
    half8_t wh[4], wl[4];
    rtn_window_fragments(a, b, h, n, q, wh, wl);
    for (int j = split; j < n_win_tiles; j += S) {
      uint2 kw[8];
      load_win_tile(a, tail_base, j, n, q, kw, (int64_t)b * a.nw.sb + (int64_t)h * a.nw.sh);
      score_win_tile(a, b, h, j, n, q, kw, wh, wl, tail_base);
    }
  }
  store_prefix(pre, 0);
  store_prefix(pre1, 1);
  if (tid < 2 * kSlots) s_sync[tid] = tid < 2 ? kRWaves : 0;   // slots 0, 1: groups 0, 1 (barrier below)

  float4_t acc[8];
#pragma unroll
  for (int bt = 0; bt < 8; ++bt) acc[bt] = float4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;
  const int my_slot = NSLOT > 1 ? n / SW : 0;
  NibMasks nm;
  nm.init();
  __syncthreads();
  __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): group 0 has landed

  for (int gi = 0; gi < n_groups; ++gi) {
    const int gn = min(gi + 1, n_groups - 1);   // group whose codes are fetched during this one
    const int gp = min(gi + 2, n_groups - 1);   // group whose scales are fetched during this one
    if ((gp + 1) * kRGroupPages - pid_base > kRPidWindow) {
      pid_base = gn * kRGroupPages;
      pidv = load_ids(pid_base, n_pages);
    }
    // the last groups fetch nothing they would not use
    Pre pre_n{};
    if (gi + 2 < n_groups) pre_n = load_prefix(gp);
    uint4 kc_n[kRGroupPages], vc_n[kRGroupPages];
    if (active && gi + 1 < n_groups) {
#pragma unroll
      for (int pp = 0; pp < kRGroupPages; ++pp) {
        kc_n[pp] = load_kc(gn, pp);
        vc_n[pp] = load_vc(gn, pp);
      }
    }
    // every wave has stored this group's scales (use gi / 3 of slot gi % 3)
    const int slot = gi % kSlots;
    wait_count(&s_sync[slot], kRWaves * (gi / kSlots + 1));
    if (active) {
      // ---- keys: scores of the 4 pages.  MFMA bb spans channels 32bb .. +31,
      // inside one scale group: the exact integer codes meet the query, and the
      // fp16 scale of (token, group) multiplies the product in fp32 ----
      float4_t sc[kRGroupPages];
#pragma unroll
      for (int pp = 0; pp < kRGroupPages; ++pp) {
        if constexpr (NGK == 0) {
          // channel-arm keys: the scale varies along the MFMA's K axis, so it
          // goes into the A operand, as an fp16 sum hi + lo of code * scale:
          // hi = fp16(code * s_hi), lo = its rounding residual (one packed
          // FMA) plus code * s_lo, the fp32 scale being s_hi + s_lo
          const uint4* ksp = reinterpret_cast<const uint4*>(&ring[slot][pp][a.L.kscale]) + h * 16 + q;
          const uint4* ksl = ksp + a.h_kv * 16;
          const uint32_t kw4[4] = {kc[pp].x, kc[pp].y, kc[pp].z, kc[pp].w};
          float4_t s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int bb = 0; bb < 4; ++bb) {
            const uint4 sp = ksp[4 * bb], sl = ksl[4 * bb];
            const uint32_t s4[4] = {sp.x, sp.y, sp.z, sp.w};
            const uint32_t l4[4] = {sl.x, sl.y, sl.z, sl.w};
            uint32_t cp[4];
            nibble_pairs(nm, kw4[bb], cp);
            union { uint32_t u[4]; half8_t v; } khi, klo;
#pragma unroll
            for (int p = 0; p < 4; ++p) {
              const half2_t hi = as_h2r(cp[p]) * as_h2r(s4[p]);
              khi.u[p] = as_u32r(hi);
              const half2_t res = __builtin_elementwise_fma(as_h2r(cp[p]), as_h2r(s4[p]), -hi);
              klo.u[p] = as_u32r(__builtin_elementwise_fma(as_h2r(cp[p]), as_h2r(l4[p]), res));
            }
            s = __builtin_amdgcn_mfma_f32_16x16x32_f16(khi.v, qh[bb], s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_16x16x32_f16(khi.v, ql[bb], s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_16x16x32_f16(klo.v, qh[bb], s, 0, 0, 0);
          }
          sc[pp] = s;
          continue;
        } else {
        // scales of the lane's score rows, tokens 4q .. 4q + 3: [4][NGK] fp16
        const uint16_t* ksp = reinterpret_cast<const uint16_t*>(&ring[slot][pp][a.L.kscale]) +
                              (h * kPT + 4 * q) * NGK;
        float ksc[4][NGK];
        if constexpr (NGK == 4) {
          const uint4 s0 = *reinterpret_cast<const uint4*>(ksp), s1 = *reinterpret_cast<const uint4*>(ksp + 8);
          const uint32_t w[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
          for (int e = 0; e < 16; ++e) ksc[e >> 2][e & 3] = half_bits_to_float((w[e >> 1] >> (16 * (e & 1))) & 0xffffu);
        } else if constexpr (NGK == 2) {
          const uint4 s0 = *reinterpret_cast<const uint4*>(ksp);
          const uint32_t w[4] = {s0.x, s0.y, s0.z, s0.w};
#pragma unroll
          for (int e = 0; e < 8; ++e) ksc[e >> 1][e & 1] = half_bits_to_float((w[e >> 1] >> (16 * (e & 1))) & 0xffffu);
        } else {
          const uint2 s0 = *reinterpret_cast<const uint2*>(ksp);
          const uint32_t w[2] = {s0.x, s0.y};
#pragma unroll
          for (int e = 0; e < 4; ++e) ksc[e][0] = half_bits_to_float((w[e >> 1] >> (16 * (e & 1))) & 0xffffu);
        }
        const uint32_t kw4[4] = {kc[pp].x, kc[pp].y, kc[pp].z, kc[pp].w};
        float4_t s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int bb = 0; bb < 4; ++bb) {
          union { uint32_t u[4]; half8_t v; } ka;
          nibble_pairs(nm, kw4[bb], ka.u);
          const float4_t z = {0.f, 0.f, 0.f, 0.f};
          float4_t d = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka.v, qh[bb], z, 0, 0, 0);
          d = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka.v, ql[bb], d, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 4; ++i) s[i] = __builtin_fmaf(ksc[i][(bb * NGK) / 4], d[i], s[i]);
        }
        sc[pp] = s;
        }
      }
      // ---- compaction: page r*NSLOT + s moves to columns [s*SW, (s+1)*SW) ----
      float4_t cr[NCR];
#pragma unroll
      for (int r = 0; r < NCR; ++r) {
        cr[r] = sc[r * NSLOT];
        if constexpr (NSLOT == 4) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            cr[r][i] = dpp_r<kRRowShr + 4, 0x2>(cr[r][i], sc[r * NSLOT + 1][i]);
            cr[r][i] = dpp_r<kRRowShr + 8, 0x4>(cr[r][i], sc[r * NSLOT + 2][i]);
            cr[r][i] = dpp_r<kRRowShr + 12, 0x8>(cr[r][i], sc[r * NSLOT + 3][i]);
          }
        } else if constexpr (NSLOT == 2) {
#pragma unroll
          for (int i = 0; i < 4; ++i) cr[r][i] = dpp_r<kRRowShr + 8, 0xC>(cr[r][i], sc[r * NSLOT + 1][i]);
        }
      }
      // ---- online softmax over the group ----
      float mx = -INFINITY;
#pragma unroll
      for (int r = 0; r < NCR; ++r)
        mx = fmaxf(mx, fmaxf(fmaxf(cr[r][0], cr[r][1]), fmaxf(cr[r][2], cr[r][3])));
      if (__any(mx > m_run)) {
        if constexpr (NSLOT == 4) mx = fmaxf(mx, dpp_all_r<kRRowRor + 4>(mx));
        if constexpr (NSLOT >= 2) mx = fmaxf(mx, dpp_all_r<kRRowRor + 8>(mx));
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        l_run *= alpha;
#pragma unroll
        for (int bt = 0; bt < 8; ++bt) acc[bt] *= alpha;
        m_run = m_new;
      }
      // P of the lane's page (its slot), tokens 4q .. 4q + 3, fp16 pairs
      uint2 pd[NCR];
#pragma unroll
      for (int r = 0; r < NCR; ++r) {
        float p[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p[i] = __builtin_amdgcn_exp2f(cr[r][i] - m_run);
          l_run += p[i];
        }
        const half2_t h01 = {(_Float16)p[0], (_Float16)p[1]}, h23 = {(_Float16)p[2], (_Float16)p[3]};
        pd[r] = make_uint2(as_u32r(h01), as_u32r(h23));
      }
      // ---- P.V on MFMA, pages (2u, 2u + 1): K index 8q + 2t + e is token 4q + t
      // of page 2u + e; A = the exact codes, B = P times the value scale of the
      // tile's channel group ----
#pragma unroll
      for (int u = 0; u < kRGroupPages / 2; ++u) {
        const int pa = 2 * u, pbb = 2 * u + 1;
        const uint2 za = (NSLOT == 1 || my_slot == pa % NSLOT) ? pd[pa / NSLOT] : make_uint2(0u, 0u);
        const uint2 zb = (NSLOT == 1 || my_slot == pbb % NSLOT) ? pd[pbb / NSLOT] : make_uint2(0u, 0u);
        // (P_a(t), P_b(t)) pairs, t = 0..3
        const uint32_t pab[4] = {__builtin_amdgcn_perm(zb.x, za.x, 0x05040100u),
                                 __builtin_amdgcn_perm(zb.x, za.x, 0x07060302u),
                                 __builtin_amdgcn_perm(zb.y, za.y, 0x05040100u),
                                 __builtin_amdgcn_perm(zb.y, za.y, 0x07060302u)};
        const uint32_t va4[4] = {vc[pa].x, vc[pa].y, vc[pa].z, vc[pa].w};
        const uint32_t vb4[4] = {vc[pbb].x, vc[pbb].y, vc[pbb].z, vc[pbb].w};
        const uint16_t* vsa = reinterpret_cast<const uint16_t*>(&ring[slot][pa][a.L.vscale]) +
                              (h * 4 + q) * a.L.ngv * 4;
        const uint16_t* vsb = reinterpret_cast<const uint16_t*>(&ring[slot][pbb][a.L.vscale]) +
                              (h * 4 + q) * a.L.ngv * 4;
        union { uint32_t u[4]; half8_t v; } bp;
        int g_cur = -1;
#pragma unroll
        for (int bt = 0; bt < 8; ++bt) {
          const int g = (16 * bt) / a.gv;
          if (g != g_cur) {   // uniform: the B operand of this channel group
            const uint2 sa = *reinterpret_cast<const uint2*>(vsa + 4 * g);
            const uint2 sb = *reinterpret_cast<const uint2*>(vsb + 4 * g);
            const uint32_t sab[4] = {__builtin_amdgcn_perm(sb.x, sa.x, 0x05040100u),
                                     __builtin_amdgcn_perm(sb.x, sa.x, 0x07060302u),
                                     __builtin_amdgcn_perm(sb.y, sa.y, 0x05040100u),
                                     __builtin_amdgcn_perm(sb.y, sa.y, 0x07060302u)};
#pragma unroll
            for (int t = 0; t < 4; ++t) bp.u[t] = as_u32r(as_h2r(pab[t]) * as_h2r(sab[t]));
            g_cur = g;
          }
          const uint32_t x = __builtin_amdgcn_perm(vb4[bt >> 1], va4[bt >> 1],
                                                   (bt & 1) ? 0x07060302u : 0x05040100u);
          union { uint32_t u[4]; half8_t v; } av;
          nibble_pairs(nm, x, av.u);
          acc[bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av.v, bp.v, acc[bt], 0, 0, 0);
        }
      }
    }
    // the scales of group gi + 2 go to slot (gi + 2) % 3, last read by group gi - 1
    count_wave(&s_sync[kSlots + slot]);   // done reading group gi
    if (gi + 2 < n_groups) {
      const int slot2 = (gi + 2) % kSlots;
      if (gi >= 1) wait_count(&s_sync[kSlots + slot2], kRWaves * ((gi - 1) / kSlots + 1));
      store_prefix(pre_n, slot2);
      count_wave(&s_sync[slot2]);
    }
    if (active) {
#pragma unroll
      for (int pp = 0; pp < kRGroupPages; ++pp) {
        kc[pp] = kc_n[pp];
        vc[pp] = vc_n[pp];
      }
    }
  }
  if (active) {
    if constexpr (NSLOT == 4) {
#pragma unroll
      for (int bt = 0; bt < 8; ++bt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[bt][i] += dpp_all_r<kRRowRor + 4>(acc[bt][i]);
      l_run += dpp_all_r<kRRowRor + 4>(l_run);
    }
    if constexpr (NSLOT >= 2) {
#pragma unroll
      for (int bt = 0; bt < 8; ++bt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[bt][i] += dpp_all_r<kRRowRor + 8>(acc[bt][i]);
      l_run += dpp_all_r<kRRowRor + 8>(l_run);
    }
    rtn_store_partial(a, b, split, h, n, q, acc, m_run, l_run);
  }
}

}  // namespace bmx

using namespace bmx;

static int rfail(int code, const std::string& msg) {
  bmx_set_error(msg);
  return code;
}

static bool rtn_geom_ok(const bmx_rtn_geom* g, int max_h, std::string& why) {
  if (!g) { why = "geom is NULL"; return false; }
  if (g->h_kv < 1 || g->h_kv > max_h) { why = "h_kv must be 1.." + std::to_string(max_h); return false; }
  if (g->k_bits < 2 || g->k_bits > 4 || g->v_bits < 2 || g->v_bits > 4) {
    why = "k_bits and v_bits must be 2..4 (4-bit code cells)";
    return false;
  }
  auto gok = [](int x) { return x == 32 || x == 64 || x == 128; };
  if (!gok(g->k_group) || !gok(g->v_group)) { why = "k_group and v_group must be 32, 64 or 128"; return false; }
  if (g->k_arm != BMX_RTN_TOKEN && g->k_arm != BMX_RTN_CHANNEL) {
    why = "k_arm must be BMX_RTN_TOKEN or BMX_RTN_CHANNEL";
    return false;
  }
  return true;
}

extern "C" size_t bmx_rtn_page_bytes(const bmx_rtn_geom* g) {
  std::string why;
  if (!rtn_geom_ok(g, 16, why)) return 0;
  return (size_t)RtnLayout::make(g->h_kv, g->k_arm, g->k_group, g->v_group).bytes;
}

extern "C" int bmx_rtn_append(const bmx_rtn_append_args* a, void* stream) {
  if (!a) return rfail(BMX_E_INVALID, "bmx_rtn_append: args is NULL");
  std::string why;
  if (!rtn_geom_ok(&a->geom, 16, why)) return rfail(BMX_E_INVALID, "bmx_rtn_append: " + why);
  if (a->n_codec_pages < 0) return rfail(BMX_E_INVALID, "bmx_rtn_append: n_codec_pages < 0");
  if (a->n_codec_pages == 0) return BMX_OK;
  if (!a->k || !a->v || !a->pages || !a->page_ids)
    return rfail(BMX_E_INVALID, "bmx_rtn_append: null pointer argument");
  if (a->n_pool_pages < 1) return rfail(BMX_E_INVALID, "bmx_rtn_append: n_pool_pages must be >= 1");
  auto dok = [](int d) { return d == BMX_K2B_F16 || d == BMX_K2B_F32 || d == BMX_K2B_BF16; };
  if (!dok(a->k_dtype) || !dok(a->v_dtype))
    return rfail(BMX_E_INVALID, "bmx_rtn_append: k_dtype / v_dtype must be BMX_K2B_F16, _F32 or _BF16");
  RtnAppendKArgs k{};
  const bmx_rtn_geom& g = a->geom;
  k.h_kv = g.h_kv; k.kbits = g.k_bits; k.vbits = g.v_bits; k.gk = g.k_group; k.gv = g.v_group;
  k.n_pool = a->n_pool_pages;
  k.k = a->k; k.ksh = a->k_stride_h; k.kst = a->k_stride_t; k.kdt = a->k_dtype;
  k.v = a->v; k.vsh = a->v_stride_h; k.vst = a->v_stride_t; k.vdt = a->v_dtype;
  k.pages = a->pages; k.page_ids = a->page_ids; k.karm = g.k_arm;
  k.L = RtnLayout::make(g.h_kv, g.k_arm, g.k_group, g.v_group);
  if (g.k_arm == BMX_RTN_CHANNEL)
    hipLaunchKernelGGL(rtn_append_kchan_kernel, dim3(a->n_codec_pages * (kCodec / g.k_group), g.h_kv), dim3(kD),
                       0, (hipStream_t)stream, k);
  hipLaunchKernelGGL(rtn_append_kernel, dim3(a->n_codec_pages * (kCodec / kPT), g.h_kv), dim3(256), 0,
                     (hipStream_t)stream, k);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return rfail(BMX_E_HIP, std::string("bmx_rtn_append: launch: ") + hipGetErrorString(e));
  return BMX_OK;
}

extern "C" int bmx_rtn_dequant(const bmx_rtn_dequant_args* a, void* stream) {
  if (!a) return rfail(BMX_E_INVALID, "bmx_rtn_dequant: args is NULL");
  std::string why;
  if (!rtn_geom_ok(&a->geom, 16, why)) return rfail(BMX_E_INVALID, "bmx_rtn_dequant: " + why);
  if (a->n_pages < 0) return rfail(BMX_E_INVALID, "bmx_rtn_dequant: n_pages < 0");
  if (a->n_pages == 0) return BMX_OK;
  if (!a->pages || !a->page_ids || !a->k_out || !a->v_out || a->n_pool_pages < 1)
    return rfail(BMX_E_INVALID, "bmx_rtn_dequant: null pointer argument or empty pool");
  if (a->out_dtype < BMX_K2B_F16 || a->out_dtype > BMX_K2B_BF16)
    return rfail(BMX_E_INVALID, "bmx_rtn_dequant: out_dtype must be BMX_K2B_F16, _F32 or _BF16");
  if (a->out_rows != 0 && a->out_rows < (int64_t)a->n_pages * kPT)
    return rfail(BMX_E_INVALID, "bmx_rtn_dequant: out_rows must be 0 or >= 16 * n_pages");
  RtnDequantKArgs k{};
  const bmx_rtn_geom& g = a->geom;
  k.h_kv = g.h_kv; k.n_pool = a->n_pool_pages; k.pages = a->pages; k.page_ids = a->page_ids;
  k.n_tok = a->out_rows ? a->out_rows : (int64_t)a->n_pages * kPT; k.k_out = a->k_out; k.v_out = a->v_out; k.out_dtype = a->out_dtype;
  k.gk = g.k_group; k.gv = g.v_group; k.karm = g.k_arm;
  k.L = RtnLayout::make(g.h_kv, g.k_arm, g.k_group, g.v_group);
  hipLaunchKernelGGL(rtn_dequant_kernel, dim3(a->n_pages, g.h_kv), dim3(256), 0, (hipStream_t)stream, k);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return rfail(BMX_E_HIP, std::string("bmx_rtn_dequant: launch: ") + hipGetErrorString(e));
  return BMX_OK;
}

static int rtn_cu_count() { return bmx_device_cu_count(); }

// as for k2b: one workgroup per CU over the batch (or split_tokens), never more
// than the 64-token groups, and at least one per 16-token window tile (up to
// one per CU)
static int rtn_choose_splits(const bmx_rtn_decode_args* a) {
  const int units = (a->max_packed_len + kRGroup - 1) / kRGroup;
  const int per_seq = std::max(1, rtn_cu_count() / a->batch);
  int S = a->split_tokens > 0 ? (a->max_packed_len + a->split_tokens - 1) / a->split_tokens : per_seq;
  if (S > units) S = units;
  const int tiles = (a->tail_cap + 15) / 16;
  if (S < tiles) S = std::min(tiles, std::max(S, per_seq));
  return S < 1 ? 1 : S;
}

static size_t rtn_ws_bytes(const bmx_rtn_decode_args* a, int splits) {
  const size_t rows = (size_t)a->batch * a->geom.h_kv * a->geom.n_q_groups;
  return partial_bytes(rows, (size_t)splits) + rows * (size_t)a->tail_cap * sizeof(float);
}

extern "C" size_t bmx_rtn_decode_workspace_bytes(const bmx_rtn_decode_args* a) {
  if (!a || a->batch < 1) return 0;
  return rtn_ws_bytes(a, rtn_choose_splits(a));
}

template <int SW, bool kNT>
static void launch_rtn_split_nt(int ngk, dim3 grid, const RtnDecodeKArgs& k, hipStream_t st) {
  if (ngk == 0)
    hipLaunchKernelGGL((rtn_decode_split_kernel<SW, 0, kNT>), grid, dim3(kRThreads), 0, st, k);
  else if (ngk == 4)
    hipLaunchKernelGGL((rtn_decode_split_kernel<SW, 4, kNT>), grid, dim3(kRThreads), 0, st, k);
  else if (ngk == 2)
    hipLaunchKernelGGL((rtn_decode_split_kernel<SW, 2, kNT>), grid, dim3(kRThreads), 0, st, k);
  else
    hipLaunchKernelGGL((rtn_decode_split_kernel<SW, 1, kNT>), grid, dim3(kRThreads), 0, st, k);
}

// Page loads are non-temporal when a call reads at least kRNtBytes of pages:
// from there a 32-layer step's calls exceed the 256 MB MALL and stream from
// HBM (non-temporal measured faster from 8k tokens at h_kv 8); below it a
// step's pages stay in the MALL, which non-temporal reads would bypass
// (measured slower at 4k).
constexpr int64_t kRNtBytes = 8ll << 20;

template <int SW>
static void launch_rtn_split(int ngk, bool nt, dim3 grid, const RtnDecodeKArgs& k, hipStream_t st) {
  if (nt)
    launch_rtn_split_nt<SW, true>(ngk, grid, k, st);
  else
    launch_rtn_split_nt<SW, false>(ngk, grid, k, st);
}

extern "C" int bmx_rtn_decode(const bmx_rtn_decode_args* a, void* stream) {
  if (!a) return rfail(BMX_E_INVALID, "bmx_rtn_decode: args is NULL");
  std::string why;
  if (!rtn_geom_ok(&a->geom, kRWaves, why)) return rfail(BMX_E_INVALID, "bmx_rtn_decode: " + why);
  const bmx_rtn_geom& g = a->geom;
  if (g.n_q_groups < 1 || g.n_q_groups > 16)
    return rfail(BMX_E_INVALID, "bmx_rtn_decode: n_q_groups must be 1..16");
  if (a->batch < 1) return rfail(BMX_E_INVALID, "bmx_rtn_decode: batch must be >= 1");
  if (a->max_packed_len < 0 || a->max_packed_len % kCodec != 0)
    return rfail(BMX_E_INVALID, "bmx_rtn_decode: max_packed_len must be a multiple of 128");
  if (a->max_packed_len > 0 && a->max_pages * kPT < a->max_packed_len)
    return rfail(BMX_E_INVALID, "bmx_rtn_decode: max_pages*16 < max_packed_len");
  if (a->tail_cap < 0 || a->tail_cap > 4096)
    return rfail(BMX_E_INVALID, "bmx_rtn_decode: tail_cap must be 0..4096");
  if (a->split_tokens < 0 || a->split_tokens % kRGroup != 0)
    return rfail(BMX_E_INVALID, "bmx_rtn_decode: split_tokens must be a multiple of 64");
  if (!a->q || !a->out || !a->packed_len)
    return rfail(BMX_E_INVALID, "bmx_rtn_decode: q/out/packed_len must be non-NULL");
  if (a->io_dtype < BMX_K2B_IO_F32 || a->io_dtype > BMX_K2B_IO_BF16)
    return rfail(BMX_E_INVALID, "bmx_rtn_decode: io_dtype must be BMX_K2B_IO_F32, _F16 or _BF16");
  if (a->tail_dtype != BMX_K2B_TAIL_F16 && a->tail_dtype != BMX_K2B_TAIL_BF16)
    return rfail(BMX_E_INVALID, "bmx_rtn_decode: tail_dtype must be BMX_K2B_TAIL_F16 or _BF16");
  if (!a->tail_len && (a->tail_len_value < 0 || a->tail_len_value > a->tail_cap))
    return rfail(BMX_E_INVALID, "bmx_rtn_decode: with tail_len NULL, tail_len_value must be 0..tail_cap");
  if (a->n_new < 0 || (a->n_new > 0 && (a->tail_len || a->n_new > a->tail_len_value || !a->new_k ||
                                        !a->new_v)))
    return rfail(BMX_E_INVALID, "bmx_rtn_decode: n_new rows given apart need tail_len NULL, "
                                "n_new <= tail_len_value and new_k/new_v non-NULL");
  if (a->n_new > 0 && (a->new_stride_b % 8 != 0 || a->new_stride_h % 8 != 0 || a->new_stride_t % 8 != 0))
    return rfail(BMX_E_INVALID, "bmx_rtn_decode: new_k/new_v strides must be multiples of 8 elements");
  if (a->max_packed_len > 0 && (!a->pages || !a->page_table || a->n_pool_pages < 1))
    return rfail(BMX_E_INVALID, "bmx_rtn_decode: pages/page_table must be non-NULL and the pool non-empty");
  if (a->tail_cap > 0 && (!a->k_tail || !a->v_tail))
    return rfail(BMX_E_INVALID, "bmx_rtn_decode: k_tail/v_tail must be non-NULL when tail_cap > 0");
  if (a->tail_cap > 0 && (a->tail_stride_t % 8 != 0 || a->tail_stride_h % 8 != 0 || a->tail_stride_b % 8 != 0))
    return rfail(BMX_E_INVALID, "bmx_rtn_decode: tail strides must be multiples of 8 elements");
  const int S = rtn_choose_splits(a);
  if (S > 8192) return rfail(BMX_E_INVALID, "bmx_rtn_decode: more than 8192 splits; use a larger split_tokens");
  const size_t need = rtn_ws_bytes(a, S);
  if (!a->workspace || a->workspace_bytes < need)
    return rfail(BMX_E_WORKSPACE, "bmx_rtn_decode: workspace missing or smaller than "
                                  "bmx_rtn_decode_workspace_bytes()");
  const size_t rows = (size_t)a->batch * S * g.h_kv * g.n_q_groups;
  uint16_t* ws_acc = (uint16_t*)a->workspace;
  float* ws_ml = (float*)(ws_acc + rows * kD);
  float* ws_win = ws_ml + rows * 2;
  hipStream_t st = (hipStream_t)stream;

  RtnDecodeKArgs k{};
  k.h_kv = g.h_kv; k.G = g.n_q_groups; k.max_splits = S; k.max_pages = a->max_pages;
  k.max_packed_len = a->max_packed_len; k.n_pool = a->n_pool_pages > 0 ? a->n_pool_pages : 1;
  k.gk = g.k_group; k.gv = g.v_group;
  k.L = RtnLayout::make(g.h_kv, g.k_arm, g.k_group, g.v_group);
  k.prefix_bytes = k.L.kcode;
  k.q = a->q; k.io_dtype = a->io_dtype; k.ws_acc = ws_acc; k.ws_ml = ws_ml;
  k.pages = a->pages; k.page_table = a->page_table; k.packed_len = a->packed_len;
  k.qscale = a->sm_scale * 1.4426950408889634f;
  k.k_tail = a->k_tail; k.ts_b = a->tail_stride_b; k.ts_h = a->tail_stride_h; k.ts_t = a->tail_stride_t;
  k.tail_bf16 = a->tail_dtype == BMX_K2B_TAIL_BF16;
  k.tail_cap = a->tail_cap; k.win_rescale = 1.0f; k.ws_win = ws_win;
  k.nw.k = a->new_k; k.nw.v = a->new_v;
  k.nw.sb = a->new_stride_b; k.nw.sh = a->new_stride_h; k.nw.st = a->new_stride_t;
  k.nw.n = a->n_new;
  k.nw.T = a->tail_len ? -1 : a->tail_len_value;
  k.nw.k_dst = const_cast<uint16_t*>(a->k_tail);
  k.nw.v_dst = const_cast<uint16_t*>(a->v_tail);
  dim3 grid(S, a->batch);
  const int ngk = g.k_arm == BMX_RTN_CHANNEL ? 0 : kD / g.k_group;
  const bool nt = (int64_t)a->batch * (a->max_packed_len / kPT) * k.L.bytes >= kRNtBytes;
  if (g.n_q_groups <= 4)
    launch_rtn_split<4>(ngk, nt, grid, k, st);
  else if (g.n_q_groups <= 8)
    launch_rtn_split<8>(ngk, nt, grid, k, st);
  else
    launch_rtn_split<16>(ngk, nt, grid, k, st);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return rfail(BMX_E_HIP, std::string("bmx_rtn_decode: split kernel launch: ") + hipGetErrorString(e));
  CombineKArgs c{};
  c.h_kv = g.h_kv; c.G = g.n_q_groups; c.max_splits = S; c.tail_cap = a->tail_cap;
  c.out = a->out; c.io_dtype = a->io_dtype; c.ws_acc = ws_acc; c.ws_ml = ws_ml; c.ws_win = ws_win;
  c.v_tail = a->v_tail;
  c.ts_b = a->tail_stride_b; c.ts_h = a->tail_stride_h; c.ts_t = a->tail_stride_t;
  c.tail_bf16 = k.tail_bf16;
  c.tail_len = a->tail_len;
  c.nw = k.nw;
  c.packed_scale = 1.0f;
  launch_combine<false>(c, g.h_kv * g.n_q_groups, a->batch, st);
  e = hipGetLastError();
  if (e != hipSuccess)
    return rfail(BMX_E_HIP, std::string("bmx_rtn_decode: combine kernel launch: ") + hipGetErrorString(e));
  return BMX_OK;
}
