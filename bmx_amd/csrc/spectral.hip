// Spectral (K4) key path on gfx950: the write kernel (encode, MSE-refined RTN
// per direction, page packing) and the dense dequantization (tier codes ->
// Y_hat, Y_hat dec^T on MFMA, RoPE), with the k2b value codec in value-only
// pages.  Reference semantics: cache/spectral.py:763-841, quant/rtn.py:10-53,
// cache/chunked_attention.py:52-194; the page format is in
// include/bmx_spectral.h.  Built without floating-point contraction: every
// product and sum of the write kernel is rounded on its own, in a fixed order.

#include <mutex>
#include <type_traits>

#include "bmx_spectral.h"
#include "k2b_common.h"

namespace bmx {

constexpr int kSpCh = 64;                          // key channels staged per pass
constexpr int kSpMaxSlices = BMX_SPECTRAL_MAX_CPAD / 8;

__device__ __forceinline__ int sp_width(int b) { return b == 2 ? 2 : (b <= 4 ? 4 : 8); }

// The Lloyd payload's level table: tier b's 2^b levels at lq_off(b)
constexpr int kLqLevels = BMX_SPECTRAL_LLOYD_LEVELS;
__device__ __forceinline__ int lq_off(int b) { return b == 8 ? 124 : (1 << b) - 4; }

// Pair tables of the narrow Lloyd tiers (2, 3, 4): entry key of tier b holds
// the fp16 levels of the two codes in the key's 2w bits (w the container
// width), low code first; 16 entries for tier 2, 256 each for tiers 3 and 4.
constexpr int kLqPairs = 16 + 256 + 256;
__device__ __forceinline__ int lq_pair_base(int b) { return b == 2 ? 0 : (b == 3 ? 16 : 272); }

// Entry i of the pair tables from the fp32 levels lq (kLqLevels)
__device__ __forceinline__ uint32_t lq_pair_entry(const float* lq, int i) {
  const int b = i < 16 ? 2 : (i < 272 ? 3 : 4), key = i - lq_pair_base(b);
  const int w = sp_width(b), m = (1 << b) - 1;
  const half2_t h = {(_Float16)lq[lq_off(b) + (key & m)], (_Float16)lq[lq_off(b) + ((key >> w) & m)]};
  return as_u32(h);
}

// Index of the level nearest to x among tier b's sorted levels: the number of
// the 2^b - 1 midpoints mid[0 ..] below x (torch.bucketize, right=False)
__device__ __forceinline__ int lq_index(const float* mid, int b, float x) {
  int i = 0;
  for (int k = b - 1; k >= 0; --k)
    if (mid[i + (1 << k) - 1] < x) i += 1 << k;
  return i;
}

// sin and cos of an fp32 angle x (|x| < 2^40): x - k pi/2 in double (pi/2 in
// two parts, the first with 33 significant bits so that k times it is exact),
// rounded once to fp32 (|r| <= pi/4: within 3e-8 of the exact reduced angle),
// then the fp32 sin/cos of r on its short path and the quadrant's swap and
// signs.  The library's sincosf takes a long reduction for large arguments
// (positions times frequencies reach 1e5 at long context).
// (cos, sin) of x - e from those of x, |e| <= 2^-7 (half an fp32 ulp at 2^17):
// cos e and sin e to second and third order (the next terms are below 1e-10)
__device__ __forceinline__ void rotate_back(float c, float s, float e, float* cn, float* sn) {
  const float e2 = e * e;
  const float ce = __builtin_fmaf(-0.5f, e2, 1.0f), se = e * __builtin_fmaf(-e2, 1.0f / 6.0f, 1.0f);
  *cn = __builtin_fmaf(c, ce, s * se);
  *sn = __builtin_fmaf(s, ce, -(c * se));
}

__device__ __forceinline__ void sincos_reduced(float x, float* sn, float* cn) {
  const double xd = x;
  const double k = rint(xd * 0.63661977236758134308);   // 2/pi
  double rd = __builtin_fma(-k, 1.5707963267341256142, xd);     // pi/2, high part
  rd = __builtin_fma(-k, 6.0771005065061922e-11, rd);            // pi/2 - high part
  float sr, cr;
  sincosf((float)rd, &sr, &cr);
  const int qd = (int)(int64_t)k & 3;
  *sn = qd == 0 ? sr : qd == 1 ? cr : qd == 2 ? -sr : -cr;
  *cn = qd == 0 ? cr : qd == 1 ? -sr : qd == 2 ? -cr : sr;
}

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
  const float* lq;   // the Lloyd levels, or nullptr (rtn payload)
};

// grid (ceil(c_pad / 64), n_groups), block 512: wave w of block x
// accumulates Y[t][j] for tokens 8w .. 8w + 7 of group y and page column
// 64x + j (lane j) over the C channels, staged 64 at a time through LDS with
// the chunk's enc rows (every product and sum rounded on its own, channels in
// order); then wave 0's lane j takes column 64x + j's 64 values from LDS for
// the step (max|Y| / qmax and 10 rounds of <Y, Q> / <Q, Q>; for the Lloyd
// payload the sample deviation and 3 rounds of <Y, l> / <l, l>) and its
// codes, and the block's 8 slices are assembled in LDS and written with dword
// stores.
template <bool kLloyd>
__global__ __launch_bounds__(512) void spectral_encode_kernel(const SpEncodeKArgs a) {
  __shared__ __align__(16) float s_m[kGroup][kSpCh + 4];   // the chunk's keys: [token][channel] (row pad 4: measured faster than 1)
  __shared__ float s_e[kSpCh][64];           // the chunk's enc rows: [channel][column]
  __shared__ float s_y[kGroup][65];          // Y: [token][column]
  __shared__ uint32_t s_code[8 * kGroup * 8 / 4];   // 8 slices of at most 512 bytes
  __shared__ float s_lv[kLloyd ? kLqLevels : 1], s_mid[kLloyd ? kLqLevels : 1];   // levels, midpoints
  __shared__ float s_l[kLloyd ? kGroup : 1][65];      // Lloyd: the level of each (token, column)
  __shared__ uint8_t s_cd[kLloyd ? kGroup : 1][64];   // Lloyd: the final level indices
  __shared__ float s_sc[64];                          // Lloyd: each column's current step
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = blockIdx.x * 64 + lane, g = blockIdx.y;
  const bool active = j < a.c_pad;
  constexpr bool lloyd = kLloyd;
  if (lloyd)
    for (int i = tid; i < kLqLevels; i += 512) s_lv[i] = a.lq[i];
  float y[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) y[t] = 0.f;
  // the next chunk's keys and enc rows are loaded into registers while the
  // current one is summed
  float mreg[8], ereg[8];
  auto load_chunk = [&](int c0) {
    const int c = c0 + lane, h = c >> 7, d = c & (kD - 1);
#pragma unroll
    for (int t = 0; t < 8; ++t)
      mreg[t] = sp_load(a.k, h * a.ksh + (int64_t)(g * kGroup + 8 * wave + t) * a.kst + d, a.k_dtype);
#pragma unroll
    for (int r = 0; r < 8; ++r)
      ereg[r] = active ? a.encp[(int64_t)(c0 + 8 * wave + r) * a.c_pad + j] : 0.f;
  };
  load_chunk(0);
  for (int c0 = 0; c0 < a.C; c0 += kSpCh) {
    __syncthreads();   // the previous chunk read
#pragma unroll
    for (int t = 0; t < 8; ++t) s_m[8 * wave + t][lane] = mreg[t];
#pragma unroll
    for (int r = 0; r < 8; ++r) s_e[8 * wave + r][lane] = ereg[r];
    __syncthreads();
    if (c0 + kSpCh < a.C) load_chunk(c0 + kSpCh);
    // channels in order (16-byte reads of 4 channels measured slower)
#pragma unroll 4
    for (int cc = 0; cc < kSpCh; ++cc) {
      const float e = s_e[cc][lane];
#pragma unroll
      for (int t = 0; t < 8; ++t) y[t] = __fadd_rn(y[t], __fmul_rn(s_m[8 * wave + t][cc], e));
    }
  }
#pragma unroll
  for (int t = 0; t < 8; ++t) s_y[8 * wave + t][lane] = y[t];
  // midpoints (l_i + l_{i+1}) / 2 within each tier (the slot after a tier's
  // last level is never read); s_lv was written before the chunk loop's barriers
  if (lloyd)
    for (int i = tid; i + 1 < kLqLevels; i += 512) s_mid[i] = (s_lv[i] + s_lv[i + 1]) * 0.5f;
  __syncthreads();
  const int s = j >> 3, k = j & 7;
  const uint32_t tab = active ? (uint32_t)a.slice_tab[s] : 0u;
  const int b = active ? (int)(tab >> 24) : 2, w = sp_width(b);
  const float qmax = (float)((1 << (b - 1)) - 1);
  const float* lv = s_lv + (kLloyd ? lq_off(b) : 0);
  const float* mid = s_mid + (kLloyd ? lq_off(b) : 0);
  float scale = 1e-12f;
  if constexpr (kLloyd) {
    // the starting step in wave 0 (lane = column), then 4 rounds: every wave
    // finds the level indices of 8 tokens (binary searches in parallel), and
    // for the 3 refits wave 0 sums <Y, l> and <l, l> left to right
    if (wave == 0) {
      double sum = 0.0;
      for (int t = 0; t < kGroup; ++t) sum += (double)s_y[t][lane];
      const double mean = sum / 64.0;
      double ss = 0.0;
      for (int t = 0; t < kGroup; ++t) {
        const double d = (double)s_y[t][lane] - mean;
        ss += d * d;
      }
      s_sc[lane] = fmaxf((float)__dsqrt_rn(ss / 63.0), 1e-12f);
    }
    for (int r = 0; r <= 3; ++r) {
      __syncthreads();   // the step written; the previous round's levels read
      const float sc = s_sc[lane];
      for (int t = wave; t < kGroup; t += 8) {
        const int c = lq_index(mid, b, s_y[t][lane] / sc);
        if (r < 3) s_l[t][lane] = lv[c];
        else s_cd[t][lane] = (uint8_t)c;
      }
      if (r == 3) break;
      __syncthreads();
      if (wave == 0) {
        float num = 0.f, den = 0.f;
        for (int t = 0; t < kGroup; ++t) {
          const float yv = s_y[t][lane], l = s_l[t][lane];
          num = __fadd_rn(num, __fmul_rn(yv, l));
          den = __fadd_rn(den, __fmul_rn(l, l));
        }
        s_sc[lane] = fmaxf(num / fmaxf(den, 1e-12f), 1e-12f);
      }
    }
    scale = s_sc[lane];
  } else if (active && wave == 0) {
    float amax = 0.f;
    for (int t = 0; t < kGroup; ++t) amax = fmaxf(amax, fabsf(s_y[t][lane]));
    scale = fmaxf(amax, 1e-12f) / qmax;
    for (int it = 0; it < 10; ++it) {
      float num = 0.f, den = 0.f;
      for (int t = 0; t < kGroup; ++t) {
        const float yv = s_y[t][lane];
        const float qv = fminf(fmaxf(rintf(yv / scale), -qmax - 1.f), qmax);
        num = __fadd_rn(num, __fmul_rn(yv, qv));
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
  for (int i = tid; i < n_words; i += 512) s_code[i] = 0u;
  __syncthreads();
  if (active && wave == 0) {
    const int bit0 = ((int)(tab & 0xFFFFFFu) - base) * 8 + k * w;
    const uint32_t bias = 1u << (b - 1);
    for (int t = 0; t < kGroup; ++t) {
      const float qv = fminf(fmaxf(rintf(s_y[t][lane] / scale), -qmax - 1.f), qmax);
      const uint32_t stored = lloyd ? (uint32_t)s_cd[kLloyd ? t : 0][lane] : (uint32_t)((int)qv + (int)bias);
      const int bit = bit0 + t * w * 8;
      atomicOr(&s_code[bit >> 5], stored << (bit & 31));
    }
  }
  __syncthreads();
  uint8_t* page = a.pages + clamp_page(a.page_ids[g], a.n_pool) * (int64_t)a.page_bytes;
  uint32_t* dst = reinterpret_cast<uint32_t*>(page + base);
  for (int i = tid; i < n_words; i += 512) dst[i] = s_code[i];
  if (active && wave == 0) reinterpret_cast<uint16_t*>(page)[j] = float_to_half_bits(scale);
}

struct SpVFullKArgs {
  int h_kv, n_pool, v_dtype;
  const void* v;
  int64_t vsh, vst;
  uint8_t* pages;
  const int32_t* page_ids;
  PageLayout L;
  float codebook[4];
  uint32_t sign_c[32];
};

constexpr int kSpMaxC = 1024;

// The full-C value codec (codecs.py:616-636 at h = 1): grid (16-token pages x
// 4), block 256, one quarter q of a page (tokens 4q .. 4q + 3: the tokens of
// one VCODE dword) per workgroup.  Per token the fp16 norm of all C channels
// (squares in 8 strided fp32 FMA accumulators, then those left to right:
// torch's CPU order), the unit row times the C signs, a C-point FWHT in LDS
// (stages as quant/hadamard.py:19-25), / sqrt(C) * sqrt(C) in fp32, then the
// 2-bit codes against the codebook's midpoints, packed per 128-channel slice
// in the per-head VCODE layout.
constexpr int kVfTok = 4;   // tokens per workgroup
__global__ __launch_bounds__(256) void spectral_vfull_kernel(const SpVFullKArgs a) {
  const int pg = blockIdx.x >> 2, qt = blockIdx.x & 3, tid = threadIdx.x;
  const int C = kD * a.h_kv, lc = 7 + __builtin_ctz((unsigned)a.h_kv);   // C = 2^lc (h_kv a power of two)
  __shared__ float x[kVfTok][kSpMaxC];
  __shared__ float s_acc[kVfTok][8];
  __shared__ float s_norm[kVfTok];
  __shared__ uint8_t code[kVfTok][kSpMaxC];
  uint8_t* page = a.pages + clamp_page(a.page_ids[pg], a.n_pool) * (int64_t)a.L.bytes;
  const int tok0 = pg * kPT + kVfTok * qt;
  for (int e = tid; e < kVfTok * C; e += 256) {
    const int t = e >> lc, c = e & (C - 1);
    x[t][c] = sp_load(a.v, (c >> 7) * a.vsh + (int64_t)(tok0 + t) * a.vst + (c & (kD - 1)), a.v_dtype);
  }
  __syncthreads();
  if (tid < kVfTok * 8) {
    const int t = tid >> 3, j = tid & 7;
    float acc = 0.f;
#pragma unroll 16
    for (int i = j; i < C; i += 8) acc = __builtin_fmaf(x[t][i], x[t][i], acc);
    s_acc[t][j] = acc;
  }
  __syncthreads();
  if (tid < kVfTok) {
    float ss = s_acc[tid][0];
#pragma unroll
    for (int j = 1; j < 8; ++j) ss = ss + s_acc[tid][j];
    const float nrm = fmaxf(__builtin_sqrtf(ss), 1e-12f);
    const uint16_t nb = float_to_half_bits(nrm);
    s_norm[tid] = half_bits_to_float(nb);
    reinterpret_cast<uint16_t*>(page + a.L.vnorm)[kVfTok * qt + tid] = nb;
  }
  __syncthreads();
  for (int e = tid; e < kVfTok * C; e += 256) {
    const int t = e >> lc, c = e & (C - 1);
    const float u = x[t][c] / s_norm[t];
    x[t][c] = ((a.sign_c[c >> 5] >> (c & 31)) & 1u) ? -u : u;
  }
  __syncthreads();
  for (int lh = 0; lh < lc; ++lh) {   // butterflies (i, i + hb), hb = 2^lh, as the reference's stages
    const int hb = 1 << lh;
    for (int e = tid; e < kVfTok * C / 2; e += 256) {
      const int t = e >> (lc - 1), pidx = e & (C / 2 - 1);
      const int i0 = ((pidx >> lh) << (lh + 1)) | (pidx & (hb - 1));
      const float u = x[t][i0], w = x[t][i0 + hb];
      x[t][i0] = u + w;
      x[t][i0 + hb] = u - w;
    }
    __syncthreads();
  }
  // fl32(sqrt(C)), applied as / then *, as the reference does
  const float sqrt_c = C == 128 ? 11.313708498984761f : C == 256 ? 16.f : C == 512 ? 22.627416997969522f : 32.f;
  const float mid0 = (a.codebook[0] + a.codebook[1]) / 2.0f;
  const float mid1 = (a.codebook[1] + a.codebook[2]) / 2.0f;
  const float mid2 = (a.codebook[2] + a.codebook[3]) / 2.0f;
  for (int e = tid; e < kVfTok * C; e += 256) {
    const int t = e >> lc, c = e & (C - 1);
    const float r = (x[t][c] / sqrt_c) * sqrt_c;
    code[t][c] = (uint8_t)((r > mid0) + (r > mid1) + (r > mid2));
  }
  __syncthreads();
  // slice sl, lane 16 qt + m, dword w: channel 128 sl + 16 (4w + bb) + m, token 4 qt + t at bit 8bb + 2t
  if (tid < a.h_kv * 32) {
    const int sl = tid >> 5, m = (tid >> 1) & 15, w = tid & 1, lane = 16 * qt + m;
    uint32_t dword = 0;
#pragma unroll
    for (int bb = 0; bb < 4; ++bb) {
      const int c = 128 * sl + 16 * (4 * w + bb) + m;
#pragma unroll
      for (int t = 0; t < kVfTok; ++t) dword |= (uint32_t)code[t][c] << (8 * bb + 2 * t);
    }
    *reinterpret_cast<uint32_t*>(page + a.L.vcode + sl * 512 + lane * 8 + w * 4) = dword;
  }
}

struct SpDequantKArgs {
  int h_kv, c_pad, c_pad32, n_tokens, out_rows, apply_rope, n_k_pool, n_v_pool, out_dtype, k_page_bytes;
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
  const void* q;
  int q_dtype, n_q_groups;
  float* scores;
  float* partials;
  float sm_scale;
  const float* lq;   // the Lloyd levels, or nullptr (rtn payload)
  int v_full;        // values: the full-C codec (one norm per token, C-wide codes)
  uint32_t v_sign_c[32];
};

// Full-C values, one 16-token page: lane (q, n)'s 2-bit codes of every slice
// (slice sl at VCODE + 512 sl), and the H_{C/128} row h sign of slice sl
__device__ __forceinline__ bool vfull_neg(int h, int sl) { return __builtin_popcount((unsigned)(h & sl)) & 1; }

// Rotated-domain values of head h for the lane's 4 tokens x 8 channel
// blocks: y[tt][b] = sum over slices sl of (-1)^popcount(h & sl) times the
// level of slice sl's code (then H128 over the slice's channels gives head
// h's channels, the Kronecker form of the C-point Hadamard)
__device__ __forceinline__ void vfull_y(const uint8_t* vp, int vcode, int h_kv, int h, int lane, const float cb[4],
                                        float (&y)[4][8]) {
  u32x2_t cs[8];
#pragma unroll
  for (int sl = 0; sl < 8; ++sl)
    cs[sl] = *reinterpret_cast<const u32x2_t*>(vp + vcode + min(sl, h_kv - 1) * 512 + lane * 8);
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int b = 0; b < 8; ++b) y[tt][b] = 0.f;
#pragma unroll
  for (int sl = 0; sl < 8; ++sl) {
    if (sl >= h_kv) break;
    const bool neg = vfull_neg(h, sl);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const uint32_t D = b < 4 ? cs[sl].x : cs[sl].y;
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const float l = level4((D >> (8 * (b & 3) + 2 * tt)) & 3u, cb[0], cb[1], cb[2], cb[3]);
        y[tt][b] = neg ? y[tt][b] - l : y[tt][b] + l;
      }
    }
  }
}

constexpr int kSpBRow = 40;   // halves per token row of the staged code tile (32 + 8 pad)
constexpr int kSpMaxKPage = 72 * 1024;   // key page bytes staged in LDS at most (c_pad 1072, 8 bits: 70768)
constexpr int kSpPageLoads = kSpMaxKPage / (16 * 512);   // 16-byte loads per thread at most
// dynamic LDS of the dequant kernel: the group's key page while the main loop
// decodes it, then the waves' staging tiles
constexpr size_t sp_dyn_bytes(int k_page_bytes) {
  return (size_t)k_page_bytes > 8 * sizeof(DqTile) ? (size_t)k_page_bytes : 8 * sizeof(DqTile);
}

// Workgroup barrier over LDS only: this wave's LDS accesses complete, then
// s_barrier.  Global loads in flight stay in flight (__syncthreads would wait
// for them too, and with them for the next step's prefetched dec rows).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// The MFMA operands of Y_hat dec^T.  Below tier kSpWideTier the B side holds
// fp16(code * step) (exact for 2-bit codes, one rounding for 3 and 4 bits);
// from it on, where the codes are wide and the directions the ones of
// largest variance, the B side holds the code itself (exact) and the A side
// the dec rows times the step (one rounding of an exact product), so that no
// wide product is rounded: in fp16 that rounding of the leading directions
// was the largest error of the keys.  Tiers ascend in the page, so the narrow
// slices lead; the steps made of them alone skip the A-side products.
constexpr uint32_t kSpWideTier = 5;
// Codes 0 .. 255 of width w from the low bits of word, 4 of them as fp16
// (1024 + c, from the bits, minus 1024 + 2^(b-1)).
__device__ __forceinline__ uint2 sp_codes4(uint64_t word, int w, int b) {
  const uint32_t mask = (1u << w) - 1u;
  uint32_t c[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) c[e] = ((uint32_t)(word >> (e * w)) & mask) | 0x6400u;
  const uint32_t off = 0x6400u | (1u << (b - 1));   // fp16 1024 + 2^(b-1): spacing 1 in [1024, 2048)
  const half2_t o2 = as_h2(off | (off << 16));
  return make_uint2(as_u32(as_h2(c[0] | (c[1] << 16)) - o2), as_u32(as_h2(c[2] | (c[3] << 16)) - o2));
}

// Partial records, per (head, query) row r of n_parts partials: (m, l) of
// partial p at row base + 2p, its channels 16k .. 16k + 15 at row base +
// 2 n_parts + 16 (k n_parts + p): a merge workgroup of one 16-channel chunk
// reads contiguous records.
__device__ __forceinline__ float* sp_part_ml(float* partials, int64_t r, int n_parts, int p) {
  return partials + r * 130 * (int64_t)n_parts + 2 * p;
}
__device__ __forceinline__ float* sp_part_ch(float* partials, int64_t r, int n_parts, int chunk, int p) {
  return partials + r * 130 * (int64_t)n_parts + 2 * (int64_t)n_parts + 16 * ((int64_t)chunk * n_parts + p);
}

// The 128-point Hadamard (unnormalized; pairs (a, b) -> (a + b, a - b)) of
// the channel sums, channel 16 ct + n: H8 over ct = H over the channel's
// bits 4..6, applied to each partial by the dequant kernels; H16 over n (bits
// 0..3, within a 16-channel chunk), applied by the merge to the merged sums
// of its chunk, held by the lanes n of one 16-lane row.
// The partner lanes come by DPP within the 16-lane row (no LDS crossbar):
// lane ^ 1 and ^ 2 by quad permutes, ^ 4 by a quad reversal then the
// half-row mirror (i ^ 3 ^ 7), ^ 8 by a row rotation of 8.
template <int kCtrl>
__device__ __forceinline__ float dpp_f(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), kCtrl, 0xF, 0xF, true));
}

__device__ __forceinline__ float h16_lanes(float x, int n) {
  float o = dpp_f<0xB1>(x);                 // quad_perm [1, 0, 3, 2]
  x = (n & 1) ? o - x : x + o;
  o = dpp_f<0x4E>(x);                       // quad_perm [2, 3, 0, 1]
  x = (n & 2) ? o - x : x + o;
  o = dpp_f<0x141>(dpp_f<0x1B>(x));         // quad_perm [3, 2, 1, 0], row_half_mirror
  x = (n & 4) ? o - x : x + o;
  o = dpp_f<0x128>(x);                      // row_ror:8
  x = (n & 8) ? o - x : x + o;
  return x;
}

__device__ __forceinline__ uint32_t sp_hmul2(uint32_t x, uint32_t y) { return as_u32(as_h2(x) * as_h2(y)); }

constexpr uint32_t kHalfOnes = 0x3C003C00u;   // fp16 (1, 1)

// The B-side factor of slice s's 8 columns (the fp16 steps of a narrow tier,
// else 1) and the A-side one (1 for a narrow tier, else the steps; 0 past the
// last slice, whose codes are stored as 0 too), from the key page in LDS.
__device__ __forceinline__ uint4 sp_b_factor(const uint8_t* kp, int s_clamped, int b) {
  // read always, chosen by a mask: a select of the load became a branch
  // around it, splitting the main loop's basic block
  const uint4 r = *reinterpret_cast<const uint4*>(kp + 16 * s_clamped);
  const uint32_t keep = (uint32_t)b < kSpWideTier ? 0xFFFFFFFFu : 0u, ones = kHalfOnes & ~keep;
  return make_uint4((r.x & keep) | ones, (r.y & keep) | ones, (r.z & keep) | ones, (r.w & keep) | ones);
}

__device__ __forceinline__ half8_t sp_a_factor(const uint8_t* kp, const uint32_t* s_tab, int s, int n_sl) {
  const int sc = min(s, n_sl - 1);
  const uint4 r = *reinterpret_cast<const uint4*>(kp + 16 * sc);
  const bool narrow = (s_tab[sc] >> 24) < kSpWideTier, ok = s < n_sl;
  const uint32_t f[4] = {r.x, r.y, r.z, r.w};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = ok ? (narrow ? kHalfOnes : f[i]) : 0u;
  return __builtin_bit_cast(half8_t, make_uint4(o[0], o[1], o[2], o[3]));
}

// Leading 32-column steps made of narrow slices only (their A side is the dec
// rows as they are).  tabv: this thread's slice_tab entry (slice min(tid,
// n_sl - 1)); every thread of the block calls this, in place of a barrier.
__device__ __forceinline__ int sp_narrow_steps(uint32_t tabv, int tid, int n_sl, int n_steps) {
  const int nn = __syncthreads_count(tid < n_sl && (tabv >> 24) < kSpWideTier);
  // the count is the narrow prefix only if no wide slice comes before slice nn
  const int out_of_order = __syncthreads_count(tid < nn && (tabv >> 24) >= kSpWideTier);
  if (out_of_order) return 0;
  return nn == n_sl ? n_steps : nn >> 2;
}

// grid (n_tokens / 64), block 512: one 64-token group, wave w = head w.  The
// group's key page is copied to LDS first (one round trip for the whole page,
// issued with every other load of the prologue).  Per 32-column step the
// group's code tile (exact fp16 integers) is decoded from there
// once, by all 512 threads (4 codes each), into one of two LDS buffers; every
// head's wave reads its B fragments from there (lane 16q + n: token n of the
// tile, columns 8q .. 8q + 7) and multiplies with its dec rows times the
// columns' steps (A, lane 16q + n: row n of the tile, columns 8q ..; rows
// loaded a step ahead), 8 row tiles x 4 token tiles in fp32.  The group's RoPE table is made once for all heads.  Then each
// wave rotates its pairs (channels j, j + 64 in row tiles bb, bb + 4), stages
// 16 rows at a time in LDS and writes them coalesced, and dequantizes its
// head's 4 value pages.
//
// kLloyd (the Lloyd payload): a code is a level index, read through the
// levels in LDS; the B side holds v = level * the column's B factor (its step
// in a narrow slice, else 1).  The leading narrow steps (an even number) take
// fp16(v); every later step runs twice on one A operand, with B = fp16(v) and
// then B = fp16(v - fp16(v)), so that the pair of halves carries v to 2^-22:
// a single fp16 level of the wide tiers was the keys' largest error, as the
// product code * step was in the rtn payload (levels are no integers, so no
// exact fp16 form exists).
template <bool kLloyd>
__global__ __launch_bounds__(512) void spectral_dequant_kernel(const SpDequantKArgs a) {
  const int g = blockIdx.x;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, n = lane & 15, q = lane >> 4;
  const int h = wave;
  const bool head_ok = h < a.h_kv;
  __shared__ uint32_t s_tab[kSpMaxSlices];
  __shared__ __align__(16) _Float16 s_b[4][kGroup][kSpBRow];
  __shared__ __align__(16) float s_cs[2][kGroup][kCsPad];   // rows padded: conflict-free 16-byte reads
  // fp16 codebook levels of the 4 codes of one value-code byte (the P.V B operand)
  __shared__ uint2 s_cbl[256];
  __shared__ float s_lq[kLloyd ? kLqLevels : 1];   // the key payload's Lloyd levels
  __shared__ uint32_t s_lqp[kLloyd ? kLqPairs : 1];   // and their fp16 pair tables
  extern __shared__ __align__(16) uint8_t sp_dyn[];
  uint8_t* kp = sp_dyn;                                 // the key page, until the main loop ends
  DqTile* s_tile = reinterpret_cast<DqTile*>(sp_dyn);   // then the staging tiles
  const int n_sl = a.c_pad >> 3;
  const int hh = head_ok ? h : 0;   // waves past the heads load head 0's operands (unused)
  // ---- every global load of the prologue is issued first, the RoPE
  // frequency first of all: the table below waits for it alone (loads
  // complete in issue order), not for the page ----
  const int fj = tid & 63;
  const float fq = a.inv_freq[fj];   // every table entry of this thread has frequency fj
  __builtin_amdgcn_sched_barrier(0);
  const uint8_t* page = a.k_pages + clamp_page(a.k_table[g], a.n_k_pool) * (int64_t)a.k_page_bytes;
  // the key page's 16-byte chunks (threads past the last chunk re-read it: no
  // branch around the loads)
  const int n16 = a.k_page_bytes >> 4;
  u32x4_t kpw[kSpPageLoads];   // a native vector type: an array of uint4 stays in scratch
#pragma unroll
  for (int i = 0; i < kSpPageLoads; ++i)
    kpw[i] = reinterpret_cast<const u32x4_t*>(page)[min(tid + 512 * i, n16 - 1)];
  const uint32_t tabv = (uint32_t)a.slice_tab[min(tid, n_sl - 1)];   // n_sl <= 134 < 512
  float lqv = 0.f;
  uint32_t lqp0 = 0u, lqp1 = 0u;
  if constexpr (kLloyd) {
    lqv = a.lq[min(tid, kLqLevels - 1)];
    lqp0 = lq_pair_entry(a.lq, tid);
    lqp1 = lq_pair_entry(a.lq, min(tid + 512, kLqPairs - 1));
  }
  u32x2_t vcd[4], nrm[4];   // native vectors: an array of uint2 stays in scratch
#pragma unroll
  for (int pg = 0; pg < 4; ++pg) {
    const uint8_t* vp = a.v_pages + clamp_page(a.v_table[4 * g + pg], a.n_v_pool) * (int64_t)a.VL.bytes;
    vcd[pg] = *reinterpret_cast<const u32x2_t*>(vp + a.VL.vcode + hh * 512 + lane * 8);
    nrm[pg] = *reinterpret_cast<const u32x2_t*>(vp + a.VL.vnorm + ((a.v_full ? 0 : hh * kPT) + 4 * q) * 2);
  }
  // dec tiled: [h][c_pad32 / 32 steps][8 row tiles][16 rows][32 columns], a
  // contiguous KB per (step, row tile): lane 16q + n reads row n, columns 8q ..
  const uint16_t* decb = a.dec + (int64_t)hh * kD * a.c_pad32 + n * 32 + 8 * q;
  constexpr int tile_stride = 512, step_stride = 4096;
  half8_t An[8];
#pragma unroll
  for (int bt = 0; bt < 8; ++bt) An[bt] = *reinterpret_cast<const half8_t*>(decb + bt * tile_stride);
  if (tid < 256) {
    const float l0 = a.codebook[0], l1 = a.codebook[1], l2 = a.codebook[2], l3 = a.codebook[3];
    half4_t lv;
#pragma unroll
    for (int i = 0; i < 4; ++i) lv[i] = (_Float16)level4(((uint32_t)tid >> (2 * i)) & 3u, l0, l1, l2, l3);
    s_cbl[tid] = *reinterpret_cast<const uint2*>(&lv);
  }
  if (a.apply_rope) {
    // HF's fp32 angle fl(inv_freq_j * pos) of the group's 64 positions: this
    // thread has frequency fj at positions p0 + 8k (k < 8).  cos/sin of the exact
    // product fq * pos from one accurate start and a rotation by 8 fq per step,
    // then corrected to the fp32 angle: cos(ang) = cos(x - e) with the rounding
    // error e = fq * pos - fl(fq * pos) (exact by FMA)
    const int t0 = tid >> 6, p0 = g * kGroup + t0;
    float ss, cc, s8, c8;
    sincos_reduced(fq * (float)p0, &ss, &cc);   // fq * p0 rounded: corrected below like the rest
    {   // the exact product's: rotate forward by the rounding error e0
      const float a0 = fq * (float)p0, e0 = __builtin_fmaf(fq, (float)p0, -a0);
      float cx, sx;
      rotate_back(cc, ss, -e0, &cx, &sx);
      cc = cx;
      ss = sx;
    }
    sincos_reduced(8.0f * fq, &s8, &c8);   // 8 fq: exact in fp32
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int t = t0 + 8 * k;
      const float tf = (float)(p0 + 8 * k);
      const float ang = fq * tf;
      const float e = __builtin_fmaf(fq, tf, -ang);
      float cn, sn;
      rotate_back(cc, ss, e, &cn, &sn);
      cn *= a.rope_scaling;
      sn *= a.rope_scaling;
      if (a.apply_rope == 2) {
        cn = half_bits_to_float(float_to_half_bits(fp32_rounded(cn)));
        sn = half_bits_to_float(float_to_half_bits(fp32_rounded(sn)));
      }
      s_cs[0][t][fj] = cn;
      s_cs[1][t][fj] = sn;
      const float cnx = cc * c8 - ss * s8;
      ss = ss * c8 + cc * s8;
      cc = cnx;
    }
  }
  if (tid < n_sl) s_tab[tid] = tabv;
  if constexpr (kLloyd) {
    if (tid < kLqLevels) s_lq[tid] = lqv;
    s_lqp[tid] = lqp0;
    if (tid + 512 < kLqPairs) s_lqp[tid + 512] = lqp1;
  }
#pragma unroll
  for (int i = 0; i < kSpPageLoads; ++i)
    if (tid + 512 * i < n16) reinterpret_cast<u32x4_t*>(kp)[tid + 512 * i] = kpw[i];
  const int n_steps = a.c_pad32 / 32;
  // a barrier: s_tab, s_cbl, s_lq, the RoPE table, the key page
  const int n_narrow = sp_narrow_steps(tabv, tid, n_sl, n_steps);
  // Lloyd: steps 0 .. nn - 1 once each, the others as (fp16(v), remainder)
  // halves: virtual step u < nn is step u, else step nn + (u - nn) / 2, half
  // (u - nn) & 1; nn is even, so every barrier pair of the later steps holds
  // one step's two halves
  const int nn = kLloyd ? (n_narrow & ~1) : n_steps;

  // lane (sq, hf, t) of wave w decodes codes 4 hf .. 4 hf + 3 of slice 4 step + sq, token 8w + t
  // (a row of 16 lanes shares one slice, so that its code-word reads fall in
  // distinct banks: lanes on 4 slices 128 B apart hit the same banks)
  const int dsq = (lane >> 4) & 3, dhf = (lane >> 3) & 1, dt = 8 * wave + (lane & 7);
  auto decode_b = [&](int ks, int buf) {
    // no branch: slices past the last decode the last slice and store zeros
    const int s = 4 * ks + dsq, sc = min(s, n_sl - 1);
    const uint32_t tab = s_tab[sc];
    const int b = (int)(tab >> 24), off = (int)(tab & 0xFFFFFFu), w = sp_width(b);
    const int p = off + dt * w;
    const uint2 cw = *reinterpret_cast<const uint2*>(kp + (p & ~7));
    const uint4 f = sp_b_factor(kp, sc, b);
    const uint64_t word = ((((uint64_t)cw.y << 32) | cw.x) >> (8 * (p & 7))) >> (4 * dhf * w);
    const uint2 c = sp_codes4(word, w, b);
    const bool ok = s < n_sl;
    const uint32_t f0 = dhf ? f.z : f.x, f1 = dhf ? f.w : f.y;
    *reinterpret_cast<uint2*>(&s_b[buf][dt][8 * dsq + 4 * dhf]) =
        make_uint2(ok ? sp_hmul2(c.x, f0) : 0u, ok ? sp_hmul2(c.y, f1) : 0u);
  };
  // Lloyd: virtual step u's B tile (see nn above).  A step taken once holds
  // narrow slices only: fp16 level pairs from the pair tables times the fp16
  // steps (two roundings, against the exact product: within the bound of the
  // keys); a split step the fp32 level times the B factor, in two halves.
  auto decode_lq = [&](int u, int buf, auto split_t) {
    constexpr bool split = decltype(split_t)::value;   // u >= nn, known where it is called
    const int ks = split ? nn + ((u - nn) >> 1) : u;
    const bool rem = split && ((u - nn) & 1);
    const int s = 4 * ks + dsq, sc = min(s, n_sl - 1);
    const uint32_t tab = s_tab[sc];
    const int b = (int)(tab >> 24), off = (int)(tab & 0xFFFFFFu), w = sp_width(b);
    const int p = off + dt * w;
    const uint2 cw = *reinterpret_cast<const uint2*>(kp + (p & ~7));
    const uint4 f = sp_b_factor(kp, sc, b);
    const uint64_t word = ((((uint64_t)cw.y << 32) | cw.x) >> (8 * (p & 7))) >> (4 * dhf * w);
    const uint32_t f0 = dhf ? f.z : f.x, f1 = dhf ? f.w : f.y;
    // every load unconditional and the result masked: a select of an LDS
    // load becomes a branch around it, which splits the loop's basic block
    const uint32_t okm = s < n_sl ? 0xFFFFFFFFu : 0u;
    uint2 o;
    if constexpr (!split) {
      const int base = lq_pair_base(b);
      const uint32_t km = ((1u << (2 * w)) - 1u) & 0xFFu;   // narrow: w <= 4
      o.x = sp_hmul2(s_lqp[base + ((uint32_t)word & km)], f0) & okm;
      o.y = sp_hmul2(s_lqp[base + ((uint32_t)(word >> (2 * w)) & km)], f1) & okm;
    } else {
      const half2_t f01 = as_h2(f0), f23 = as_h2(f1);
      const float fe[4] = {(float)f01[0], (float)f01[1], (float)f23[0], (float)f23[1]};
      const float* lv = s_lq + lq_off(b);
      const uint32_t mask = (1u << w) - 1u;
      _Float16 h[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float v = lv[(uint32_t)(word >> (e * w)) & mask] * fe[e];
        const _Float16 hv = (_Float16)v;
        h[e] = rem ? (_Float16)(v - (float)hv) : hv;
      }
      o = make_uint2(as_u32(half2_t{h[0], h[1]}) & okm, as_u32(half2_t{h[2], h[3]}) & okm);
    }
    *reinterpret_cast<uint2*>(&s_b[buf][dt][8 * dsq + 4 * dhf]) = o;
  };
  // decode(u, buf, split): split tells a Lloyd decode that u >= nn
  auto decode = [&](int u, int buf, auto split_t) {
    if constexpr (kLloyd) decode_lq(u, buf, split_t);
    else decode_b(u, buf);
  };

  float4_t acc[8][4];
#pragma unroll
  for (int bt = 0; bt < 8; ++bt)
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) acc[bt][tt] = (float4_t){0.f, 0.f, 0.f, 0.f};
  // Two steps per workgroup barrier: buffers 2p and 2p + 1 hold steps ks and
  // ks + 1 while the next two are decoded into the other pair; each step's
  // MFMAs are interleaved with the next pair's decode (VALU and LDS reads).
  if (nn >= 2) {
    decode(0, 0, std::false_type{});
    decode(1, 1, std::false_type{});
  } else {
    decode(0, 0, std::true_type{});
    decode(1, 1, std::true_type{});
  }
  __syncthreads();
  half8_t A[8];
  // A = the dec rows, times the group's steps of the lane's 8 columns in a
  // step with wider tiers; then the next step's rows are loaded
  auto a_operand = [&](int ks, auto wide) {
    if constexpr (decltype(wide)::value) {
      const half8_t f = sp_a_factor(kp, s_tab, 4 * ks + q, n_sl);
#pragma unroll
      for (int bt = 0; bt < 8; ++bt) A[bt] = An[bt] * f;
    } else {
#pragma unroll
      for (int bt = 0; bt < 8; ++bt) A[bt] = An[bt];
    }
    const int kn = min(ks + 1, n_steps - 1);   // the last step re-reads its own rows: no branch
#pragma unroll
    for (int bt = 0; bt < 8; ++bt)
      An[bt] = *reinterpret_cast<const half8_t*>(decb + bt * tile_stride + step_stride * kn);
  };
  auto mfma_b = [&](int buf) {
    half8_t B[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) B[tt] = *reinterpret_cast<const half8_t*>(&s_b[buf][16 * tt + n][8 * q]);
#pragma unroll
    for (int bt = 0; bt < 8; ++bt)
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
        acc[bt][tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[bt], B[tt], acc[bt][tt], 0, 0, 0);
  };
  auto mfma_step = [&](int ks, int buf, auto wide) {
    a_operand(ks, wide);
    mfma_b(buf);
  };
  // whole pairs of steps in one basic block each (decodes past the last step
  // store zeros into buffers nobody reads), then an odd last step; the
  // compiler's own interleave measured faster than a fixed MFMA/VALU/LDS
  // pattern
  const int n_pairs = n_steps >> 1, n_narrow_pairs = n_narrow >> 1;
  auto pair = [&](int kq, auto wide, auto split_t) {
    const int ks = 2 * kq, pb = kq & 1;
    if (head_ok) {
      mfma_step(ks, 2 * pb, wide);
      decode(ks + 2, 2 * (pb ^ 1), split_t);
      mfma_step(ks + 1, 2 * pb + 1, wide);
      decode(ks + 3, 2 * (pb ^ 1) + 1, split_t);
    } else {
      decode(ks + 2, 2 * (pb ^ 1), split_t);
      decode(ks + 3, 2 * (pb ^ 1) + 1, split_t);
    }
    lds_barrier();   // the next pair decoded, this pair read by every wave
  };
  int kq = 0;
  if constexpr (kLloyd) {
    // the narrow pairs (the last of them decodes the first split step), then
    // one step per pair: its two halves on one A operand
    for (; kq + 1 < (nn >> 1); ++kq) pair(kq, std::false_type{}, std::false_type{});
    if (kq < (nn >> 1)) pair(kq++, std::false_type{}, std::true_type{});
    for (; kq < (nn >> 1) + n_steps - nn; ++kq) {
      const int u = 2 * kq, pb = kq & 1;
      if (head_ok) {
        a_operand(nn + kq - (nn >> 1), std::true_type{});
        mfma_b(2 * pb);
        decode(u + 2, 2 * (pb ^ 1), std::true_type{});
        mfma_b(2 * pb + 1);
        decode(u + 3, 2 * (pb ^ 1) + 1, std::true_type{});
      } else {
        decode(u + 2, 2 * (pb ^ 1), std::true_type{});
        decode(u + 3, 2 * (pb ^ 1) + 1, std::true_type{});
      }
      lds_barrier();
    }
  } else {
    for (; kq < n_narrow_pairs; ++kq) pair(kq, std::false_type{}, std::false_type{});
    for (; kq < n_pairs; ++kq) pair(kq, std::true_type{}, std::false_type{});
    if ((n_steps & 1) && head_ok) mfma_step(n_steps - 1, 2 * (n_pairs & 1), std::true_type{});
    // the last step's A factors read the key page, whose space takes the
    // staging tiles below
    if (n_steps & 1) __syncthreads();
  }

  // query fragments (decode form), loaded after the main loop: the MFMA B operand of the scores, lane
  // 16q + n: query n, K index 8q + 2i + e = channel 16bb + 4q + i + 64e
  half8_t qf[4];
  const bool scoring = a.q != nullptr;
  if (scoring && head_ok) {
    // the lane's 8 runs of 4 channels (16bb + 4q .. + 3, and + 64), all loads issued first
    float qv[8][4];
    const int64_t qrow = ((int64_t)h * a.n_q_groups + (n < a.n_q_groups ? n : 0)) * kD + 4 * q;
    if (a.q_dtype == BMX_K2B_F32) {
      float4_t r[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        r[u] = *reinterpret_cast<const float4_t*>(static_cast<const float*>(a.q) + qrow + 16 * (u & 3) + 64 * (u >> 2));
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i) qv[u][i] = r[u][i];
    } else {
      uint2 r[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        r[u] = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(a.q) + qrow + 16 * (u & 3) + 64 * (u >> 2));
      const bool bf = a.q_dtype == BMX_K2B_BF16;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const uint32_t w[4] = {r[u].x & 0xffffu, r[u].x >> 16, r[u].y & 0xffffu, r[u].y >> 16};
#pragma unroll
        for (int i = 0; i < 4; ++i) qv[u][i] = bf ? __uint_as_float(w[i] << 16) : half_bits_to_float(w[i]);
      }
    }
    const bool qok = n < a.n_q_groups;
#pragma unroll
    for (int bb = 0; bb < 4; ++bb)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 2; ++e) qf[bb][2 * i + e] = (_Float16)(qok ? qv[bb + 4 * e][i] : 0.f);
  }
  // keys: RoPE of the lane's pairs, channel j = 16bb + 4q + i and j + 64, token
  // 16tt + n; 16 rows staged per token tile.  Each wave stages through its own
  // tile only: no workgroup barrier from here on (a wave's LDS accesses take
  // effect in program order; wave_lds_order keeps the compiler from moving
  // them and waits for them)
  DqTile& tl = s_tile[wave];
  const int64_t row_h = (int64_t)(head_ok ? h : 0) * a.out_rows + g * kGroup;
  float4_t sct[4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    if (head_ok) {
      float4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int bb = 0; bb < 4; ++bb) {
        half8_t ka;
        const float4_t c4 = *reinterpret_cast<const float4_t*>(&s_cs[0][16 * tt + n][16 * bb + 4 * q]);
        const float4_t s4 = *reinterpret_cast<const float4_t*>(&s_cs[1][16 * tt + n][16 * bb + 4 * q]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = 16 * bb + 4 * q + i;
          float k0 = acc[bb][tt][i], k1 = acc[bb + 4][tt][i];
          if (a.apply_rope) {
            const float cn = c4[i], sn = s4[i];
            const float r0 = __fmul_rn(k0, cn) - __fmul_rn(k1, sn);
            k1 = __fmul_rn(k1, cn) + __fmul_rn(k0, sn);
            k0 = r0;
          }
          if (a.k_out) {
            tl.v[n][j] = k0;
            tl.v[n][j + 64] = k1;
          }
          ka[2 * i] = (_Float16)k0;
          ka[2 * i + 1] = (_Float16)k1;
        }
        // scores: A = the tile's rotated keys (token n, K index 8q + 2i + e)
        if (scoring) sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qf[bb], sc, 0, 0, 0);
      }
      sct[tt] = sc;
      if (scoring && !a.partials && n < a.n_q_groups) {   // lane 16q + n: tokens 4q .. 4q + 3, query n
        float* dst = a.scores + ((int64_t)h * a.n_q_groups + n) * a.out_rows + g * kGroup + 16 * tt + 4 * q;
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[i] = sc[i];
      }
      if (a.k_out) {
        wave_lds_order();
        dq_store_tile(tl, a.k_out, row_h + 16 * tt, a.out_dtype);
        wave_lds_order();
      }
    }
  }
  if (a.partials) {   // partial form: the group's softmax partial per query, no dense values
    if (head_ok) {
      // lane 16q + n holds query n's scores of tokens 16tt + 4q + i
      float m = -INFINITY;
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) m = fmaxf(m, sct[tt][i] * a.sm_scale);
      m = fmaxf(m, __shfl_xor(m, 16));
      m = fmaxf(m, __shfl_xor(m, 32));
      const bool qok = n < a.n_q_groups;
      half4_t pw[4];
      float l = 0.f;
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const _Float16 p = qok ? (_Float16)__expf(sct[tt][i] * a.sm_scale - m) : (_Float16)0.f;
          pw[tt][i] = p;
          l += (float)p;
        }
      l += __shfl_xor(l, 16);
      l += __shfl_xor(l, 32);
      // P.V in the rotated value domain, per value page (= token tile): A = the
      // weights times the token norms (query n, tokens 4q .. 4q + 3), B = the
      // codebook levels of rotated channel 16ct + n, tokens 4q .. 4q + 3: byte
      // ct of the lane's own code pair.  The inverse Hadamard, the signs and
      // 1/128 are linear and left to the merge.
      float4_t pv[8];
#pragma unroll
      for (int ct = 0; ct < 8; ++ct) pv[ct] = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int pg = 0; pg < 4; ++pg) {
        const float nv[4] = {half_bits_to_float(nrm[pg].x & 0xffffu), half_bits_to_float(nrm[pg].x >> 16),
                             half_bits_to_float(nrm[pg].y & 0xffffu), half_bits_to_float(nrm[pg].y >> 16)};
        half4_t aw;
#pragma unroll
        for (int i = 0; i < 4; ++i) aw[i] = (_Float16)((float)pw[pg][i] * nv[i]);
        if (a.v_full) {
          // every slice's codes, A = the weights times H_{C/128}[h][slice]
          const uint8_t* vp = a.v_pages + clamp_page(a.v_table[4 * g + pg], a.n_v_pool) * (int64_t)a.VL.bytes;
          u32x2_t cs[8];
#pragma unroll
          for (int sl = 0; sl < 8; ++sl)
            cs[sl] = *reinterpret_cast<const u32x2_t*>(vp + a.VL.vcode + min(sl, a.h_kv - 1) * 512 + lane * 8);
          // two slices per 32-deep MFMA (K index 8q + i: tokens 4q + i of
          // slice 2sp for i < 4, of slice 2sp + 1 after)
#pragma unroll
          for (int sp = 0; sp < 4; ++sp) {
            if (2 * sp >= a.h_kv) break;
            const half4_t z4 = {(_Float16)0.f, (_Float16)0.f, (_Float16)0.f, (_Float16)0.f};
            const half4_t a0 = vfull_neg(h, 2 * sp) ? -aw : aw;
            const half4_t a1 = 2 * sp + 1 < a.h_kv ? (vfull_neg(h, 2 * sp + 1) ? -aw : aw) : z4;
            const half8_t A8 = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
            const u32x2_t c0 = cs[2 * sp], c1 = cs[2 * sp + 1];
#pragma unroll
            for (int ct = 0; ct < 8; ++ct) {
              const uint2 l0 = s_cbl[((ct < 4 ? c0.x : c0.y) >> (8 * (ct & 3))) & 0xFFu];
              const uint2 l1 = s_cbl[((ct < 4 ? c1.x : c1.y) >> (8 * (ct & 3))) & 0xFFu];
              const half8_t B8 = __builtin_bit_cast(half8_t, make_uint4(l0.x, l0.y, l1.x, l1.y));
              pv[ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A8, B8, pv[ct], 0, 0, 0);
            }
          }
        } else {
#pragma unroll
          for (int ct = 0; ct < 8; ++ct) {
            const uint32_t byte = ((ct < 4 ? vcd[pg].x : vcd[pg].y) >> (8 * (ct & 3))) & 0xFFu;
            const uint2 lvb = s_cbl[byte];
            const half4_t vb = *reinterpret_cast<const half4_t*>(&lvb);
            pv[ct] = __builtin_amdgcn_mfma_f32_16x16x16f16(aw, vb, pv[ct], 0, 0, 0);
          }
        }
      }
      // lane 16q + n holds queries 4q + i, channel 16ct + n: H8 over ct in
      // registers (the merge applies H16 over n to its chunk's merged sums)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int sb = 1; sb < 8; sb <<= 1)
#pragma unroll
          for (int ct = 0; ct < 8; ++ct)
            if (!(ct & sb)) {
              const float u = pv[ct][i], w = pv[ct | sb][i];
              pv[ct][i] = u + w;
              pv[ct | sb][i] = u - w;
            }
      const int n_grp = a.n_tokens / kGroup;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int qi = 4 * q + i;
        if (qi < a.n_q_groups) {
          const int64_t r = (int64_t)h * a.n_q_groups + qi;
#pragma unroll
          for (int ct = 0; ct < 8; ++ct) sp_part_ch(a.partials, r, n_grp, ct, g)[n] = pv[ct][i];
        }
      }
      if (q == 0 && qok) {
        float* dst = sp_part_ml(a.partials, (int64_t)h * a.n_q_groups + n, n_grp, g);
        dst[0] = m;
        dst[1] = l;
      }
    }
    return;
  }
  // values: the head's 4 pages of the group
  if (head_ok) {
#pragma unroll
    for (int pg = 0; pg < 4; ++pg) {
      if (a.v_full) {
        const uint8_t* vp = a.v_pages + clamp_page(a.v_table[4 * g + pg], a.n_v_pool) * (int64_t)a.VL.bytes;
        float y[4][8];
        vfull_y(vp, a.VL.vcode, a.h_kv, h, lane, a.codebook, y);
        dq_value_tile_rot(y, make_uint2(nrm[pg].x, nrm[pg].y), a.v_sign_c + 4 * h, 1.0f / (float)(kD * a.h_kv), n,
                          q, tl, a.out_dtype);
      } else {
        dq_value_tile(make_uint2(vcd[pg].x, vcd[pg].y), make_uint2(nrm[pg].x, nrm[pg].y), a.codebook,
                      a.v_sign_bits, n, q, tl, a.out_dtype);
      }
      wave_lds_order();
      dq_store_tile(tl, a.v_out, row_h + 16 * pg, a.out_dtype);
      wave_lds_order();
    }
  }
}

// Partial form over 128-token blocks (two key pages), four heads per
// workgroup: grid (n_tokens / 128, ceil(h_kv / 4)), block 512.  Wave w serves
// head 4 blockIdx.y + (w >> 1) and half r = w & 1 of its rows: row tiles 2r,
// 2r + 1 and their RoPE partners 2r + 4, 2r + 5 (channels 32r .. 32r + 31 and
// + 64), times the block's 8 token tiles.  Against the 64-token form, each
// dec row read from L2 feeds twice the MFMAs (the main loop's second cost
// after the MFMAs); the block's code tile is decoded once for 4 heads
// instead of 8.  Each token tile takes the A operand of its page (the dec
// rows times that page's steps).  The two halves of a head add their partial
// scores through LDS, then each takes 4 of the head's 8 rotated value-channel
// blocks.  The
// RoPE table is the fp16-rounded one (apply_rope 2), kept as fp16 pairs.
// kLloyd: the Lloyd payload, decoded as in spectral_dequant_kernel<true>.
// kVFull: full-C values; the P.V runs over every slice's codes (read from
// the value pages after the main loop: staged in LDS they would not fit
// beside the key pages), the block's 4 heads sharing the MFMA rows, each
// row's weights signed by H_{C/128}[h][slice].
constexpr int kSpBlk = 128;
constexpr int kSpVfAwOff = 8 * 4 * 64 * 16;   // full-C: the weight table's offset in the dynamic LDS
constexpr int kSpBlkMaxPages = 56 * 1024;   // two key pages staged in LDS at most

template <bool kLloyd, bool kVFull>
__global__ __launch_bounds__(512) void spectral_partial128_kernel(const SpDequantKArgs a, int kpb) {
  const int blk = blockIdx.x, hq = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, n = lane & 15, q = lane >> 4;
  const int hl = wave >> 1, r2 = wave & 1;
  const int h = 4 * hq + hl;
  const bool head_ok = h < a.h_kv;
  const int hh = head_ok ? h : 0;
  __shared__ uint32_t s_tab[kSpMaxSlices];
  __shared__ __align__(16) _Float16 s_b[4][kSpBlk][kSpBRow];
  __shared__ __align__(16) uint32_t s_cs[kSpBlk][kCsPad];   // (cos, sin) fp16 of (position, frequency)
  __shared__ uint2 s_cbl[256];
  __shared__ uint2 s_vcd[kVFull ? 1 : 4][8][64];   // (local head, value page, lane)
  __shared__ uint2 s_nrm[kVFull ? 1 : 4][8][4];    // (local head, value page, quarter)
  __shared__ float s_lq[kLloyd ? kLqLevels : 1];   // the key payload's Lloyd levels
  __shared__ uint32_t s_lqp[kLloyd ? kLqPairs : 1];   // and their fp16 pair tables
  extern __shared__ __align__(16) uint8_t sp_dyn[];   // the two key pages; after the loop, the score exchange
  const int n_sl = a.c_pad >> 3;
  const int fj = tid & 63;
  const float fq = a.inv_freq[fj];
  __builtin_amdgcn_sched_barrier(0);
  // ---- every global load first: the two key pages (kpb bytes apart in LDS),
  // the slice table, the value codes and norms of the 8 value pages, dec rows
  const int n16 = kpb >> 4;            // 16-byte chunks per page in LDS
  const int p16 = a.k_page_bytes >> 4; // 16-byte chunks per page read
  const uint8_t* pg0 = a.k_pages + clamp_page(a.k_table[2 * blk], a.n_k_pool) * (int64_t)a.k_page_bytes;
  const uint8_t* pg1 = a.k_pages + clamp_page(a.k_table[2 * blk + 1], a.n_k_pool) * (int64_t)a.k_page_bytes;
  constexpr int kLoads = (kSpBlkMaxPages / 2 + 16 * 512 - 1) / (16 * 512);   // per page per thread
  u32x4_t kw0[kLoads], kw1[kLoads];   // a native vector type: an array of uint4 stays in scratch
#pragma unroll
  for (int i = 0; i < kLoads; ++i) {
    const int c = min(tid + 512 * i, p16 - 1);
    kw0[i] = reinterpret_cast<const u32x4_t*>(pg0)[c];
    kw1[i] = reinterpret_cast<const u32x4_t*>(pg1)[c];
  }
  const uint32_t tabv = (uint32_t)a.slice_tab[min(tid, n_sl - 1)];
  float lqv = 0.f;
  uint32_t lqp0 = 0u, lqp1 = 0u;
  if constexpr (kLloyd) {
    lqv = a.lq[min(tid, kLqLevels - 1)];
    lqp0 = lq_pair_entry(a.lq, tid);
    lqp1 = lq_pair_entry(a.lq, min(tid + 512, kLqPairs - 1));
  }
  // value pages: thread (local head tid >> 7, page (tid >> 6) & 1 + 2 k, lane)
  uint2 vcw[4], nrw[4];
  const int vh = min(4 * hq + (tid >> 7), a.h_kv - 1), vl = tid & 63;
  if constexpr (kVFull) {
    {   // norms: thread tid < 32 takes page tid >> 2, tokens 4 (tid & 3) ..
      const int vp_i = (tid >> 2) & 7;
      const uint8_t* vp = a.v_pages + clamp_page(a.v_table[8 * blk + vp_i], a.n_v_pool) * (int64_t)a.VL.bytes;
      nrw[0] = *reinterpret_cast<const uint2*>(vp + a.VL.vnorm + 4 * (tid & 3) * 2);
    }
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int vp_i = ((tid >> 6) & 1) + 2 * k;
      const uint8_t* vp = a.v_pages + clamp_page(a.v_table[8 * blk + vp_i], a.n_v_pool) * (int64_t)a.VL.bytes;
      vcw[k] = *reinterpret_cast<const uint2*>(vp + a.VL.vcode + vh * 512 + vl * 8);
      nrw[k] = *reinterpret_cast<const uint2*>(vp + a.VL.vnorm + (vh * kPT + 4 * (vl >> 4)) * 2);
    }
  }
  // dec rows of this wave's 4 row tiles: rt(i) = 2 r2 + (i & 1) + 4 (i >> 1)
  const uint16_t* decb = a.dec + (int64_t)hh * kD * a.c_pad32 + n * 32 + 8 * q;
  constexpr int tile_stride = 512, step_stride = 4096;
  auto rt = [&](int i) { return 2 * r2 + (i & 1) + 4 * (i >> 1); };
  half8_t An[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) An[i] = *reinterpret_cast<const half8_t*>(decb + rt(i) * tile_stride);
  if (tid < 256) {
    const float l0 = a.codebook[0], l1 = a.codebook[1], l2 = a.codebook[2], l3 = a.codebook[3];
    half4_t lv;
#pragma unroll
    for (int i = 0; i < 4; ++i) lv[i] = (_Float16)level4(((uint32_t)tid >> (2 * i)) & 3u, l0, l1, l2, l3);
    s_cbl[tid] = *reinterpret_cast<const uint2*>(&lv);
  }
  {   // RoPE table, fp16 (cos, sin): frequency fj at positions p0 + 8k, k < 16
    const int t0 = tid >> 6, p0 = blk * kSpBlk + t0;
    float ss, cc, s8, c8;
    sincos_reduced(fq * (float)p0, &ss, &cc);
    {
      const float a0 = fq * (float)p0, e0 = __builtin_fmaf(fq, (float)p0, -a0);
      float cx, sx;
      rotate_back(cc, ss, -e0, &cx, &sx);
      cc = cx;
      ss = sx;
    }
    sincos_reduced(8.0f * fq, &s8, &c8);
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int t = t0 + 8 * k;
      const float tf = (float)(p0 + 8 * k);
      const float ang = fq * tf;
      const float e = __builtin_fmaf(fq, tf, -ang);
      float cn, sn;
      rotate_back(cc, ss, e, &cn, &sn);
      const half2_t cs = {(_Float16)fp32_rounded(cn * a.rope_scaling), (_Float16)fp32_rounded(sn * a.rope_scaling)};
      s_cs[t][fj] = as_u32(cs);
      const float cnx = cc * c8 - ss * s8;
      ss = ss * c8 + cc * s8;
      cc = cnx;
    }
  }
  if (tid < n_sl) s_tab[tid] = tabv;
  if constexpr (kLloyd) {
    if (tid < kLqLevels) s_lq[tid] = lqv;
    s_lqp[tid] = lqp0;
    if (tid + 512 < kLqPairs) s_lqp[tid + 512] = lqp1;
  }
  uint8_t* kp0 = sp_dyn;
  uint8_t* kp1 = sp_dyn + kpb;
#pragma unroll
  for (int i = 0; i < kLoads; ++i)
    if (tid + 512 * i < n16) {
      reinterpret_cast<u32x4_t*>(kp0)[tid + 512 * i] = kw0[i];
      reinterpret_cast<u32x4_t*>(kp1)[tid + 512 * i] = kw1[i];
    }
  if constexpr (kVFull) {
    if (tid < 32) s_nrm[0][tid >> 2][tid & 3] = nrw[0];
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int vp_i = ((tid >> 6) & 1) + 2 * k;
      s_vcd[tid >> 7][vp_i][vl] = vcw[k];
      if ((vl & 15) == 0) s_nrm[tid >> 7][vp_i][vl >> 4] = nrw[k];
    }
  }
  const int n_steps = a.c_pad32 / 32;
  // a barrier: s_tab, s_cbl, s_cs, s_lq, the key pages, the value codes
  const int n_narrow = sp_narrow_steps(tabv, tid, n_sl, n_steps);
  // Lloyd: virtual steps as in spectral_dequant_kernel<true>
  const int nn = kLloyd ? (n_narrow & ~1) : n_steps;

  // lane (sq, t) of wave w decodes the 8 codes of slice 4 step + sq, token 16w + t
  // (a row of 16 lanes shares one slice, so that its code-word reads fall in
  // distinct banks: lanes on 4 slices 128 B apart hit the same banks)
  const int dsq = (lane >> 4) & 3, dt = 16 * wave + (lane & 15);
  const uint8_t* kpt = dt < kGroup ? kp0 : kp1;
  const int dtp = dt & (kGroup - 1);
  auto decode_b = [&](int ks, int buf) {
    // no branch: slices past the last (the padding of the last step, or a
    // step past the last) decode the last slice and store zeros
    const int s = 4 * ks + dsq, sc = min(s, n_sl - 1);
    const uint32_t tab = s_tab[sc];
    const int b = (int)(tab >> 24), off = (int)(tab & 0xFFFFFFu), w = sp_width(b);
    const int pp = off + dtp * w;
    const uint2 cw = *reinterpret_cast<const uint2*>(kpt + (pp & ~7));
    const uint4 f = sp_b_factor(kpt, sc, b);
    const uint64_t word = (((uint64_t)cw.y << 32) | cw.x) >> (8 * (pp & 7));
    const uint2 lo = sp_codes4(word, w, b), hi = sp_codes4(word >> (4 * w), w, b);
    const bool ok = s < n_sl;
    const uint4 v = make_uint4(ok ? sp_hmul2(lo.x, f.x) : 0u, ok ? sp_hmul2(lo.y, f.y) : 0u,
                               ok ? sp_hmul2(hi.x, f.z) : 0u, ok ? sp_hmul2(hi.y, f.w) : 0u);
    *reinterpret_cast<uint4*>(&s_b[buf][dt][8 * dsq]) = v;
  };
  auto decode_lq = [&](int u, int buf, auto split_t) {
    constexpr bool split = decltype(split_t)::value;   // u >= nn, known where it is called
    const int ks = split ? nn + ((u - nn) >> 1) : u;
    const bool rem = split && ((u - nn) & 1);
    const int s = 4 * ks + dsq, sc = min(s, n_sl - 1);
    const uint32_t tab = s_tab[sc];
    const int b = (int)(tab >> 24), off = (int)(tab & 0xFFFFFFu), w = sp_width(b);
    const int pp = off + dtp * w;
    const uint2 cw = *reinterpret_cast<const uint2*>(kpt + (pp & ~7));
    const uint4 f = sp_b_factor(kpt, sc, b);
    const uint64_t word = (((uint64_t)cw.y << 32) | cw.x) >> (8 * (pp & 7));
    const uint32_t fw[4] = {f.x, f.y, f.z, f.w};
    const uint32_t okm = s < n_sl ? 0xFFFFFFFFu : 0u;   // loads unconditional, results masked
    uint32_t o[4];
    if constexpr (!split) {
      const int base = lq_pair_base(b);
      const uint32_t km = ((1u << (2 * w)) - 1u) & 0xFFu;   // narrow: w <= 4
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2)
        o[e2] = sp_hmul2(s_lqp[base + ((uint32_t)(word >> (2 * e2 * w)) & km)], fw[e2]) & okm;
    } else {
      const float* lv = s_lq + lq_off(b);
      const uint32_t mask = (1u << w) - 1u;
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        const half2_t fe = as_h2(fw[e2]);
        half2_t r;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const float v = lv[(uint32_t)(word >> ((2 * e2 + i) * w)) & mask] * (float)fe[i];
          const _Float16 h16 = (_Float16)v;
          r[i] = rem ? (_Float16)(v - (float)h16) : h16;
        }
        o[e2] = as_u32(r) & okm;
      }
    }
    *reinterpret_cast<uint4*>(&s_b[buf][dt][8 * dsq]) = make_uint4(o[0], o[1], o[2], o[3]);
  };
  // decode(u, buf, split): split tells a Lloyd decode that u >= nn
  auto decode = [&](int u, int buf, auto split_t) {
    if constexpr (kLloyd) decode_lq(u, buf, split_t);
    else decode_b(u, buf);
  };

  float4_t acc[4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int tt = 0; tt < 8; ++tt) acc[i][tt] = (float4_t){0.f, 0.f, 0.f, 0.f};
  if (nn >= 2) {
    decode(0, 0, std::false_type{});
    decode(1, 1, std::false_type{});
  } else {
    decode(0, 0, std::true_type{});
    decode(1, 1, std::true_type{});
  }
  __syncthreads();
  half8_t A[2][4];
  // A = the dec rows, times each page's steps of the lane's 8 columns in a
  // step with wider tiers; then the next step's rows are loaded
  auto a_operand = [&](int ks, auto wide) {
    if constexpr (decltype(wide)::value) {
      const half8_t f0 = sp_a_factor(kp0, s_tab, 4 * ks + q, n_sl), f1 = sp_a_factor(kp1, s_tab, 4 * ks + q, n_sl);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        A[0][i] = An[i] * f0;
        A[1][i] = An[i] * f1;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) A[0][i] = A[1][i] = An[i];
    }
    const int kn = min(ks + 1, n_steps - 1);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      An[i] = *reinterpret_cast<const half8_t*>(decb + rt(i) * tile_stride + step_stride * kn);
  };
  auto mfma_b = [&](int buf) {
    half8_t B[8];
#pragma unroll
    for (int tt = 0; tt < 8; ++tt) B[tt] = *reinterpret_cast<const half8_t*>(&s_b[buf][16 * tt + n][8 * q]);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int tt = 0; tt < 8; ++tt)
        acc[i][tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[tt >> 2][i], B[tt], acc[i][tt], 0, 0, 0);
  };
  auto mfma_step = [&](int ks, int buf, auto wide) {
    a_operand(ks, wide);
    mfma_b(buf);
  };
  // whole pairs of steps in one basic block each (decodes past the last step
  // store zeros into buffers nobody reads), then an odd last step; the
  // compiler's own interleave of the MFMAs, the decode and the dec loads
  // measured faster here than a fixed MFMA/VALU/LDS pattern
  const int n_pairs = n_steps >> 1, n_narrow_pairs = n_narrow >> 1;
  auto pair = [&](int kp, auto wide, auto split_t) {
    const int ks = 2 * kp, pb = kp & 1;
    mfma_step(ks, 2 * pb, wide);
    decode(ks + 2, 2 * (pb ^ 1), split_t);
    mfma_step(ks + 1, 2 * pb + 1, wide);
    decode(ks + 3, 2 * (pb ^ 1) + 1, split_t);
    lds_barrier();
  };
  int kp = 0;
  if constexpr (kLloyd) {
    // the narrow pairs (the last of them decodes the first split step), then
    // one step per pair: its two halves on one A operand
    for (; kp + 1 < (nn >> 1); ++kp) pair(kp, std::false_type{}, std::false_type{});
    if (kp < (nn >> 1)) pair(kp++, std::false_type{}, std::true_type{});
    for (; kp < (nn >> 1) + n_steps - nn; ++kp) {
      const int u = 2 * kp, pb = kp & 1;
      a_operand(nn + kp - (nn >> 1), std::true_type{});
      mfma_b(2 * pb);
      decode(u + 2, 2 * (pb ^ 1), std::true_type{});
      mfma_b(2 * pb + 1);
      decode(u + 3, 2 * (pb ^ 1) + 1, std::true_type{});
      lds_barrier();
    }
  } else {
    for (; kp < n_narrow_pairs; ++kp) pair(kp, std::false_type{}, std::false_type{});
    for (; kp < n_pairs; ++kp) pair(kp, std::true_type{}, std::false_type{});
    if (n_steps & 1) mfma_step(n_steps - 1, 2 * (n_pairs & 1), std::true_type{});
  }

  // ---- query fragments of this wave's channels: bb = 2 r2 + bl ----
  half8_t qf[2];
  {
    float qv[4][4];   // runs (bl, e): channels 16 bb + 4q .. + 3 + 64 e
    const int64_t qrow = ((int64_t)hh * a.n_q_groups + (n < a.n_q_groups ? n : 0)) * kD + 4 * q;
    if (a.q_dtype == BMX_K2B_F32) {
      float4_t r[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        r[u] = *reinterpret_cast<const float4_t*>(static_cast<const float*>(a.q) + qrow + 16 * (2 * r2 + (u & 1)) +
                                                  64 * (u >> 1));
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i) qv[u][i] = r[u][i];
    } else {
      uint2 r[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        r[u] = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(a.q) + qrow + 16 * (2 * r2 + (u & 1)) +
                                               64 * (u >> 1));
      const bool bf = a.q_dtype == BMX_K2B_BF16;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t w[4] = {r[u].x & 0xffffu, r[u].x >> 16, r[u].y & 0xffffu, r[u].y >> 16};
#pragma unroll
        for (int i = 0; i < 4; ++i) qv[u][i] = bf ? __uint_as_float(w[i] << 16) : half_bits_to_float(w[i]);
      }
    }
    const bool qok = n < a.n_q_groups;
#pragma unroll
    for (int bl = 0; bl < 2; ++bl)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 2; ++e) qf[bl][2 * i + e] = (_Float16)(qok ? qv[bl + 2 * e][i] : 0.f);
  }
  // ---- the wave's partial scores: RoPE of its pairs, fp16 keys, MFMA ----
  float4_t sct[8];
#pragma unroll
  for (int tt = 0; tt < 8; ++tt) {
    float4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int bl = 0; bl < 2; ++bl) {
      const int bb = 2 * r2 + bl;
      const uint4 cs4 = *reinterpret_cast<const uint4*>(&s_cs[16 * tt + n][16 * bb + 4 * q]);
      const uint32_t csw[4] = {cs4.x, cs4.y, cs4.z, cs4.w};
      half8_t ka;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const half2_t cs = as_h2(csw[i]);
        const float cn = (float)cs[0], sn = (float)cs[1];
        const float k0 = acc[bl][tt][i], k1 = acc[bl + 2][tt][i];
        const float r0 = __fmul_rn(k0, cn) - __fmul_rn(k1, sn);
        const float r1 = __fmul_rn(k1, cn) + __fmul_rn(k0, sn);
        ka[2 * i] = (_Float16)r0;
        ka[2 * i + 1] = (_Float16)r1;
      }
      sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qf[bl], sc, 0, 0, 0);
    }
    sct[tt] = sc;
  }
  // full-C values: the block's value codes (8 pages x h_kv slices x 512 B),
  // loaded now in 16-byte chunks and staged in the RoPE table's space once
  // the scores have read it
  u32x4_t vfc[4];
  const int vf_chunks = 32 * a.h_kv;   // 16-byte chunks of one page's VCODE
  if constexpr (kVFull) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = min(tid + 512 * i, 8 * vf_chunks - 1), pgi = c / vf_chunks;
      const uint8_t* vp = a.v_pages + clamp_page(a.v_table[8 * blk + pgi], a.n_v_pool) * (int64_t)a.VL.bytes;
      vfc[i] = *reinterpret_cast<const u32x4_t*>(vp + a.VL.vcode + (c - pgi * vf_chunks) * 16);
    }
  }
  // ---- the two halves of a head add their scores through LDS, in one
  // round: token tiles 0..3 in the pages' space, 4..7 in the code tiles'
  // (both free after the loop) ----
  float4_t* xch0 = reinterpret_cast<float4_t*>(sp_dyn);        // [8 waves][4 tiles][64 lanes]
  float4_t* xch1 = reinterpret_cast<float4_t*>(&s_b[0][0][0]);
  __syncthreads();   // every wave is past the last step (whose A factors read the pages)
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    xch0[(wave * 4 + k) * 64 + lane] = sct[k];
    xch1[(wave * 4 + k) * 64 + lane] = sct[4 + k];
  }
  __syncthreads();   // also: every wave's scores read s_cs, which takes the H8 exchange below
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float4_t o0 = xch0[((wave ^ 1) * 4 + k) * 64 + lane], o1 = xch1[((wave ^ 1) * 4 + k) * 64 + lane];
    // the same sum in both waves: the lower half's value first
    sct[k] = r2 == 0 ? sct[k] + o0 : o0 + sct[k];
    sct[4 + k] = r2 == 0 ? sct[4 + k] + o1 : o1 + sct[4 + k];
  }
  // lane 16q + n holds query n's scores of tokens 16tt + 4q + i
  float m = -INFINITY;
#pragma unroll
  for (int tt = 0; tt < 8; ++tt)
#pragma unroll
    for (int i = 0; i < 4; ++i) m = fmaxf(m, sct[tt][i] * a.sm_scale);
  m = fmaxf(m, __shfl_xor(m, 16));
  m = fmaxf(m, __shfl_xor(m, 32));
  const bool qok = n < a.n_q_groups;
  half4_t pw[8];
  float l = 0.f;
#pragma unroll
  for (int tt = 0; tt < 8; ++tt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const _Float16 pr = qok ? (_Float16)__expf(sct[tt][i] * a.sm_scale - m) : (_Float16)0.f;
      pw[tt][i] = pr;
      l += (float)pr;
    }
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  if constexpr (kVFull) {
    // Full-C values: every head of the block reads the same slice codes, so
    // the 4 heads' weights share the A rows, (local head, query) = divmod(r,
    // G) for row r, each signed by H_{C/128}[h][slice], and wave w takes the
    // 16-channel block ct = w of all of them: G <= 4 fills one 16-row tile.
    if (r2 == 0 && q == 0 && qok && head_ok) {
      float* dst = sp_part_ml(a.partials, (int64_t)h * a.n_q_groups + n, a.n_tokens / kSpBlk, blk);
      dst[0] = m;
      dst[1] = l;
    }
    // the weights times the token norms, [local head][value page][q][query]
    // half4, in the pages' space past the score exchange (dynamic LDS of 48
    // KB at least), and the codes, [page][slice][lane][2] u32, in the RoPE
    // table's (every wave's scores have read it): one barrier for both
    uint8_t* vcl = reinterpret_cast<uint8_t*>(&s_cs[0][0]);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (tid + 512 * i < 8 * vf_chunks) reinterpret_cast<u32x4_t*>(vcl)[tid + 512 * i] = vfc[i];
    u32x2_t* s_aw = reinterpret_cast<u32x2_t*>(sp_dyn + kSpVfAwOff);
    if (r2 == 0) {
#pragma unroll
      for (int tt = 0; tt < 8; ++tt) {
        const uint2 nr = s_nrm[0][tt][q];
        const float nv[4] = {half_bits_to_float(nr.x & 0xffffu), half_bits_to_float(nr.x >> 16),
                             half_bits_to_float(nr.y & 0xffffu), half_bits_to_float(nr.y >> 16)};
        half4_t aw;
#pragma unroll
        for (int i = 0; i < 4; ++i) aw[i] = (_Float16)((float)pw[tt][i] * nv[i]);
        s_aw[((hl * 8 + tt) * 4 + q) * 16 + n] = __builtin_bit_cast(u32x2_t, aw);
      }
    }
    __syncthreads();
    const int G = a.n_q_groups, nrg = (4 * G + 15) >> 4;
    float4_t* xv = reinterpret_cast<float4_t*>(sp_dyn);   // [8 blocks][4 row groups][64 lanes]
    for (int rg = 0; rg < nrg; ++rg) {
      const int r = 16 * rg + n, hr = r / G, qr = r - hr * G;
      const uint32_t amsk = hr < 4 ? 0xffffffffu : 0u;
      const int hg = 4 * hq + hr;
      const u32x2_t* ap = s_aw + (min(hr, 3) * 32 + q) * 16 + qr;
      float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int tt = 0; tt < 8; ++tt) {
        const u32x2_t aw = ap[tt * 64] & amsk;
        // two slices per 32-deep MFMA: K index 8q + i is token 4q + i of
        // slice 2sp for i < 4, of slice 2sp + 1 after
#pragma unroll
        for (int sp = 0; sp < 4; ++sp) {
          const int s0 = 2 * sp;
          if (s0 >= a.h_kv) break;
          const bool has1 = s0 + 1 < a.h_kv;
          const int s1 = has1 ? s0 + 1 : s0;
          const uint32_t n0 = vfull_neg(hg, s0) ? 0x80008000u : 0u;
          const uint32_t n1 = vfull_neg(hg, s0 + 1) ? 0x80008000u : 0u;
          const uint32_t m1 = has1 ? 0xffffffffu : 0u;
          const u32x4_t A4 = {aw[0] ^ n0, aw[1] ^ n0, (aw[0] ^ n1) & m1, (aw[1] ^ n1) & m1};
          const uint32_t b0 = vcl[(tt * a.h_kv + s0) * 512 + lane * 8 + wave];
          const uint32_t b1 = vcl[(tt * a.h_kv + s1) * 512 + lane * 8 + wave];
          const uint2 l0 = s_cbl[b0], l1 = s_cbl[b1];
          const u32x4_t B4 = {l0.x, l0.y, l1.x, l1.y};
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, A4),
                                                       __builtin_bit_cast(half8_t, B4), acc, 0, 0, 0);
        }
      }
      xv[(wave * 4 + rg) * 64 + lane] = acc;
    }
    __syncthreads();
    // H8 over the block index ct (bits 0, 1, 2 in turn) in every wave; wave
    // w stores block w: rows 16 rg + 4q + i, channel n (the merge applies
    // H16 over that channel)
    const int n_parts = a.n_tokens / kSpBlk;
    for (int rg = 0; rg < nrg; ++rg) {
      float4_t y[8];
#pragma unroll
      for (int ct = 0; ct < 8; ++ct) y[ct] = xv[(ct * 4 + rg) * 64 + lane];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int sb = 1; sb < 8; sb <<= 1)
#pragma unroll
          for (int ct = 0; ct < 8; ++ct)
            if (!(ct & sb)) {
              const float u = y[ct][i], w = y[ct | sb][i];
              y[ct][i] = u + w;
              y[ct | sb][i] = u - w;
            }
      float4_t o = y[0];
#pragma unroll
      for (int ct = 1; ct < 8; ++ct)
        if (wave == ct) o = y[ct];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 16 * rg + 4 * q + i, hr = r / G, qr = r - hr * G, hg = 4 * hq + hr;
        if (hr < 4 && hg < a.h_kv) sp_part_ch(a.partials, (int64_t)hg * G + qr, n_parts, wave, blk)[n] = o[i];
      }
    }
  } else {
  // P.V in the rotated value domain, value page tt (= token tile tt), this
  // wave's channel blocks ct = 4 r2 + c (waves past the heads compute head 0's)
  float4_t pv[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) pv[c] = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int tt = 0; tt < 8; ++tt) {
    const uint2 nr = s_nrm[hl][tt][q];
    const float nv[4] = {half_bits_to_float(nr.x & 0xffffu), half_bits_to_float(nr.x >> 16),
                         half_bits_to_float(nr.y & 0xffffu), half_bits_to_float(nr.y >> 16)};
    half4_t aw;
#pragma unroll
    for (int i = 0; i < 4; ++i) aw[i] = (_Float16)((float)pw[tt][i] * nv[i]);
    const uint32_t vc = r2 == 0 ? s_vcd[hl][tt][lane].x : s_vcd[hl][tt][lane].y;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint2 lvb = s_cbl[(vc >> (8 * c)) & 0xFFu];
      const half4_t vb = *reinterpret_cast<const half4_t*>(&lvb);
      pv[c] = __builtin_amdgcn_mfma_f32_16x16x16f16(aw, vb, pv[c], 0, 0, 0);
    }
  }
  // H8 over the block index ct = 4 r2 + c: c in registers, r2 (the
  // channel's bit 6) with the head's other wave through LDS (the RoPE
  // table's space, read before the barrier above); the merge applies H16
  // over n
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int sb = 1; sb < 4; sb <<= 1)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (!(c & sb)) {
          const float u = pv[c][i], w = pv[c | sb][i];
          pv[c][i] = u + w;
          pv[c | sb][i] = u - w;
        }
  // [8 waves][4 blocks][64 lanes]: 32 KB, in the RoPE table's space
  float4_t* xv = reinterpret_cast<float4_t*>(&s_cs[0][0]);
#pragma unroll
  for (int c = 0; c < 4; ++c) xv[(wave * 4 + c) * 64 + lane] = pv[c];
  __syncthreads();
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const float4_t o = xv[((wave ^ 1) * 4 + c) * 64 + lane];
#pragma unroll
    for (int i = 0; i < 4; ++i) pv[c][i] = r2 == 0 ? pv[c][i] + o[i] : o[i] - pv[c][i];
  }
  if (!head_ok) return;
  const int n_parts = a.n_tokens / kSpBlk;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int qi = 4 * q + i;
    if (qi < a.n_q_groups) {
      const int64_t r = (int64_t)h * a.n_q_groups + qi;
#pragma unroll
      for (int c = 0; c < 4; ++c) sp_part_ch(a.partials, r, n_parts, 4 * r2 + c, blk)[n] = pv[c][i];
    }
  }
  if (r2 == 0 && q == 0 && qok) {
    float* dst = sp_part_ml(a.partials, (int64_t)h * a.n_q_groups + n, n_parts, blk);
    dst[0] = m;
    dst[1] = l;
  }
  }
}

constexpr int kSpMaxWin = 4096;

struct SpMergeKArgs {
  int h_kv, G, n_groups, q_dtype, win_len, out_dtype;
  int win_bf16;     // k_win / v_win in bf16, else fp16
  int64_t win_sh;   // elements between heads in k_win / v_win
  const float* partials;
  const void* q;
  const uint16_t* k_win;
  const uint16_t* v_win;
  float sm_scale;
  void* out;
  uint32_t sign_h[8][4];   // the value codec's signs of head h's 128 channels
  float v_scale;           // 1/128 (per-head codec) or 1/C (full-C codec)
};

constexpr int kSpMergeMaxGroups = 16384;   // 1M committed tokens
constexpr int kSpMergeBatch = 8;           // parts per thread whose loads are in flight together

// Max or sum of one value per thread over a 256-thread block (the result in
// every thread); s_red holds 4 floats.
template <bool kMax>
__device__ __forceinline__ float reduce256(float v, float* s_red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float u = __shfl_xor(v, o);
    v = kMax ? fmaxf(v, u) : v + u;
  }
  __syncthreads();   // s_red free from any earlier reduction
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = v;
  __syncthreads();
  return kMax ? fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]))
              : (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
}

__device__ __forceinline__ float4_t f4_fma(float w, float4_t x, float4_t acc) {
  return (float4_t){fmaf(w, x[0], acc[0]), fmaf(w, x[1], acc[1]), fmaf(w, x[2], acc[2]), fmaf(w, x[3], acc[3])};
}

// grid (8 chunks, G, h_kv), block 256: channels 16 chunk .. 16 chunk + 15 of
// query row (h, g).  The partials come in the value domain up to the codec's
// signs and 1/128 (the dequant kernels apply the 128-point Hadamard to each),
// so a chunk needs only its 16 channels of every partial, the partials'
// (m, l) and the window; the 256 workgroups do the merge in one pass.
// Thread (slot s = tid >> 2, quad c4 = tid & 3) takes the partials and window
// rows s + 64k and channels 16 chunk + 4 c4 .. + 3; for the window scores,
// thread tid takes token tid >> 1 of each 128-token pass and half tid & 1 of
// the dims.  Every load of the first batch of partials and of the first pass
// of the window is issued before anything waits.
__global__ __launch_bounds__(256) void spectral_merge_kernel(const SpMergeKArgs a) {
  const int chunk = blockIdx.x, g = blockIdx.y, h = blockIdx.z, tid = threadIdx.x;
  const int slot = tid >> 2, c4 = tid & 3, c0 = 16 * chunk + 4 * c4;
  const int tw = tid >> 1, half = tid & 1;
  __shared__ float s_q[kD];
  __shared__ float s_s[kSpMaxWin];
  __shared__ float s_red[4];
  __shared__ float4_t s_sum[4][4], s_sumw[4][4];
  const int64_t row = (int64_t)h * a.G + g;
  const float* pml = a.partials + row * 130 * (int64_t)a.n_groups;          // (m, l) of partial p at 2p
  const float* pch = pml + 2 * (int64_t)a.n_groups + 16 * (int64_t)chunk * a.n_groups + 4 * c4;   // + 16p
  const int P = a.n_groups, T = a.win_len;
  const uint16_t* kbase = a.k_win + (int64_t)h * a.win_sh;
  const uint16_t* vbase = a.v_win + (int64_t)h * a.win_sh;
  const bool wbf = a.win_bf16;
  auto wcvt = [wbf](uint32_t bits) {   // a window element's 16 low bits as fp32
    return wbf ? __uint_as_float(bits << 16) : half_bits_to_float(bits & 0xffffu);
  };
  // ---- loads: the query, the first batch of partials, the first window pass
  float qv = 0.f;
  if (tid < kD) qv = sp_load(a.q, row * kD + tid, a.q_dtype);
  float2 ml[kSpMergeBatch];
  float4_t y[kSpMergeBatch];
  auto load_part = [&](int p, float2& m_l, float4_t& yy) {   // p clamped by the caller
    m_l = *reinterpret_cast<const float2*>(pml + 2 * (int64_t)p);
    const float* r = pch + 16 * (int64_t)p;   // 8-byte aligned: two 8-byte loads
    const float2 lo = *reinterpret_cast<const float2*>(r), hi = *reinterpret_cast<const float2*>(r + 2);
    yy = (float4_t){lo.x, lo.y, hi.x, hi.y};
  };
  if (P > 0) {
#pragma unroll
    for (int k = 0; k < kSpMergeBatch; ++k) load_part(min(slot + 64 * k, P - 1), ml[k], y[k]);
  }
  uint4 kr[8];
  uint2 vr[2];
  if (T > 0) {
    const uint16_t* kp = kbase + (int64_t)min(tw, T - 1) * kD + 64 * half;
#pragma unroll
    for (int i = 0; i < 8; ++i) kr[i] = reinterpret_cast<const uint4*>(kp)[i];
#pragma unroll
    for (int k = 0; k < 2; ++k)
      vr[k] = *reinterpret_cast<const uint2*>(vbase + (int64_t)min(slot + 64 * k, T - 1) * kD + c0);
  }
  if (tid < kD) s_q[tid] = qv;
  __syncthreads();
  // ---- the window's scaled scores, 128 tokens a pass, into s_s
  float mx = -INFINITY;
  for (int t0 = 0; t0 < T; t0 += 128) {
    const int t = t0 + tw;
    if (t0 > 0) {
      const uint16_t* kp = kbase + (int64_t)min(t, T - 1) * kD + 64 * half;
#pragma unroll
      for (int i = 0; i < 8; ++i) kr[i] = reinterpret_cast<const uint4*>(kp)[i];
    }
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t w4[4] = {kr[i].x, kr[i].y, kr[i].z, kr[i].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int d = 64 * half + 8 * i + 2 * e;
        acc = fmaf(s_q[d], wcvt(w4[e] & 0xffffu), acc);
        acc = fmaf(s_q[d + 1], wcvt(w4[e] >> 16), acc);
      }
    }
    acc += __shfl_xor(acc, 1);
    if (t < T) {
      const float sc = acc * a.sm_scale;
      if (half == 0) s_s[t] = sc;
      mx = fmaxf(mx, sc);
    }
  }
  // ---- the partials' maxima (later batches: the maxima alone)
#pragma unroll
  for (int k = 0; k < kSpMergeBatch; ++k)
    if (slot + 64 * k < P) mx = fmaxf(mx, ml[k].x);
  for (int p0 = 64 * kSpMergeBatch; p0 < P; p0 += 64)
    if (p0 + slot < P) mx = fmaxf(mx, pml[2 * (int64_t)(p0 + slot)]);
  const float M = reduce256<true>(mx, s_red);   // its barriers also publish s_s
  // ---- weights and sums: L counts each partial and token once (quad 0)
  float L = 0.f;
  float4_t A = {0.f, 0.f, 0.f, 0.f}, W = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < kSpMergeBatch; ++k)
    if (slot + 64 * k < P) {
      const float w = __expf(ml[k].x - M);
      if (c4 == 0) L = fmaf(w, ml[k].y, L);
      A = f4_fma(w, y[k], A);
    }
  for (int p0 = 64 * kSpMergeBatch; p0 < P; p0 += 64 * kSpMergeBatch) {
#pragma unroll
    for (int k = 0; k < kSpMergeBatch; ++k) load_part(min(p0 + slot + 64 * k, P - 1), ml[k], y[k]);
#pragma unroll
    for (int k = 0; k < kSpMergeBatch; ++k)
      if (p0 + slot + 64 * k < P) {
        const float w = __expf(ml[k].x - M);
        if (c4 == 0) L = fmaf(w, ml[k].y, L);
        A = f4_fma(w, y[k], A);
      }
  }
  for (int t0 = 0; t0 < T; t0 += 128) {
    if (t0 > 0) {
#pragma unroll
      for (int k = 0; k < 2; ++k)
        vr[k] = *reinterpret_cast<const uint2*>(vbase + (int64_t)min(t0 + slot + 64 * k, T - 1) * kD + c0);
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int t = t0 + slot + 64 * k;
      if (t < T) {
        const float w = __expf(s_s[t] - M);
        if (c4 == 0) L += w;
        const float4_t v = {wcvt(vr[k].x & 0xffffu), wcvt(vr[k].x >> 16), wcvt(vr[k].y & 0xffffu),
                            wcvt(vr[k].y >> 16)};
        W = f4_fma(w, v, W);
      }
    }
  }
  // ---- sums over the slots: the lanes of a wave with this quad, then the waves
#pragma unroll
  for (int o = 4; o <= 32; o <<= 1)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      A[e] += __shfl_xor(A[e], o);
      W[e] += __shfl_xor(W[e], o);
    }
  const float Ls = reduce256<false>(L, s_red);
  if ((tid & 63) < 4) {
    s_sum[tid >> 6][c4] = A;
    s_sumw[tid >> 6][c4] = W;
  }
  __syncthreads();
  if (tid < 64) {   // wave 0; lanes 0..15 hold the chunk's channels
    const int cc = tid & 15, q4 = cc >> 2, e = cc & 3;
    float x = (s_sum[0][q4][e] + s_sum[1][q4][e]) + (s_sum[2][q4][e] + s_sum[3][q4][e]);
    const float w = (s_sumw[0][q4][e] + s_sumw[1][q4][e]) + (s_sumw[2][q4][e] + s_sumw[3][q4][e]);
    x = h16_lanes(x, cc);   // the Hadamard's bits 0..3, then the codec's signs and scale
    const int c = 16 * chunk + cc;
    if (tid < 16) store_elem(a.out, row * kD + c, ((sign_neg(a.sign_h[h], c) ? -x : x) * a.v_scale + w) / Ls,
                             a.out_dtype);
  }
}

// Value-only pages: VNORM (h_kv x 16 fp16, or 16 for the full-C codec), then VCODE
static PageLayout value_layout(int h_kv, bool full = false) {
  PageLayout L{};
  L.vnorm = 0;
  L.vcode = (full ? 1 : h_kv) * kPT * 2;
  L.bytes = L.vcode + h_kv * 64 * 8;
  return L;
}

static bool v_codec_ok(int v_codec, int h_kv) {
  return v_codec == BMX_SPECTRAL_V_PERHEAD ||
         (v_codec == BMX_SPECTRAL_V_FULL && (h_kv == 1 || h_kv == 2 || h_kv == 4 || h_kv == 8));
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

// The 128-token partial form serves a decode step whose two key pages fit in
// LDS together, with the fp16-rounded RoPE table and 128-token multiples.
// The partial form runs on 128-token blocks when both key pages of a block
// fit in LDS together; the partials pointer itself is not consulted, so the
// count below can be asked before the buffer exists.
static bool sp_block_shape(const bmx_spectral_dequant_args* a) {
  return a->q && !a->k_out && a->apply_rope == 2 && a->n_tokens % kSpBlk == 0 &&
         2 * (int64_t)a->L.k_page_bytes <= kSpBlkMaxPages;
}

static bool sp_blocked(const bmx_spectral_dequant_args* a) { return a->partials && sp_block_shape(a); }

constexpr size_t kLdsBytes = 160 * 1024;   // per workgroup on gfx950

// A launch whose static and dynamic LDS exceed the CU's is not a valid
// allocation: refuse it on the host instead.  The kernels' static sizes are
// asked once each (a few kernels: a small table under a lock).
static bool sp_lds_fits(const void* kernel, size_t dyn) {
  static std::mutex mu;
  static const void* keys[16];
  static size_t vals[16];
  static int n = 0;
  size_t stat = (size_t)-1;
  {
    std::lock_guard<std::mutex> lock(mu);
    for (int i = 0; i < n; ++i)
      if (keys[i] == kernel) stat = vals[i];
  }
  if (stat == (size_t)-1) {
    hipFuncAttributes attr{};
    if (hipFuncGetAttributes(&attr, kernel) != hipSuccess) return false;
    stat = attr.sharedSizeBytes;
    std::lock_guard<std::mutex> lock(mu);
    if (n < 16) {
      keys[n] = kernel;
      vals[n++] = stat;
    }
  }
  return stat + dyn <= kLdsBytes;
}

}  // namespace bmx

using namespace bmx;

extern "C" int64_t bmx_spectral_v_page_bytes(int32_t h_kv) {
  return (h_kv < 1 || h_kv > 8) ? -1 : (int64_t)value_layout(h_kv).bytes;
}

extern "C" int64_t bmx_spectral_v_page_bytes_codec(int32_t h_kv, int32_t v_codec) {
  if (h_kv < 1 || h_kv > 8 || !v_codec_ok(v_codec, h_kv)) return -1;
  return (int64_t)value_layout(h_kv, v_codec == BMX_SPECTRAL_V_FULL).bytes;
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
  if (!v_codec_ok(a->v_codec, a->L.h_kv))
    return sp_fail(fn, "v_codec must be BMX_SPECTRAL_V_PERHEAD, or BMX_SPECTRAL_V_FULL with h_kv 1, 2, 4 or 8");
  hipStream_t st = (hipStream_t)stream;
  SpEncodeKArgs k{};
  k.C = kD * a->L.h_kv; k.c_pad = a->L.c_pad; k.n_pool = a->n_k_pool; k.k_dtype = a->k_dtype;
  k.page_bytes = a->L.k_page_bytes;
  k.k = a->k_pre; k.ksh = a->k_sh; k.kst = a->k_st;
  k.encp = a->enc_perm; k.slice_tab = a->L.slice_tab; k.pages = a->k_pages; k.page_ids = a->k_page_ids;
  k.lq = a->L.lloyd_levels;
  if (k.lq)
    hipLaunchKernelGGL(spectral_encode_kernel<true>, dim3((a->L.c_pad + 63) / 64, a->n_groups), dim3(512), 0, st, k);
  else
    hipLaunchKernelGGL(spectral_encode_kernel<false>, dim3((a->L.c_pad + 63) / 64, a->n_groups), dim3(512), 0, st, k);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess && a->v_codec == BMX_SPECTRAL_V_FULL) {
    SpVFullKArgs v{};
    v.h_kv = a->L.h_kv; v.n_pool = a->n_v_pool; v.v_dtype = a->v_dtype;
    v.v = a->v; v.vsh = a->v_sh; v.vst = a->v_st;
    v.pages = a->v_pages; v.page_ids = a->v_page_ids; v.L = value_layout(a->L.h_kv, true);
    for (int i = 0; i < 4; ++i) v.codebook[i] = a->v_codebook[i];
    for (int i = 0; i < 32; ++i) v.sign_c[i] = a->v_sign_bits_c[i];
    hipLaunchKernelGGL(spectral_vfull_kernel, dim3(4 * 4 * a->n_groups), dim3(256), 0, st, v);
    e = hipGetLastError();
  } else if (e == hipSuccess) {
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
  if (a->out_rows != 0 && a->out_rows < a->n_tokens) return sp_fail(fn, "out_rows must be 0 or >= n_tokens");
  if (a->L.k_page_bytes > kSpMaxKPage) return sp_fail(fn, "k_page_bytes above 73728 (the LDS-staged page)");
  if (!a->k_pages || !a->k_page_table || !a->v_pages || !a->v_page_table || !a->dec_perm ||
      (!a->v_out && !a->partials) || (!a->k_out && !a->q) || a->n_k_pool < 1 || a->n_v_pool < 1)
    return sp_fail(fn, "null pointer argument or empty pool");
  if (a->q && ((!a->scores && !a->partials) || a->n_q_groups < 1 || a->n_q_groups > 16 || !dtype_ok(a->q_dtype) ||
               !a->apply_rope))
    return sp_fail(fn, "the decode form needs scores or partials, n_q_groups 1..16, a q_dtype and apply_rope");
  if (a->partials && !a->q) return sp_fail(fn, "the partial form needs q");
  if (!v_codec_ok(a->v_codec, a->L.h_kv))
    return sp_fail(fn, "v_codec must be BMX_SPECTRAL_V_PERHEAD, or BMX_SPECTRAL_V_FULL with h_kv 1, 2, 4 or 8");
  SpDequantKArgs k{};
  k.h_kv = a->L.h_kv; k.c_pad = a->L.c_pad; k.c_pad32 = (a->L.c_pad + 31) / 32 * 32;
  k.n_tokens = a->n_tokens; k.out_rows = a->out_rows ? a->out_rows : a->n_tokens;
  k.apply_rope = a->apply_rope; k.n_k_pool = a->n_k_pool; k.n_v_pool = a->n_v_pool;
  k.out_dtype = a->out_dtype; k.k_page_bytes = a->L.k_page_bytes;
  k.k_pages = a->k_pages; k.k_table = a->k_page_table; k.v_pages = a->v_pages; k.v_table = a->v_page_table;
  k.slice_tab = a->L.slice_tab; k.dec = a->dec_perm;
  k.v_full = a->v_codec == BMX_SPECTRAL_V_FULL;
  k.VL = value_layout(a->L.h_kv, k.v_full);
  for (int i = 0; i < 32; ++i) k.v_sign_c[i] = a->v_sign_bits_c[i];
  k.rope_scaling = a->rope_scaling;
  for (int j = 0; j < 64; ++j) k.inv_freq[j] = a->inv_freq[j];
  for (int i = 0; i < 4; ++i) { k.codebook[i] = a->v_codebook[i]; k.v_sign_bits[i] = a->v_sign_bits[i]; }
  k.k_out = a->k_out; k.v_out = a->v_out;
  k.q = a->q; k.q_dtype = a->q_dtype; k.n_q_groups = a->n_q_groups; k.scores = a->scores;
  k.partials = a->partials; k.sm_scale = a->sm_scale; k.lq = a->L.lloyd_levels;
  if (sp_blocked(a)) {
    const int kpb = a->L.k_page_bytes;
    // the two pages, then the score exchange (and, full-C, the weight table)
    const size_t dyn = std::max<size_t>(2 * (size_t)kpb, (size_t)kSpVfAwOff + (k.v_full ? 4 * 8 * 4 * 16 * 8 : 0));
    const dim3 grid(a->n_tokens / kSpBlk, (a->L.h_kv + 3) / 4);
    const void* kern = k.lq ? (k.v_full ? (const void*)spectral_partial128_kernel<true, true>
                                        : (const void*)spectral_partial128_kernel<true, false>)
                            : (k.v_full ? (const void*)spectral_partial128_kernel<false, true>
                                        : (const void*)spectral_partial128_kernel<false, false>);
    if (!sp_lds_fits(kern, dyn)) return sp_fail(fn, "the 128-token kernel's LDS does not fit this key page size");
    if (k.lq && k.v_full)
      hipLaunchKernelGGL((spectral_partial128_kernel<true, true>), grid, dim3(512), dyn, (hipStream_t)stream, k, kpb);
    else if (k.lq)
      hipLaunchKernelGGL((spectral_partial128_kernel<true, false>), grid, dim3(512), dyn, (hipStream_t)stream, k, kpb);
    else if (k.v_full)
      hipLaunchKernelGGL((spectral_partial128_kernel<false, true>), grid, dim3(512), dyn, (hipStream_t)stream, k, kpb);
    else
      hipLaunchKernelGGL((spectral_partial128_kernel<false, false>), grid, dim3(512), dyn, (hipStream_t)stream, k,
                         kpb);
  } else if (!sp_lds_fits(k.lq ? (const void*)spectral_dequant_kernel<true> : (const void*)spectral_dequant_kernel<false>,
                          sp_dyn_bytes(a->L.k_page_bytes))) {
    return sp_fail(fn, "the 64-token kernel's LDS does not fit this key page size");
  } else if (k.lq) {
    hipLaunchKernelGGL(spectral_dequant_kernel<true>, dim3(a->n_tokens / kGroup), dim3(512),
                       sp_dyn_bytes(a->L.k_page_bytes), (hipStream_t)stream, k);
  } else {
    hipLaunchKernelGGL(spectral_dequant_kernel<false>, dim3(a->n_tokens / kGroup), dim3(512),
                       sp_dyn_bytes(a->L.k_page_bytes), (hipStream_t)stream, k);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    bmx_set_error(std::string(fn) + ": launch: " + hipGetErrorString(e));
    return BMX_E_HIP;
  }
  return BMX_OK;
}

extern "C" int32_t bmx_spectral_partial_count(const bmx_spectral_dequant_args* a) {
  if (!a || a->n_tokens < 0 || a->n_tokens % kGroup != 0) return -1;
  return sp_block_shape(a) ? a->n_tokens / kSpBlk : a->n_tokens / kGroup;
}

extern "C" int32_t bmx_spectral_merge(const bmx_spectral_merge_args* a, void* stream) {
  const char* fn = "bmx_spectral_merge";
  if (!a) return sp_fail(fn, "args is NULL");
  if (a->h_kv < 1 || a->h_kv > 8 || a->n_q_groups < 1 || a->n_q_groups > 16)
    return sp_fail(fn, "h_kv must be 1..8 and n_q_groups 1..16");
  if (a->n_groups < 0 || a->n_groups > kSpMergeMaxGroups || a->win_len < 0 || a->win_len > kSpMaxWin ||
      a->n_groups + a->win_len == 0)
    return sp_fail(fn, "n_groups 0..16384, win_len 0..4096, and at least one token");
  if (!dtype_ok(a->q_dtype) || !dtype_ok(a->out_dtype)) return sp_fail(fn, "q_dtype / out_dtype");
  if (!a->q || !a->out || (a->n_groups && !a->partials) || (a->win_len && (!a->k_win || !a->v_win)))
    return sp_fail(fn, "null pointer argument");
  if (a->win_len && (((uintptr_t)a->k_win & 15) != 0 || a->win_stride_h % 8 != 0 ||
                     (a->win_stride_h != 0 && a->win_stride_h < (int64_t)a->win_len * kD)))
    return sp_fail(fn, "k_win must be 16-byte aligned and win_stride_h 0 or a multiple of 8 >= 128 win_len");
  if (!v_codec_ok(a->v_codec, a->h_kv))
    return sp_fail(fn, "v_codec must be BMX_SPECTRAL_V_PERHEAD, or BMX_SPECTRAL_V_FULL with h_kv 1, 2, 4 or 8");
  if (a->win_dtype != BMX_K2B_TAIL_F16 && a->win_dtype != BMX_K2B_TAIL_BF16)
    return sp_fail(fn, "win_dtype must be BMX_K2B_TAIL_F16 or _BF16");
  SpMergeKArgs k{};
  k.win_bf16 = a->win_dtype == BMX_K2B_TAIL_BF16;
  k.h_kv = a->h_kv; k.G = a->n_q_groups; k.n_groups = a->n_groups; k.q_dtype = a->q_dtype;
  k.win_len = a->win_len; k.out_dtype = a->out_dtype; k.partials = a->partials; k.q = a->q;
  k.k_win = a->k_win; k.v_win = a->v_win; k.sm_scale = a->sm_scale; k.out = a->out;
  k.win_sh = a->win_stride_h ? a->win_stride_h : (int64_t)a->win_len * kD;
  const bool full = a->v_codec == BMX_SPECTRAL_V_FULL;
  for (int h = 0; h < 8; ++h)
    for (int i = 0; i < 4; ++i) k.sign_h[h][i] = full ? a->v_sign_bits_c[4 * h + i] : a->v_sign_bits[i];
  k.v_scale = 1.0f / (float)(full ? kD * a->h_kv : kD);
  hipLaunchKernelGGL(spectral_merge_kernel, dim3(kD / 16, a->n_q_groups, a->h_kv), dim3(256), 0, (hipStream_t)stream,
                     k);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    bmx_set_error(std::string(fn) + ": launch: " + hipGetErrorString(e));
    return BMX_E_HIP;
  }
  return BMX_OK;
}
