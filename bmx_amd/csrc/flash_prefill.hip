// Prefill attention (flash attention) over dense fp16 / bf16 K/V rows on
// gfx950: the attention of the packed cache's prefill, after the page dequant
// has written the committed rows and the window (chunked_attention.py:320-395
// runs torch SDPA at this point).
//
// Rows: for kv head h, row r = i * G + g is query position i of query head
// h * G + g, so the G heads that read one K/V head share every K/V tile.
//
// prefill_kernel<DT>: 1-D grid of (row tile, key split, kv head) workgroups,
// numbered so that each XCD (workgroups go to the 8 XCDs in turn) takes whole
// (head, split) ranges and the longest row tiles start first.  Block 256 =
// 4 waves, 128 rows per workgroup, 32 per wave.  Per 64-key tile:
//   * the tile is staged in LDS, two stages (the loads of tile t + 1 are in
//     flight while tile t is computed): K as 256-byte rows with the 16-byte
//     columns XOR-swizzled by key, V transposed (one 144-byte row of 64 keys
//     per channel), so that every MFMA operand is one conflict-free 16-byte
//     LDS read;
//   * scores S^T = K . Q^T on v_mfma_f32_32x32x16 (Q in registers), one
//     32x32 block per 32 keys.  The A-operand rows are a permutation of the
//     block's keys chosen so that result elements 8 u .. 8 u + 7 of lane half
//     hf are keys 16 u + 8 hf .. +7: the B operand of P^T for the values'
//     MFMA over key sub-block u, converted in place;
//   * online softmax in base 2: a lane holds 32 scores of one row, the row's
//     2 lanes exchange the maximum; only tiles that cross the causal edge or
//     the end of the keys are masked;
//   * O^T += V^T . P^T (V^T read from the transposed tile).
// With one key split per row tile the workgroup writes the normalized rows;
// with several it writes (O, m, l) partials that prefill_combine_kernel
// merges by their softmax weights.

#include "bmx_prefill.h"
#include "k2b_common.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <string>
#include <type_traits>

namespace bmx {
namespace {

constexpr int kPfD = 128;                         // head dim
constexpr int kPfKeys = 64;                       // keys per tile
constexpr int kPfWaves = 4;
constexpr int kPfThreads = 64 * kPfWaves;
constexpr int kPfRows = 32 * kPfWaves;            // rows per workgroup
constexpr int kPfKsBytes = kPfKeys * kPfD * 2;    // K tile: 64 rows of 256 B
constexpr int kPfVtPitch = 2 * kPfKeys + 16;      // V tile transposed: 144 B per channel
constexpr int kPfVtBytes = kPfD * kPfVtPitch;
constexpr int kPfStage = kPfKsBytes + kPfVtBytes;
constexpr int kPfLds = 2 * kPfStage;              // 69,632 B: two workgroups per CU
constexpr int kPfMaxSplit = 16;
constexpr int kPfBufWord3 = 0x00020000;           // raw buffer descriptor, word 3

struct PfArgs {
  const uint16_t* q;
  int64_t qsh, qst;      // elements
  const uint16_t* k;
  const uint16_t* v;
  int64_t sh, st;        // elements
  uint16_t* out;         // [h_kv * G][n_q][128]
  float* part_o;         // [h_kv][n_split][R][128]
  float* part_ml;        // [h_kv][n_split][R][2]: m (base 2, scaled), l
  int G, n_q, n_kv, R, off, causal, n_split, n_rt;
  float qscale;          // sm_scale * log2(e)
};

template <int DT>
__device__ __forceinline__ uint32_t pf_pack(float x, float y) {
  if constexpr (DT == BMX_PREFILL_F16) {
    const half2_t h = {(_Float16)x, (_Float16)y};
    return __builtin_bit_cast(uint32_t, h);
  } else {
    typedef __bf16 bf2_t __attribute__((ext_vector_type(2)));
    const bf2_t b = {(__bf16)x, (__bf16)y};
    return __builtin_bit_cast(uint32_t, b);
  }
}

typedef float float16_t __attribute__((ext_vector_type(16)));

template <int DT>
__device__ __forceinline__ float16_t pf_mma32(u32x4_t a, u32x4_t b, float16_t c) {
  if constexpr (DT == BMX_PREFILL_F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, a), __builtin_bit_cast(half8_t, b),
                                                  c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// byte offset of 16-byte column c of key row `key` in the K tile: the 16
// keys one MFMA operand phase reads (16 consecutive keys) land on 16
// different columns of the 256-byte bank window
__device__ __forceinline__ int ks_off(int key, int c) {
  return key * (2 * kPfD) + ((c ^ (key & 15)) << 4);
}

template <int DT>
__global__ __launch_bounds__(kPfThreads) __attribute__((amdgpu_waves_per_eu(2)))
void prefill_kernel(const PfArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, col = lane & 15, grp = lane >> 4;
  const int total = gridDim.x, lin = blockIdx.x;
  const int logical = (total & 7) == 0 ? (lin & 7) * (total >> 3) + (lin >> 3) : lin;
  const int rt = a.n_rt - 1 - logical % a.n_rt;
  const int rest = logical / a.n_rt;
  const int split = rest % a.n_split, h = rest / a.n_split;
  const int R0 = rt * kPfRows;
  const int i_lo = R0 / a.G, i_hi = (min(R0 + kPfRows, a.R) - 1) / a.G;
  // keys the tile's rows see: [0, kend); every row sees [0, edge)
  const int kend = a.causal ? min(a.n_kv, i_hi + a.off + 1) : a.n_kv;
  const int edge = a.causal ? min(a.n_kv, i_lo + a.off + 1) : a.n_kv;
  const int nt = (kend + kPfKeys - 1) / kPfKeys;
  const int t0 = (int)((int64_t)split * nt / a.n_split), t1 = (int)((int64_t)(split + 1) * nt / a.n_split);
  const int t_mask = edge / kPfKeys;   // tiles from here on cross the edge or the end of the keys

  // the wave's 32 rows: Q as the B operand of the 32x32x16 MFMA (row =
  // lane % 32, channels 16 dc + 8 hf .. +7, hf = lane / 32), and the last key
  // the lane's row sees
  const int r32 = lane & 31, hf = lane >> 5;
  u32x4_t qb[8];
  int last_key;
  {
    const int r = min(R0 + 32 * wave + r32, a.R - 1);
    const int i = r / a.G, g = r - i * a.G;
    last_key = a.causal ? i + a.off : a.n_kv - 1;   // < n_kv either way
    const uint16_t* qp = a.q + (int64_t)(h * a.G + g) * a.qsh + (int64_t)i * a.qst + 8 * hf;
#pragma unroll
    for (int dc = 0; dc < 8; ++dc) qb[dc] = *reinterpret_cast<const u32x4_t*>(qp + 16 * dc);
  }
  // Q is in registers before the loop starts (vmcnt(0)): a wait inside the
  // loop, where the next tile's loads are in flight, is never needed for it
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __builtin_amdgcn_sched_barrier(0);

  // K and V of the head through buffer descriptors: rows past n_kv read zeros
  const uint32_t nrec = (uint32_t)((int64_t)a.n_kv * a.st * 2);
  const __amdgpu_buffer_rsrc_t krs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.k + (int64_t)h * a.sh), (short)0, nrec, kPfBufWord3);
  const __amdgpu_buffer_rsrc_t vrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.v + (int64_t)h * a.sh), (short)0, nrec, kPfBufWord3);
  // tile loads.  K: thread (lr, lc) = (tid / 16, tid % 16) loads 16 bytes of
  // key lr + 16 j at column lc (a 16-lane row reads a whole key row).  V:
  // thread (vr4, vc) = (tid % 16, tid / 16) loads keys 4 vr4 + j at channels
  // 8 vc .. +7, a 4-key x 8-channel block it writes transposed; the 16 lanes
  // of an LDS write phase then hold 16 different key groups of one channel
  // row: 128 contiguous bytes, every bank once
  const int lr = tid >> 4, lc = tid & 15;
  const int vr4 = tid & 15, vc = tid >> 4;
  u32x4_t kr[4], vr[4];
  auto issue = [&](int t) {
    const int k0 = t * kPfKeys;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      kr[j] = __builtin_amdgcn_raw_buffer_load_b128(
          krs, (uint32_t)(((int64_t)(k0 + lr + 16 * j) * a.st + 8 * lc) * 2), 0, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      vr[j] = __builtin_amdgcn_raw_buffer_load_b128(
          vrs, (uint32_t)(((int64_t)(k0 + 4 * vr4 + j) * a.st + 8 * vc) * 2), 0, 0);
  };
  auto stash = [&](int stage) {
    uint8_t* ks = smem + stage * kPfStage;
    uint8_t* vt = ks + kPfKsBytes;
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<u32x4_t*>(ks + ks_off(lr + 16 * j, lc)) = kr[j];
#pragma unroll
    for (int p = 0; p < 4; ++p) {   // dword p of a key row: channels 8 vc + 2 p, + 1
      const u32x2_t lo = {__builtin_amdgcn_perm(vr[1][p], vr[0][p], 0x05040100u),
                          __builtin_amdgcn_perm(vr[3][p], vr[2][p], 0x05040100u)};
      const u32x2_t hi = {__builtin_amdgcn_perm(vr[1][p], vr[0][p], 0x07060302u),
                          __builtin_amdgcn_perm(vr[3][p], vr[2][p], 0x07060302u)};
      *reinterpret_cast<u32x2_t*>(vt + (8 * vc + 2 * p) * kPfVtPitch + 8 * vr4) = lo;
      *reinterpret_cast<u32x2_t*>(vt + (8 * vc + 2 * p + 1) * kPfVtPitch + 8 * vr4) = hi;
    }
  };

  float16_t o[4];   // O^T by 32-channel block: element e = channel 32 cb + 8 (e / 4) + 4 hf + e % 4
#pragma unroll
  for (int cb = 0; cb < 4; ++cb)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[cb][e] = 0.f;
  float m = -INFINITY, l = 0.f;
  // A-operand row n (= 8 j + 4 x + e) of a 32-key block reads key 16 (j / 2)
  // + 8 x + 4 (j % 2) + e: result element 8 u + w of lane half hf is then key
  // 16 u + 8 hf + w of the block, the B operand of P^T for key sub-block u
  const int kperm = 16 * (r32 >> 4) + 8 * ((r32 >> 2) & 1) + 4 * ((r32 >> 3) & 1) + (r32 & 3);

  // one 64-key tile; kMasked: the tile crosses the causal edge of some row
  // or the end of the keys
  auto tile = [&](int t, auto masked_c) {
    constexpr bool kMasked = decltype(masked_c)::value;
    const int stage = (t - t0) & 1;
    if (t + 1 < t1) issue(t + 1);
    const uint8_t* ks = smem + stage * kPfStage;
    const uint8_t* vt = ks + kPfKsBytes;
    // ---- scores.  The MFMA blocks run at raised wave priority: of the two
    // waves on a SIMD, the one entering its MFMA block takes the issue slots
    // while the other does its softmax or stash
    __builtin_amdgcn_s_setprio(1);
    float16_t s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int key = 32 * kb + kperm;
      float16_t acc;
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
      for (int dc = 0; dc < 8; ++dc) {
        const u32x4_t ka = *reinterpret_cast<const u32x4_t*>(ks + ks_off(key, 2 * dc + hf));
        acc = pf_mma32<DT>(ka, qb[dc], acc);
      }
      s[kb] = acc;
    }
    __builtin_amdgcn_s_setprio(0);
    // ---- online softmax (base 2) of the lane's row; P^T as the values' B operand
    if constexpr (kMasked) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = t * kPfKeys + 32 * kb + 16 * (e >> 3) + 8 * hf + (e & 7);
          if (key > last_key) s[kb][e] = -INFINITY;
        }
    }
    float mx = s[0][0];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[kb][e]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    // the row keeps its offset until a score passes it by more than 8 (base
    // 2): P stays <= 256, exact in the 16-bit types' range, and the wave
    // rescales only when some row's offset moved
    const float m_cand = fmaxf(m, mx * a.qscale);
    const float m_new = m_cand > m + 8.f ? m_cand : m;
    const float m_use = m_new == -INFINITY ? 0.f : m_new;   // no visible key yet
    const float alpha = __builtin_amdgcn_exp2f(m - m_use);
    m = m_new;
    // the running sum and outputs move only when some row's maximum moved
    // (scaling by 1 is exact, so skipping it changes nothing)
    if (__builtin_amdgcn_ballot_w64(alpha != 1.f) != 0) {
      l *= alpha;
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) o[cb] *= alpha;
    }
    u32x4_t pb[4];
    float ps = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      float p[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        p[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][e], a.qscale, -m_use));
        ps += p[e];
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const u32x4_t w = {pf_pack<DT>(p[8 * u], p[8 * u + 1]), pf_pack<DT>(p[8 * u + 2], p[8 * u + 3]),
                           pf_pack<DT>(p[8 * u + 4], p[8 * u + 5]), pf_pack<DT>(p[8 * u + 6], p[8 * u + 7])};
        pb[2 * kb + u] = w;
      }
    }
    l += ps;
    // the next tile goes to the other stage ahead of the values' MFMAs, so
    // that its writes overlap them
    if (t + 1 < t1) stash(stage ^ 1);
    // ---- values: O^T += V^T . P^T over the tile's four 16-key sub-blocks
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      u32x4_t va[4];
#pragma unroll
      for (int cb = 0; cb < 4; ++cb)
        va[cb] = *reinterpret_cast<const u32x4_t*>(vt + (32 * cb + r32) * kPfVtPitch + 32 * sb + 16 * hf);
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) o[cb] = pf_mma32<DT>(va[cb], pb[sb], o[cb]);
    }
    __builtin_amdgcn_s_setprio(0);
    __syncthreads();
  };

  if (t0 < t1) {
    issue(t0);
    stash(0);
    __syncthreads();
  }
  const int t_split = max(t0, min(t1, t_mask));
  for (int t = t0; t < t_split; ++t) tile(t, std::false_type{});
  for (int t = t_split; t < t1; ++t) tile(t, std::true_type{});

  // ---- rows out: lane (r32, hf) holds row r32, channels 32 cb + 8 j + 4 hf .. +3
  {
    const float lt = l + __shfl_xor(l, 32);
    const int r = R0 + 32 * wave + r32;
    if (r < a.R) {
      if (a.n_split == 1) {
        const float inv = lt > 0.f ? 1.0f / lt : 0.f;
        const int i = r / a.G, g = r - i * a.G;
        uint16_t* op = a.out + ((int64_t)(h * a.G + g) * a.n_q + i) * kPfD + 4 * hf;
#pragma unroll
        for (int cb = 0; cb < 4; ++cb)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const u32x2_t w = {pf_pack<DT>(o[cb][4 * j] * inv, o[cb][4 * j + 1] * inv),
                               pf_pack<DT>(o[cb][4 * j + 2] * inv, o[cb][4 * j + 3] * inv)};
            *reinterpret_cast<u32x2_t*>(op + 32 * cb + 8 * j) = w;
          }
      } else {
        const int64_t prow = ((int64_t)h * a.n_split + split) * a.R + r;
        float* po = a.part_o + prow * kPfD + 4 * hf;
#pragma unroll
        for (int cb = 0; cb < 4; ++cb)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float4_t w = {o[cb][4 * j], o[cb][4 * j + 1], o[cb][4 * j + 2], o[cb][4 * j + 3]};
            *reinterpret_cast<float4_t*>(po + 32 * cb + 8 * j) = w;
          }
        if (hf == 0) {
          const float2 ml = make_float2(m, lt);
          *reinterpret_cast<float2*>(a.part_ml + 2 * prow) = ml;
        }
      }
    }
  }
}

struct PfCombineArgs {
  const float* part_o;
  const float* part_ml;
  uint16_t* out;
  int G, n_q, R, n_split;
};

// one row per 32 lanes (4 channels each), 8 rows per workgroup
template <int DT>
__global__ __launch_bounds__(256) void prefill_combine_kernel(const PfCombineArgs c) {
  const int h = blockIdx.y, r = blockIdx.x * 8 + (threadIdx.x >> 5), q4 = threadIdx.x & 31;
  if (r >= c.R) return;
  const int64_t base = (int64_t)h * c.n_split * c.R + r;   // partial row of split 0
  float M = -INFINITY;
  for (int s = 0; s < c.n_split; ++s) M = fmaxf(M, c.part_ml[2 * (base + (int64_t)s * c.R)]);
  float den = 0.f;
  float4_t num = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < c.n_split; ++s) {
    const int64_t prow = base + (int64_t)s * c.R;
    const float2 ml = *reinterpret_cast<const float2*>(c.part_ml + 2 * prow);
    const float w = ml.x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml.x - M);
    den = __builtin_fmaf(w, ml.y, den);
    const float4_t v = *reinterpret_cast<const float4_t*>(c.part_o + prow * kPfD + 4 * q4);
    num += w * v;
  }
  const float inv = den > 0.f ? 1.0f / den : 0.f;
  const int i = r / c.G, g = r - i * c.G;
  const u32x2_t w = {pf_pack<DT>(num[0] * inv, num[1] * inv), pf_pack<DT>(num[2] * inv, num[3] * inv)};
  *reinterpret_cast<u32x2_t*>(c.out + ((int64_t)(h * c.G + g) * c.n_q + i) * kPfD + 4 * q4) = w;
}

int pf_fail(int code, const std::string& msg) {
  bmx_set_error("bmx_prefill: " + msg);
  return code;
}

// "" when the arguments describe a call the kernels support
std::string pf_check(const bmx_prefill_args* a) {
  if (!a) return "NULL arguments";
  if (!a->q || !a->k || !a->v || !a->out) return "q, k, v and out must be non-NULL";
  if (a->head_dim != kPfD) return "head_dim must be 128";
  if (a->dtype != BMX_PREFILL_F16 && a->dtype != BMX_PREFILL_BF16) return "dtype must be BMX_PREFILL_F16 or _BF16";
  if (a->h_kv < 1 || a->n_q_groups < 1 || a->n_q < 1 || a->n_kv < 1) return "h_kv, n_q_groups, n_q, n_kv must be >= 1";
  if (a->causal && a->n_q > a->n_kv) return "causal needs n_q <= n_kv (the queries are the last n_q positions)";
  if (a->n_split < 0 || a->n_split > kPfMaxSplit) return "n_split must be 0..16";
  if (a->q_stride_h % 8 || a->q_stride_t % 8 || a->kv_stride_h % 8 || a->kv_stride_t % 8)
    return "strides must be multiples of 8 elements (16-byte rows)";
  if (a->kv_stride_t < kPfD) return "kv_stride_t must be >= 128";
  if (((uintptr_t)a->q | (uintptr_t)a->k | (uintptr_t)a->v | (uintptr_t)a->out) & 15)
    return "q, k, v and out must be 16-byte aligned";
  // one head's rows are addressed with 32-bit byte offsets (buffer loads)
  if ((int64_t)(a->n_kv + kPfKeys) * a->kv_stride_t * 2 > INT32_MAX) return "a head's K/V rows exceed 2 GiB";
  if ((int64_t)a->n_q * a->n_q_groups > INT32_MAX / 2) return "too many rows";
  return "";
}

int pf_row_tiles(const bmx_prefill_args* a) {
  return (int)(((int64_t)a->n_q * a->n_q_groups + kPfRows - 1) / kPfRows);
}

// key splits: enough workgroups for two per CU, each split at least 4 tiles
int pf_splits(const bmx_prefill_args* a) {
  if (a->n_split > 0) return a->n_split;
  const int64_t base = (int64_t)pf_row_tiles(a) * a->h_kv;
  int s = (int)std::min<int64_t>((512 + base - 1) / base, kPfMaxSplit);
  const int nt = (a->n_kv + kPfKeys - 1) / kPfKeys;
  s = std::min(s, std::max(1, nt / 4));
  return std::max(s, 1);
}

}  // namespace
}  // namespace bmx

using namespace bmx;

extern "C" size_t bmx_prefill_workspace_bytes(const bmx_prefill_args* a) {
  if (!pf_check(a).empty()) return 0;
  const int s = pf_splits(a);
  if (s == 1) return 0;
  return (size_t)a->h_kv * s * ((size_t)a->n_q * a->n_q_groups) * (kPfD + 2) * sizeof(float);
}

extern "C" int bmx_prefill(const bmx_prefill_args* a, void* stream) {
  const std::string why = pf_check(a);
  if (!why.empty()) return pf_fail(BMX_PREFILL_E_INVALID, why);
  const int S = pf_splits(a);
  const size_t need = bmx_prefill_workspace_bytes(a);
  if (need && (!a->workspace || a->workspace_bytes < need))
    return pf_fail(BMX_PREFILL_E_INVALID, "workspace too small (bmx_prefill_workspace_bytes)");
  PfArgs k{};
  k.q = static_cast<const uint16_t*>(a->q);
  k.qsh = a->q_stride_h;
  k.qst = a->q_stride_t;
  k.k = static_cast<const uint16_t*>(a->k);
  k.v = static_cast<const uint16_t*>(a->v);
  k.sh = a->kv_stride_h;
  k.st = a->kv_stride_t;
  k.out = static_cast<uint16_t*>(a->out);
  k.G = a->n_q_groups;
  k.n_q = a->n_q;
  k.n_kv = a->n_kv;
  k.R = a->n_q * a->n_q_groups;
  k.off = a->n_kv - a->n_q;
  k.causal = a->causal ? 1 : 0;
  k.n_split = S;
  k.n_rt = pf_row_tiles(a);
  k.qscale = a->sm_scale * 1.4426950408889634f;
  if (S > 1) {
    k.part_o = static_cast<float*>(a->workspace);
    k.part_ml = k.part_o + (size_t)a->h_kv * S * k.R * kPfD;
  }
  hipStream_t st = (hipStream_t)stream;
  const int64_t blocks = (int64_t)k.n_rt * S * a->h_kv;
  if (blocks > INT32_MAX) return pf_fail(BMX_PREFILL_E_INVALID, "too many workgroups");
  const void* fn = a->dtype == BMX_PREFILL_F16 ? (const void*)prefill_kernel<BMX_PREFILL_F16>
                                                : (const void*)prefill_kernel<BMX_PREFILL_BF16>;
  if (bmx_ensure_dynamic_lds(fn, kPfLds) != hipSuccess)
    return pf_fail(BMX_PREFILL_E_HIP, "cannot reserve the kernel's LDS");
  if (a->dtype == BMX_PREFILL_F16)
    hipLaunchKernelGGL(prefill_kernel<BMX_PREFILL_F16>, dim3((unsigned)blocks), dim3(kPfThreads), kPfLds, st, k);
  else
    hipLaunchKernelGGL(prefill_kernel<BMX_PREFILL_BF16>, dim3((unsigned)blocks), dim3(kPfThreads), kPfLds, st, k);
  if (hipGetLastError() != hipSuccess) return pf_fail(BMX_PREFILL_E_HIP, "kernel launch failed");
  if (S > 1) {
    PfCombineArgs c{};
    c.part_o = k.part_o;
    c.part_ml = k.part_ml;
    c.out = k.out;
    c.G = k.G;
    c.n_q = k.n_q;
    c.R = k.R;
    c.n_split = S;
    const dim3 grid((unsigned)((k.R + 7) / 8), (unsigned)a->h_kv);
    if (a->dtype == BMX_PREFILL_F16)
      hipLaunchKernelGGL(prefill_combine_kernel<BMX_PREFILL_F16>, grid, dim3(256), 0, st, c);
    else
      hipLaunchKernelGGL(prefill_combine_kernel<BMX_PREFILL_BF16>, grid, dim3(256), 0, st, c);
    if (hipGetLastError() != hipSuccess) return pf_fail(BMX_PREFILL_E_HIP, "combine launch failed");
  }
  return 0;
}
