// Split-KV decode attention over packed k2b pages, gfx950.
//
// Two launches per call.
//
// k2b_decode_split_kernel: one workgroup of 8 waves per (split, sequence); wave
// w owns KV head w, and all waves walk the same 64-token groups (4 pages, one
// key-scale group) of the split's balanced share of the packed tokens:
//   * each wave streams its head's slice of every page (3-bit key residual and
//     2-bit value codes, 20 bytes per lane per page, 83% of the page bytes)
//     straight into VGPRs: all loads of the next group are issued at the top
//     of a group and first waited on at its end; page bytes are read once, so
//     every page load is non-temporal (streamed past the L2, which keeps the
//     kernel's code, arguments, basis and tables: ~1.7 us per 64k call);
//   * the page prefix every head reads (Us, value norms, key scales) is loaded
//     cooperatively two groups ahead and staged in a three-slot LDS ring; when
//     the prologue made every group's RoPE table, the waves hand the ring on
//     with LDS counters instead of a barrier per group, so a wave may run a
//     group ahead of the slowest;
//   * the RoPE cos/sin of the group's 64 positions is produced once per
//     workgroup, one group ahead (angle-addition recurrence from an exact start,
//     corrected to HF's fp32 angle fl(inv_freq * pos)), as fp16 pairs in LDS
//     shared by all heads;
//   * per page and head the wave rebuilds K^T (128 ch x 16 tok) on MFMA
//     (8 x mfma(V_h tile, Us^T)); lane 16q+n then holds token n, channels
//     j = 16b+4q+i and j+64 (b, i < 4), i.e. 16 RoPE pairs, which it converts to
//     packed fp16, adds residual*scale with one packed FMA per pair (3-bit codes
//     turned into fp16 integers by a mantissa/exponent trick, no per-code
//     convert), rotates with two packed ops per pair, and scores the G query
//     heads on MFMA;
//   * the 4 pages' score tiles (G useful columns of 16 each) are compacted into
//     one register set with DPP row shifts, so the online softmax runs once per
//     group on fully used lanes; the accumulator is rescaled only when a
//     running max grows;
//   * P*norm is accumulated against the fp16 codebook levels on MFMA (V stays
//     in the Hadamard-rotated domain), two pages per product; the levels are
//     looked up four codes (one code byte) at a time in a 256-entry LDS table;
//   * at the end, the accumulator is half un-rotated in registers: the
//     128-point Hadamard factors as H8 (over the 16-channel chunks) x H16
//     (within a chunk), and the split kernel applies H8;
//   * the workgroups that own a 16-token tile of the fp16 recent window score
//     it on MFMA (decode_shared.h) after their group loop, on waves 0-3: of
//     the two waves of a SIMD (w, w + 4) the older wins issue arbitration and
//     ends its groups ~2 us before the younger, so the tiles fill that slack
//     instead of delaying the workgroup's first group; the two waves of a
//     SIMD also take turns at the higher issue priority page by page.
//
// combine_kernel<true> (decode_shared.h): one wave per (16-channel chunk,
// query head, sequence) merges the packed partials of its chunk (base-2 LSE),
// applies H16, the signs and 1/128, and joins the recent window from its
// scores and fp16 values; all of its first-round loads are issued before any
// reduction.
//
// Reference semantics: cache/triton_dequant_attention.py:863-1115 (kernel),
// 409-461 (merge), 324-360 (tail), 504-575 (finalize);
// cache/chunked_attention.py:398-530 (decode loop).

#include "k2b_common.h"
#include "decode_shared.h"
#include "k2b_general.h"

#include <algorithm>
#include <type_traits>
#include <cmath>
#include <cstring>
#include <mutex>

namespace bmx {

constexpr int kWaves = 8;                   // waves per workgroup; wave w = head w
constexpr int kThreads = 64 * kWaves;
constexpr int kGroupPages = kGroup / kPT;   // 4 pages per 64-token group
constexpr int kCsRow = 68;                  // dwords per position row of the cos/sin table
                                            // (64 + 4: rows start 4 banks apart)
constexpr int kCsBuf = kGroup * kCsRow;     // dwords per group table
constexpr int kPidWindow = 64;              // page ids held per lane-vector
constexpr int kCsMaxBufs = 8;               // RoPE table buffers at most (17 KB each)
constexpr int kRingSlots = 3;               // prefix ring: group g in slot g % 3
constexpr int kBufWord3 = 0x00020000;       // buffer descriptor word 3: raw 32-bit data


// The scalar arguments the prologue reads come first, contiguous, so that one
// round trip of wide scalar loads fetches them all (the big tables follow).
struct DecodeKArgs {
  int h_kv, G, max_splits, max_pages, max_packed_len, n_pool;
  int shared_bytes;    // page prefix read by every head: US, VNORM, KSCALE (multiple of 16)
  int cs_bufs;         // RoPE table buffers in LDS (groups produced in the prologue)
  int balanced;        // a ragged batch: workgroup w of the flat grid serves the
                       // sequence batch_shares() gives it (max_splits = the slots per row)
  int n_seq;
  // floor(n / max_splits) for n < 2^32 as (t + ((n - t) >> div_sh1)) >> div_sh2,
  // t = mulhi(n, div_magic) (Granlund-Montgomery); div_ok: split * groups < 2^32
  uint32_t div_magic;
  int div_sh1, div_sh2, div_ok;
  int io_dtype;
  float qscale_rope;   // sm_scale * log2(e) * rope_scaling (the cos/sin table is unscaled)
  uint32_t level_hi[4];   // fp16 bits of the value levels as used by the MFMA:
                          // hi_c = kappa * codebook_c + mu (+ < 1e-6 relative)
  float level_mu;         // mu (the merge divides by kappa)
  const void* q;       // [B][h_kv][G][128] in io_dtype
  uint16_t* ws_acc;    // [B][h_kv][G][8][max_splits][16] partial records (H8 applied; decode_shared.h)
  float* ws_ml;        // [B][h_kv][G][max_splits][2]     (running max, sum), base 2
  const uint8_t* pages;
  const int32_t* page_table;
  const int32_t* packed_len;
  const uint16_t* basis;
  int64_t basis_stride;
  PageLayout L;
  float inv_freq[64];
  float step_c[64];    // cos / sin of 64 * inv_freq_j (exact angle), the per-group step
  float step_s[64];
  float step8_c[64];   // cos / sin of 8 * inv_freq_j, between a thread's positions
  float step8_s[64];
  // recent window: fp16 (or bf16: tail_bf16) post-RoPE keys [b * ts_b + h * ts_h + t * ts_t][128]
  const uint16_t* k_tail;
  int64_t ts_b, ts_h, ts_t;
  int tail_bf16;
  WinNew nw;           // the window's newest rows given apart (decode_shared.h)
  int tail_cap;
  float win_rescale;      // 1 / rope_scaling: window keys carry the RoPE scaling
  float* ws_win;          // [B][h_kv][G][tail_cap] window scores, base 2
};

// v_mov_b32_dpp: lanes enabled by BANK (4-lane banks of each 16-lane row) take
// src from the DPP-selected lane, the others keep old.
template <int CTRL, int BANK = 0xF>
__device__ __forceinline__ float dpp(float old, float src) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old),
                                                               __builtin_bit_cast(int, src), CTRL, 0xF,
                                                               BANK, false));
}
constexpr int kRowShr = 0x110;  // + n: lane i of a row reads lane i - n
constexpr int kRowRor = 0x120;  // + n: rotate within the row

// x from the DPP-selected lane, every lane written (foldable into a DPP ALU op).
template <int CTRL>
__device__ __forceinline__ float dpp_all(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

// RoPE of one packed pair (k_j, k_{j+64}) by the packed (cos, sin):
// (k_j c - k_{j+64} s, k_{j+64} c + k_j s) in two packed ops.
__device__ __forceinline__ half2_t rope2(half2_t p, uint32_t csu) {
  const half2_t cs = as_h2(csu);
  const half2_t cc = {cs[0], cs[0]};
  const half2_t sn = {-cs[1], cs[1]};
  const half2_t sw = {p[1], p[0]};
  return __builtin_elementwise_fma(sw, sn, p * cc);
}

// Partial (acc, m, l) of this lane's query into the workspace.  w_run is the
// lane's sum of the fp16 P*norm operands, for the level correction.  The
// rotated accumulator is half un-rotated here: the 128-point Sylvester Hadamard of
// channel c = 16bt + 4q + i factors as H8 (over bt) x H16 (over 4q + i); the
// H8 butterflies run in registers, and the merge kernel, which holds whole
// 16-channel chunks, applies H16, the signs and 1/128 after the merge (both
// linear).  Lane 16q + n stores acc[bt] at offset 4q of chunk bt.  The workspace
// row of a query is chunk-major ([chunk][split][16]), so a merge workgroup
// reads one contiguous 64-byte record per split.
__device__ __forceinline__ void store_partial(const DecodeKArgs& a, int b, int split, int h, int n,
                                              int q, float4_t acc[8], float m_run, float l_run,
                                              float w_run) {
  l_run += __shfl_xor(l_run, 16);
  l_run += __shfl_xor(l_run, 32);
  w_run += __shfl_xor(w_run, 16);
  w_run += __shfl_xor(w_run, 32);
#pragma unroll
  for (int hb = 1; hb < 8; hb <<= 1)
#pragma unroll
    for (int bt = 0; bt < 8; ++bt)
      if (!(bt & hb)) {
        const float4_t u = acc[bt], w = acc[bt | hb];
        acc[bt] = u + w;
        acc[bt | hb] = u - w;
      }
  // the levels were hi = kappa * level + mu: remove mu * sum(P*norm) from every
  // channel, which after H8 is 8 mu W on chunk 0 (the merge divides by kappa)
  const float corr = 8.0f * a.level_mu * w_run;
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[0][i] -= corr;
  if (n < a.G)
    store_partial_record(a.ws_acc, a.ws_ml, ((int64_t)b * a.h_kv + h) * a.G + n, a.max_splits, split, q, acc,
                         m_run, l_run);
}

// The recent window is scored in (16-token tile, head) pairs: pair
// p = tile * h_kv + head goes to split p mod S, and a split's k-th pair to
// its wave k mod nw (after the group loop: waves 0-3, which end their groups
// first; in a split with no packed tokens: any wave).  Each pair is one
// memory round trip (the head's query rows and the tile's rows together), so
// a wave that owns one pair ends one round trip after its groups.
__device__ __forceinline__ void score_win_pairs(const DecodeKArgs& a, int b, int split, int S, int wave, int nw,
                                                int n, int q) {
  const int n_pairs = ((a.tail_cap + 15) >> 4) * a.h_kv;
  for (int p = split + wave * S; p < n_pairs; p += nw * S) {
    const int j = p / a.h_kv, hh = p - j * a.h_kv;
    const int64_t qrow = (((int64_t)b * a.h_kv + hh) * a.G + (n < a.G ? n : 0)) * kD;
    const int64_t tb = (int64_t)b * a.ts_b + (int64_t)hh * a.ts_h;
    float4_t qraw[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) qraw[u] = load_q4(a.q, qrow + 16 * (u & 3) + 4 * q + 64 * (u >> 2), a.io_dtype);
    uint2 kw[8];
    load_win_tile(a, tb, j, n, q, kw, (int64_t)b * a.nw.sb + (int64_t)hh * a.nw.sh);
    half8_t qh[4], ql[4];
    window_fragments(qraw, n < a.G ? a.qscale_rope : 0.0f, a.tail_bf16, qh, ql);
    score_win_tile(a, b, hh, j, n, q, kw, qh, ql, tb);
  }
}

// R: key rank (16 or 32).  SW: query slot width (G rounded up to 4, 8 or 16);
// the 16 score columns of a page hold 16/SW pages after compaction.
template <int R, int SW, bool CONTIG>
__global__ __launch_bounds__(kThreads) void k2b_decode_split_kernel(const DecodeKArgs a) {
  constexpr int NSLOT = 16 / SW;             // pages per compacted score register
  constexpr int NCR = kGroupPages / NSLOT;   // compacted registers per group
  constexpr int KQ = R / 4;                  // rank elements per lane in the K^T MFMA
  typedef _Float16 hvec_t __attribute__((ext_vector_type(KQ)));
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  // MFMA value levels (fp16 hi_c) of the 4 codes of one VCODE byte:
  // s_vlut[v] = {lv(c0) | lv(c1) << 16, lv(c2) | lv(c3) << 16}, c_t = (v >> 2t) & 3
  // (static LDS: the byte index scales straight into the address)
  __shared__ uint2 s_vlut[256];
  // hand-off of the prefix ring between waves, no workgroup barrier per group:
  // s_sync[s] counts the waves that have stored a group's prefix into ring slot
  // s, s_sync[3 + s] the waves done reading a group from slot s (monotonic:
  // slot s serves groups s, s + 3, ...); s_tab[t] counts the waves that have
  // made their rows of a RoPE table in buffer t after the prologue (buffer t
  // serves groups t, t + cs_bufs, ...)
  __shared__ uint32_t s_sync[2 * kRingSlots];
  __shared__ uint32_t s_tab[kCsMaxBufs];
  // every scalar argument of the prologue requested at once, at the top: one
  // round trip of wide scalar loads instead of a chain of them behind the
  // prologue's branches
  asm volatile("" ::"s"(a.h_kv), "s"(a.G), "s"(a.max_splits), "s"(a.max_pages), "s"(a.max_packed_len),
               "s"(a.n_pool), "s"(a.shared_bytes), "s"(a.cs_bufs), "s"(a.balanced), "s"(a.n_seq),
               "s"(a.div_magic), "s"(a.div_sh1), "s"(a.div_sh2), "s"(a.div_ok), "s"(a.io_dtype));
  asm volatile("" ::"s"(a.q), "s"(a.pages), "s"(a.page_table), "s"(a.packed_len), "s"(a.basis),
               "s"(a.basis_stride), "s"(a.L.bytes), "s"(a.L.kres), "s"(a.L.vcode));
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int n = lane & 15;   // token within page (K side) / score column (softmax side)
  const int q = lane >> 4;   // quarter
  const bool active = wave < a.h_kv;
  const int h = active ? wave : 0;
  // this workgroup's sequence b, split and the sequence's split count S: the
  // grid's (x, y), or, for a ragged batch, the workgroup's place in the
  // length-proportional shares of the flat grid (read from the lengths)
  int split = blockIdx.x, b = blockIdx.y, S = a.max_splits;
  int len_known = -1;
  if (a.balanced) {
    int share, first, len_l;
    batch_shares(a.packed_len, a.max_packed_len, a.n_seq, gridDim.x, share, first, len_l);
    const uint64_t mine = __ballot(share > 0 && (int)blockIdx.x >= first && (int)blockIdx.x < first + share);
    if (mine == 0) return;   // a workgroup past every share: nothing to do
    b = __builtin_ctzll(mine);
    split = blockIdx.x - __shfl(first, b);
    S = __shfl(share, b);
    len_known = __shfl(len_l, b);
  }

  // ---- every load that depends only on the arguments is issued first, the
  // page-table read first of all, and nothing is used before the first group's
  // page loads are in flight (a wait on one load waits on all earlier ones) ----
  const int fj = tid & 63;   // RoPE frequency this thread produces
  const int len_spec = len_known >= 0 ? len_known : a.max_packed_len & ~(kGroup - 1);
  auto range = [&](int L, int& r0, int& r1) {
    const int NG = L / kGroup;
    if (!a.balanced && a.div_ok) {
      // uniform operands in scalar registers: no 64-bit divide on the vector unit
      const uint32_t ng = (uint32_t)__builtin_amdgcn_readfirstlane(NG);
      const uint32_t sp = (uint32_t)__builtin_amdgcn_readfirstlane(split);
      auto div = [&](uint32_t n) -> int {
        const uint32_t t = __umulhi(n, a.div_magic);
        return (int)((t + ((n - t) >> a.div_sh1)) >> a.div_sh2);
      };
      r0 = div(sp * ng);
      r1 = div((sp + 1) * ng);
    } else {
      r0 = (int)(((int64_t)split * NG) / S);
      r1 = (int)(((int64_t)(split + 1) * NG) / S);
    }
  };
  int g0, g1;
  range(len_spec, g0, g1);
  // no page table: the sequence's pages are contiguous, logical page i of
  // sequence b at physical page b * max_pages + i (the page ids are computed,
  // so the first pages are requested at once, with no table round trip)
  // (a template parameter: a guarded table load joined with another path
  // would make the compiler wait on it right away)
  constexpr bool contig = CONTIG;
  const int32_t* ptab_row = contig ? nullptr : a.page_table + (int64_t)b * a.max_pages;
  // Balanced static partition of the sequence's 64-token groups over the
  // max_splits workgroups.  The page ids (a page-table read) are taken for the
  // host bound max_packed_len before the device length arrives, and taken
  // again in the rare case that the sequence is shorter.
  // ids of pages first .. first+63 of the range; an empty range reads the
  // (valid) length word instead, so the load has no branch to wait in
  auto load_ids_raw = [&](int first, int count) -> int {
    if constexpr (contig) return b * a.max_pages + g0 * kGroupPages + min(first + lane, max(count - 1, 0));
    const int32_t* src = count > 0 ? ptab_row + g0 * kGroupPages + min(first + lane, count - 1)
                                   : a.packed_len + b;
    return (int)*src;
  };
  // the RoPE table constants first: the table production below waits for them
  // alone (loads complete in issue order), not for the page table
  const float fq = a.inv_freq[fj];
  const float c8 = a.step8_c[fj], s8 = a.step8_s[fj];
  const float stc = a.step_c[fj], sts = a.step_s[fj];
  // keep those loads ahead of every later one (loads complete in issue order,
  // and the table production must not wait for the basis or the pages)
  __builtin_amdgcn_sched_barrier(0);
  const int pid_raw = load_ids_raw(0, (g1 - g0) * kGroupPages);
  const int len_raw = a.packed_len[b];
  hvec_t vh[8];
  const uint16_t* basis = a.basis + (int64_t)b * a.basis_stride;
#pragma unroll
  for (int bt = 0; bt < 8; ++bt)
    vh[bt] = *reinterpret_cast<const hvec_t*>(basis + (int64_t)(h * kD + 16 * bt + n) * R + KQ * q);
  float4_t qraw[8];   // q_n[16bb + 4q .. +3] (u = bb) and [.. + 64] (u = 4 + bb)
  {
    const int64_t qrow = (((int64_t)b * a.h_kv + h) * a.G + (n < a.G ? n : 0)) * kD;
#pragma unroll
    for (int u = 0; u < 8; ++u) qraw[u] = load_q4(a.q, qrow + 16 * (u & 3) + 4 * q + 64 * (u >> 2), a.io_dtype);
  }
  // dynamic LDS: the cos/sin tables, then the prefix ring
  const int cs_bufs = a.cs_bufs;
  uint32_t* cst = reinterpret_cast<uint32_t*>(smem);                            // [cs_bufs][64][kCsRow]
  int t_begin = g0 * kGroup;
  // ---- RoPE table: fp16 (cos, sin) of HF's angle fl(fq * pos) for 64
  // positions per group, row = position, column = frequency, one LDS buffer per
  // group for the first cs_bufs groups, all written here, while the page table
  // and then the first pages are in flight.  This thread owns frequency j = tid & 63
  // at group-local positions wave + 8k, k < 8.  Angles: one exact start (the
  // angle in revolutions from the exact product, scaled in double; its
  // fraction; the hardware sin/cos of revolutions), then 8-position and
  // 64-position rotation steps, each value corrected to the fp32 angle ----
  auto produce_groups = [&](int g_first, int count, int buf_first) {
    float cc[8], ss[8];
    const int t_first = t_begin + g_first * kGroup + wave;
    const double rev = (double)fq * (double)t_first * 0.15915494309189535;
    const float fr = (float)(rev - floor(rev));
    cc[0] = __builtin_amdgcn_cosf(fr);
    ss[0] = __builtin_amdgcn_sinf(fr);
#pragma unroll
    for (int k = 1; k < 8; ++k) {
      cc[k] = cc[k - 1] * c8 - ss[k - 1] * s8;
      ss[k] = ss[k - 1] * c8 + cc[k - 1] * s8;
    }
    float tf0 = (float)t_first;   // positions below 2^24: every step exact
    int buf = buf_first % cs_bufs;
    for (int g = 0; g < count; ++g) {
      uint32_t* dst = cst + buf * kCsBuf + wave * kCsRow + fj;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float tf = tf0 + (float)(8 * k);
        const float ang = fq * tf;
        const float e = __builtin_fmaf(fq, tf, -ang);  // exact: fq*tf - fl(fq*tf)
        const half2_t v = {(_Float16)__builtin_fmaf(ss[k], e, cc[k]),
                           (_Float16)__builtin_fmaf(-cc[k], e, ss[k])};
        dst[8 * k * kCsRow] = as_u32(v);
        const float cn = cc[k] * stc - ss[k] * sts;
        ss[k] = ss[k] * stc + cc[k] * sts;
        cc[k] = cn;
      }
      tf0 += (float)kGroup;
      buf = buf + 1 == cs_bufs ? 0 : buf + 1;
    }
  };
  auto load_ids = [&](int first, int count) { return (int)clamp_page(load_ids_raw(first, count), a.n_pool); };
  const int C = kD * a.h_kv;
  const int quarter = C / 4;
  const int pb = a.L.bytes;
  const int SHB = a.shared_bytes;
  const int sh_chunks = SHB / 4;       // 16-byte chunks of the 4 pages' prefixes
  const int chunks_pp = SHB / 16;
  uint8_t* ring = smem + cs_bufs * kCsBuf * 4;                                  // [3][4][SHB]
  // page ids of the range, a window of 64 per lane-vector
  int pidv = contig ? load_ids(0, (g1 - g0) * kGroupPages) : 0;
  int pid_base = 0;
  auto page_ptr = [&](int gi, int pp) -> const uint8_t* {   // uniform (gi, pp)
    const int id = __builtin_amdgcn_readlane(pidv, gi * kGroupPages + pp - pid_base);
    return a.pages + (int64_t)id * pb;
  };
  // thread tid's 16 B of the prefixes (threads past the last chunk re-read the
  // last one: an unconditional load leaves no branch to wait in)
  auto load_prefix = [&](int gi) -> uint4 {
    const int c = min(tid, sh_chunks - 1);
    const int pp = c / chunks_pp;
    const int id = __shfl(pidv, gi * kGroupPages + pp - pid_base);
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(a.pages + (int64_t)id * pb + (c - pp * chunks_pp) * 16));
    return make_uint4(v[0], v[1], v[2], v[3]);
  };
  auto store_prefix = [&](uint4 v, int slot) {
    if (tid < sh_chunks) *reinterpret_cast<uint4*>(ring + slot * kGroupPages * SHB + tid * 16) = v;
  };
  // uniform page base + 32-bit lane offset: the scalar-base load form
  const uint32_t kres_off = (uint32_t)(a.L.kres + h * 768 + lane * 12);
  const uint32_t vcode_off = (uint32_t)(a.L.vcode + h * 512 + lane * 8);
  typedef uint32_t u32x3_t __attribute__((ext_vector_type(3)));
  // a page's sections through a buffer descriptor on its (uniform) base: the
  // address is scalar work, the lane offset a constant register, and the load
  // is non-temporal (aux 2)
  auto page_rsrc = [&](int gi, int pp) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(page_ptr(gi, pp)), (short)0, pb, kBufWord3);
  };
  auto load_kres = [&](int gi, int pp) -> uint3 {
    const u32x3_t v = __builtin_amdgcn_raw_buffer_load_b96(page_rsrc(gi, pp), (int)kres_off, 0, 2);
    return make_uint3(v[0], v[1], v[2]);
  };
  auto load_vcode = [&](int gi, int pp) -> uint2 {
    const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(page_rsrc(gi, pp), (int)vcode_off, 0, 2);
    return make_uint2(v[0], v[1]);
  };

  // ---- first group in flight: at once for contiguous pages (for the host
  // bound, before the tables are made), else after the page-table read ----
  uint4 pre, pre1;
  uint3 kres[kGroupPages];   // this group's codes (the next group's are fetched
  uint2 vcd[kGroupPages];    // into separate registers at the top of the group)
  auto issue_first = [&](int ng) {
    pre = load_prefix(0);
    pre1 = load_prefix(min(1, ng - 1));
#pragma unroll
    for (int pp = 0; pp < kGroupPages; ++pp) {
      kres[pp] = load_kres(0, pp);
      vcd[pp] = load_vcode(0, pp);
    }
  };
  if (contig && g1 > g0) issue_first(g1 - g0);

  // the tables of the range for the host bound, made while the page table (or
  // the first pages) are in flight; remade below in the rare case that the
  // sequence is shorter
  produce_groups(0, min(g1 - g0, cs_bufs), 0);

  if (!contig) pidv = (int)clamp_page(pid_raw, a.n_pool);
  // the length and the range are wave-uniform: held in scalar registers, the
  // loop's bookkeeping on them is scalar work
  const int len = __builtin_amdgcn_readfirstlane(min(len_raw, a.max_packed_len) & ~(kGroup - 1));
  if (len != len_spec) {
    range(len, g0, g1);
    pidv = load_ids(0, (g1 - g0) * kGroupPages);
    t_begin = g0 * kGroup;
    produce_groups(0, min(g1 - g0, cs_bufs), 0);
    if (contig && g1 > g0) issue_first(g1 - g0);
  }
  // a workgroup with no packed tokens runs no group: its window pairs, then an
  // empty partial (max -inf, zeros) that the merge ignores
  g0 = __builtin_amdgcn_readfirstlane(g0);
  g1 = __builtin_amdgcn_readfirstlane(g1);
  const int n_groups = g1 - g0;
  if (!contig && n_groups > 0) issue_first(n_groups);
  const int n_pages = n_groups * kGroupPages;

  if (tid < 256) {
    const uint32_t l0 = a.level_hi[0], l1 = a.level_hi[1], l2 = a.level_hi[2], l3 = a.level_hi[3];
    auto lv = [&](int c) { return c == 0 ? l0 : c == 1 ? l1 : c == 2 ? l2 : l3; };
    s_vlut[tid] = make_uint2(lv(tid & 3) | (lv((tid >> 2) & 3) << 16), lv((tid >> 4) & 3) | (lv(tid >> 6) << 16));
  }

  // query fragments (qf: the MFMA B operand of the packed pages; the low parts
  // are unused here: the window tiles remake both after the loop)
  half8_t qf[4], qlo[4];
  query_fragments(qraw, (n < a.G) ? a.qscale_rope : 0.0f, qf, qlo);

  store_prefix(pre, 0);
  store_prefix(pre1, 1);
  // slots 0 and 1 hold groups 0 and 1 (visible at the barrier)
  if (tid < 2 * kRingSlots) s_sync[tid] = tid < 2 ? kWaves : 0;
  if (tid < kCsMaxBufs) s_tab[tid] = 0;

  // ---- per-wave state ----
  float4_t acc[8];
#pragma unroll
  for (int bt = 0; bt < 8; ++bt) acc[bt] = float4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f, w_run = 0.0f;
  const int my_slot = NSLOT > 1 ? n / SW : 0;   // page slot of this lane after compaction
  KresMasks km;
  km.init();
  __syncthreads();   // LUT, table 0 and prefix slot 0 are visible
  // Group 0's codes must have landed before the loop: the compiler's wait
  // tracking merges the loop entry with the back edge, and a load still pending
  // on a current-group register at entry would make every group's key side wait
  // on the next group's loads (issued at the top of the same group).
  __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)

  // waves hand the prefix ring and the RoPE table buffers on through LDS
  // counters and may drift apart by up to a group: a range longer than the
  // prologue's tables (cs_bufs groups) remakes each buffer once every wave is
  // done with its group, each wave its own rows, at the end of the next group
  for (int gi = 0; gi < n_groups; ++gi) {
    const int gn = min(gi + 1, n_groups - 1);   // group whose codes are fetched during this one
    const int gp = min(gi + 2, n_groups - 1);   // group whose prefix is fetched during this one
    if ((gp + 1) * kGroupPages - pid_base > kPidWindow) {   // slide the page-id window
      pid_base = gn * kGroupPages;
      pidv = load_ids(pid_base, n_pages);
    }
    // every load of group gn is issued here, a whole group before its first
    // use, and the prefix of group gn + 1 with them (the last groups fetch
    // nothing they would not use)
    uint4 pre_n = make_uint4(0u, 0u, 0u, 0u);
    if (gi + 2 < n_groups) pre_n = load_prefix(gp);
    uint3 kres_n[kGroupPages];
    uint2 vcd_n[kGroupPages];
    if (active && gi + 1 < n_groups) {   // the last group fetches nothing more
#pragma unroll
      for (int pp = 0; pp < kGroupPages; ++pp) {
        kres_n[pp] = load_kres(gn, pp);
        vcd_n[pp] = load_vcode(gn, pp);
      }
    }
    // every wave has stored this group's prefix (use gi / 3 of slot gi % 3),
    // and past the prologue's tables made its rows of this group's table
    const int slot = gi % kRingSlots;
    wait_count(&s_sync[slot], kWaves * (gi / kRingSlots + 1));
    if (gi >= cs_bufs) wait_count(&s_tab[gi % cs_bufs], kWaves * (gi / cs_bufs));

    if (active) {
      const uint8_t* grp = ring + slot * kGroupPages * SHB;
      const uint32_t* csb = cst + (gi % cs_bufs) * kCsBuf;
      // key-residual scale pairs (s_j, s_{j+64}), j = 16bb + 4q + i: 16 bytes
      // per bb in the group's prefix, read once per group
      uint32_t sv[4][4];
#pragma unroll
      for (int bb = 0; bb < 4; ++bb) {
        const int f = h * kD + 2 * (16 * bb + 4 * q);
        const int slot = f / quarter, off = f - slot * quarter;
        const uint4 s4 = *reinterpret_cast<const uint4*>(grp + slot * SHB + a.L.kscale + 2 * off);
        sv[bb][0] = s4.x; sv[bb][1] = s4.y; sv[bb][2] = s4.z; sv[bb][3] = s4.w;
      }
      // ---- K side: scores of the 4 pages, a (j, j + 64) slice at a time:
      // the slice's two key tiles, its 4 residual pairs, RoPE, one score MFMA ----
      float4_t sc[kGroupPages];
#pragma unroll
      for (int pp = 0; pp < kGroupPages; ++pp) {
        const uint8_t* pre_p = grp + pp * SHB;
        const hvec_t us = *reinterpret_cast<const hvec_t*>(pre_p + a.L.us + lane * (2 * KQ));
        const uint32_t w0 = kres[pp].x, w1 = kres[pp].y, w2 = kres[pp].z;
        float4_t s = {0.f, 0.f, 0.f, 0.f};
        auto slice = [&](auto bbc) {
          constexpr int bb = decltype(bbc)::value;
          const float4_t z = {0.f, 0.f, 0.f, 0.f};
          float4_t klo, khi;
          if constexpr (R == 32) {
            klo = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh[bb], us, z, 0, 0, 0);
            khi = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh[bb + 4], us, z, 0, 0, 0);
          } else {
            klo = __builtin_amdgcn_mfma_f32_16x16x16f16(vh[bb], us, z, 0, 0, 0);
            khi = __builtin_amdgcn_mfma_f32_16x16x16f16(vh[bb + 4], us, z, 0, 0, 0);
          }
          const uint4 c4 = *reinterpret_cast<const uint4*>(csb + (pp * kPT + n) * kCsRow + 16 * bb + 4 * q);
          const uint32_t cv[4] = {c4.x, c4.y, c4.z, c4.w};
          const half2_t cp[4] = {kres_pair<4 * bb + 0>(km, w0, w1, w2), kres_pair<4 * bb + 1>(km, w0, w1, w2),
                                 kres_pair<4 * bb + 2>(km, w0, w1, w2), kres_pair<4 * bb + 3>(km, w0, w1, w2)};
          union { half2_t h2[4]; half8_t v; } ka;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            half2_t pr = {(_Float16)klo[i], (_Float16)khi[i]};
            pr = __builtin_elementwise_fma(cp[i], as_h2(sv[bb][i]), pr);
            ka.h2[i] = rope2(pr, cv[i]);
          }
          s = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka.v, qf[bb], s, 0, 0, 0);
        };
        slice(std::integral_constant<int, 0>{});
        slice(std::integral_constant<int, 1>{});
        slice(std::integral_constant<int, 2>{});
        slice(std::integral_constant<int, 3>{});
        sc[pp] = s;
        // the two waves of a SIMD (w, w + 4) take turns at the higher issue priority
        if (((pp + (wave >> 2)) & 1) != 0) __builtin_amdgcn_s_setprio(1);
        else __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_sched_barrier(0);   // bound the cross-page overlap (VGPR budget)
      }
      // ---- compaction: page r*NSLOT + s moves to columns [s*SW, (s+1)*SW) ----
      float4_t cr[NCR];
#pragma unroll
      for (int r = 0; r < NCR; ++r) {
        cr[r] = sc[r * NSLOT];
        if constexpr (NSLOT == 4) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            cr[r][i] = dpp<kRowShr + 4, 0x2>(cr[r][i], sc[r * NSLOT + 1][i]);
            cr[r][i] = dpp<kRowShr + 8, 0x4>(cr[r][i], sc[r * NSLOT + 2][i]);
            cr[r][i] = dpp<kRowShr + 12, 0x8>(cr[r][i], sc[r * NSLOT + 3][i]);
          }
        } else if constexpr (NSLOT == 2) {
#pragma unroll
          for (int i = 0; i < 4; ++i) cr[r][i] = dpp<kRowShr + 8, 0xC>(cr[r][i], sc[r * NSLOT + 1][i]);
        }
      }
      // ---- online softmax over the group (one running max per query) ----
      float mx = -INFINITY;
#pragma unroll
      for (int r = 0; r < NCR; ++r)
        mx = fmaxf(mx, fmaxf(fmaxf(cr[r][0], cr[r][1]), fmaxf(cr[r][2], cr[r][3])));
      if (__any(mx > m_run)) {
        if constexpr (NSLOT == 4) mx = fmaxf(mx, dpp_all<kRowRor + 4>(mx));
        if constexpr (NSLOT >= 2) mx = fmaxf(mx, dpp_all<kRowRor + 8>(mx));
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        l_run *= alpha;
        w_run *= alpha;
#pragma unroll
        for (int bt = 0; bt < 8; ++bt) acc[bt] *= alpha;
        m_run = m_new;
      }
      // ---- P*norm of the lane's page (its slot), tokens 4q..4q+3, fp16 ----
      uint2 pd[NCR];
#pragma unroll
      for (int r = 0; r < NCR; ++r) {
        const int pg = r * NSLOT + my_slot;
        const uint2 nr = *reinterpret_cast<const uint2*>(grp + pg * SHB + a.L.vnorm + h * 32 + q * 8);
        const float nv[4] = {half_bits_to_float(nr.x & 0xffff), half_bits_to_float(nr.x >> 16),
                             half_bits_to_float(nr.y & 0xffff), half_bits_to_float(nr.y >> 16)};
        float x[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = __builtin_amdgcn_exp2f(cr[r][i] - m_run);
          l_run += p;
          x[i] = p * nv[i];
        }
        const half2_t h01 = {(_Float16)x[0], (_Float16)x[1]}, h23 = {(_Float16)x[2], (_Float16)x[3]};
        const half2_t one2 = {(_Float16)1.0f, (_Float16)1.0f};
        w_run = __builtin_amdgcn_fdot2(h23, one2, __builtin_amdgcn_fdot2(h01, one2, w_run, false), false);
        pd[r] = make_uint2(as_u32(h01), as_u32(h23));
      }
      // ---- P.V on MFMA, two pages per product: K index 8q + j is token
      // 4q + (j & 3) of page 2u + (j >> 2), so the A operand is the two pages'
      // code bytes of the tile through the level table, and the B operand is the
      // lane's own P*norm in the half of its page (zero for the other page) ----
#pragma unroll
      for (int u = 0; u < kGroupPages / 2; ++u) {
        const int pa = 2 * u, pb = 2 * u + 1;
        const uint2 za = (NSLOT == 1 || my_slot == pa % NSLOT) ? pd[pa / NSLOT] : make_uint2(0u, 0u);
        const uint2 zb = (NSLOT == 1 || my_slot == pb % NSLOT) ? pd[pb / NSLOT] : make_uint2(0u, 0u);
        union { uint4 e; half8_t v; } bp;
        bp.e = make_uint4(za.x, za.y, zb.x, zb.y);
        const uint2 va_ = vcd[pa], vb_ = vcd[pb];
        union { uint4 e; half8_t v; } av[8];
#pragma unroll
        for (int bt = 0; bt < 8; ++bt) {
          const uint32_t Da = bt < 4 ? va_.x : va_.y, Db = bt < 4 ? vb_.x : vb_.y;
          const uint2 la = s_vlut[(Da >> (8 * (bt & 3))) & 0xFFu];
          const uint2 lb = s_vlut[(Db >> (8 * (bt & 3))) & 0xFFu];
          av[bt].e = make_uint4(la.x, la.y, lb.x, lb.y);
        }
#pragma unroll
        for (int bt = 0; bt < 8; ++bt)
          acc[bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[bt].v, bp.v, acc[bt], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // the prefix of group gi + 2 goes to slot (gi + 2) % 3 and the table of
    // group gi - 1 + cs_bufs to buffer (gi - 1) % cs_bufs: both last read by
    // group gi - 1, once every wave is done with it
    const int slot2 = (gi + 2) % kRingSlots;
    count_wave(&s_sync[kRingSlots + slot]);   // done reading group gi (prefix and table)
    const bool refill = gi >= 1 && gi - 1 + cs_bufs < n_groups;
    if (gi >= 1 && (gi + 2 < n_groups || refill))
      wait_count(&s_sync[kRingSlots + slot2], kWaves * ((gi - 1) / kRingSlots + 1));
    if (gi + 2 < n_groups) {
      store_prefix(pre_n, slot2);
      count_wave(&s_sync[slot2]);
    }
    if (refill) {
      produce_groups(gi - 1 + cs_bufs, 1, gi - 1);
      count_wave(&s_tab[(gi - 1) % cs_bufs]);
    }
    if (active) {
#pragma unroll
      for (int pp = 0; pp < kGroupPages; ++pp) {
        kres[pp] = kres_n[pp];
        vcd[pp] = vcd_n[pp];
      }
    }
  }
  // the window pairs this workgroup owns, on waves 0-3: of the two waves of a
  // SIMD (w, w + 4) these finish their groups first
  if (wave < 4) score_win_pairs(a, b, split, S, wave, 4, n, q);
  if (active) {
    // fold the page slots: column s*SW + g -> g
    if constexpr (NSLOT == 4) {
#pragma unroll
      for (int bt = 0; bt < 8; ++bt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[bt][i] += dpp_all<kRowRor + 4>(acc[bt][i]);
      l_run += dpp_all<kRowRor + 4>(l_run);
      w_run += dpp_all<kRowRor + 4>(w_run);
    }
    if constexpr (NSLOT >= 2) {
#pragma unroll
      for (int bt = 0; bt < 8; ++bt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[bt][i] += dpp_all<kRowRor + 8>(acc[bt][i]);
      l_run += dpp_all<kRowRor + 8>(l_run);
      w_run += dpp_all<kRowRor + 8>(w_run);
    }
    store_partial(a, b, split, h, n, q, acc, m_run, l_run, w_run);
  }
}

}  // namespace bmx

using namespace bmx;

static int device_cu_count() { return bmx_device_cu_count(); }

// Workgroups per sequence: one wave of workgroups over the device's CUs (one
// 8-wave workgroup per CU), or as many as split_tokens asks for; never more
// than the sequence has 64-token groups, except that the recent window's
// 16-token score tiles get a workgroup each, up to one per CU.
// A ragged batch (2..64 sequences, no split_tokens, two CUs or more per
// sequence) runs balanced: one flat wave of workgroups over the CUs, each
// sequence a share proportional to its length (batch_shares); the partial
// slots per row are then the largest share, CUs - batch + 1.
static bool balanced_batch(const bmx_k2b_decode_args* a) {
  return a->batch > 1 && a->batch <= kMaxBalancedBatch && a->split_tokens == 0 &&
         device_cu_count() >= 2 * a->batch;
}

// Partial slots per row (the split count of a sequence, at most).
static int choose_splits(const bmx_k2b_decode_args* a) {
  if (balanced_batch(a)) return device_cu_count() - a->batch + 1;
  const int units = (a->max_packed_len + kGroup - 1) / kGroup;
  const int per_seq = std::max(1, device_cu_count() / a->batch);
  int S;
  if (a->split_tokens > 0)
    S = (a->max_packed_len + a->split_tokens - 1) / a->split_tokens;
  else
    S = per_seq;
  if (S > units) S = units;
  const int tiles = (a->tail_cap + 15) / 16;
  if (S < tiles) S = std::min(tiles, std::max(S, per_seq));
  return S < 1 ? 1 : S;
}

// Workspace: split partial records [B][h_kv][G][8][S][16] fp16, then (max,
// sum) [B][h_kv][G][S][2] fp32, then window scores [B][h_kv][G][tail_cap] fp32.
static size_t ws_bytes(const bmx_k2b_decode_args* a, int splits) {
  const size_t rows = (size_t)a->batch * a->geom.h_kv * a->geom.n_q_groups;
  return partial_bytes(rows, (size_t)splits) + rows * (size_t)a->tail_cap * sizeof(float);
}

extern "C" size_t bmx_k2b_decode_workspace_bytes(const bmx_k2b_decode_args* a) {
  if (!a || a->batch < 1) return 0;
  if (Geo::from(a->geom).general) return gen_decode_workspace(a);
  return ws_bytes(a, choose_splits(a));
}

// ---------------------------------------------------------------------------
// MFMA value levels.  The P.V product takes fp16 levels; plain rounding of the
// codebook leaves a per-level error of up to 2^-11 relative that does not
// average out over a long context.  Instead the levels are an affine image
// hi_c = kappa * level_c + mu (kappa in [1/2, 2]) chosen so that all four are
// fp16 numbers to within ~1e-6 relative: then sum_t w_t hi = kappa * (the exact
// sum) + mu * sum_t w_t, and the kernels undo mu and kappa exactly.  The map is
// found by a search over fp16 values for the two extreme levels (the two middle
// levels follow) and cached per codebook.
// ---------------------------------------------------------------------------
struct LevelMap {
  uint32_t hi[4];
  float kappa, mu;
  double err;   // max |hi_c - (kappa level_c + mu)| / max |kappa level|
};

static double round_half(double v) {   // nearest fp16 value (normal range), ties to even
  return (double)(_Float16)v;
}

static uint32_t half_bits_host(double v) {
  _Float16 h = (_Float16)v;
  uint16_t u;
  memcpy(&u, &h, 2);
  return u;
}

static LevelMap search_level_map(const float cb[4]) {
  LevelMap best{};
  best.err = 1e30;
  double L[4];
  for (int c = 0; c < 4; ++c) L[c] = cb[c];
  int ia = 0;
  for (int c = 1; c < 4; ++c)
    if (fabs(L[c]) > fabs(L[ia])) ia = c;
  const int ib = (ia == 0) ? 3 : 0;   // the other extreme (levels ascend)
  int io[2], k = 0;
  for (int c = 0; c < 4; ++c)
    if (c != ia && c != ib) io[k++] = c;
  const double La = L[ia], Lb = L[ib], amax = fabs(La);
  if (amax == 0.0 || La == Lb) {   // degenerate codebook: exact as it is
    for (int c = 0; c < 4; ++c) best.hi[c] = half_bits_host(L[c]);
    best.kappa = 1.f;
    best.mu = 0.f;
    best.err = 0.0;
    return best;
  }
  const double mu_max = 0.25 * amax;
  // g_a runs over the fp16 values of [amax/2, 2 amax] with the sign of La
  const uint16_t lo_bits = (uint16_t)(half_bits_host(0.5 * amax) & 0x7fff);
  const uint16_t hi_bits = (uint16_t)(half_bits_host(2.0 * amax) & 0x7fff);
  for (uint32_t ub = lo_bits; ub <= hi_bits; ++ub) {
    uint16_t u16 = (uint16_t)ub;
    _Float16 hv;
    memcpy(&hv, &u16, 2);
    const double ga = La < 0 ? -(double)hv : (double)hv;
    // mu = ga - kappa La within +-mu_max: kappa range, then the g_b range
    double k0 = (ga - mu_max) / La, k1 = (ga + mu_max) / La;
    if (k0 > k1) std::swap(k0, k1);
    k0 = std::max(k0, 0.5);
    k1 = std::min(k1, 2.0);
    if (k0 > k1) continue;
    double gb0 = ga + k0 * (Lb - La), gb1 = ga + k1 * (Lb - La);
    if (gb0 > gb1) std::swap(gb0, gb1);
    // walk the fp16 grid over [gb0, gb1]
    double g = round_half(gb0);
    for (int guard = 0; g <= gb1 && guard < 1 << 16; ++guard) {
      const double kap = (g - ga) / (Lb - La), mu = ga - kap * La;
      if (kap >= 0.5 && kap <= 2.0 && fabs(mu) <= mu_max && fabs(g) >= 6.2e-5) {
        double e = 0.0;
        for (int j = 0; j < 2; ++j) {
          const double v = kap * L[io[j]] + mu;
          e = std::max(e, fabs(v - round_half(v)));
        }
        e /= kap * amax;
        if (e < best.err) {
          best.err = e;
          best.kappa = (float)kap;
          best.mu = (float)mu;
          for (int c = 0; c < 4; ++c) best.hi[c] = half_bits_host(kap * L[c] + mu);
        }
      }
      // next fp16 value above g
      _Float16 gh = (_Float16)g;
      uint16_t gu;
      memcpy(&gu, &gh, 2);
      if (g >= 0) ++gu; else --gu;
      if ((gu & 0x7fff) == 0 && g < 0) gu = 0;
      memcpy(&gh, &gu, 2);
      g = (double)gh;
    }
  }
  return best;
}

static LevelMap level_map(const float cb[4]) {
  struct Entry {
    float cb[4];
    LevelMap m;
  };
  static std::mutex mu;
  static Entry cache[8];
  static int n_cached = 0, next_slot = 0;
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < n_cached; ++i)
    if (memcmp(cache[i].cb, cb, sizeof(cache[i].cb)) == 0) return cache[i].m;
  Entry& e = cache[next_slot];
  memcpy(e.cb, cb, sizeof(e.cb));
  e.m = search_level_map(cb);
  next_slot = (next_slot + 1) % 8;
  n_cached = std::min(n_cached + 1, 8);
  return e.m;
}

static int fail(int code, const std::string& msg) {
  bmx_set_error(msg);
  return code;
}

template <int R, int SW, bool CONTIG>
static hipError_t launch_split_sw(const DecodeKArgs& k, dim3 grid, size_t smem, hipStream_t st) {
  const hipError_t e = bmx_ensure_dynamic_lds((const void*)k2b_decode_split_kernel<R, SW, CONTIG>, smem);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((k2b_decode_split_kernel<R, SW, CONTIG>), grid, dim3(kThreads), smem, st, k);
  return hipGetLastError();
}

template <int R, bool CONTIG>
static hipError_t launch_split_c(const DecodeKArgs& k, dim3 grid, size_t smem, hipStream_t st) {
  if (k.G <= 4) return launch_split_sw<R, 4, CONTIG>(k, grid, smem, st);
  if (k.G <= 8) return launch_split_sw<R, 8, CONTIG>(k, grid, smem, st);
  return launch_split_sw<R, 16, CONTIG>(k, grid, smem, st);
}

template <int R>
static hipError_t launch_split(const DecodeKArgs& k, dim3 grid, size_t smem, hipStream_t st) {
  return k.page_table ? launch_split_c<R, false>(k, grid, smem, st) : launch_split_c<R, true>(k, grid, smem, st);
}

static int check_decode_args(const bmx_k2b_decode_args* a, const std::string& name);

// The split and merge launches of one decode call over the workspace ws
// (ws_cap bytes usable); name prefixes every error message.
static int decode_launch(const bmx_k2b_decode_args* a, void* stream, void* ws, size_t ws_cap,
                         const std::string& name);

extern "C" int bmx_k2b_decode(const bmx_k2b_decode_args* a, void* stream) {
  if (!a) return fail(BMX_E_INVALID, "bmx_k2b_decode: args is NULL");
  return decode_launch(a, stream, a->workspace, a->workspace_bytes, "bmx_k2b_decode");
}

// ---------------------------------------------------------------------------
// Allocation-free decode.  The partials live in a file-scope device array of
// BMX_K2B_DECODE_SCRATCH_BYTES (every GPU the library runs on holds its own
// copy until the process ends).  In host code the array's name is only a
// host-side stand-in: its device address is fetched once per device with
// hipGetSymbolAddress, with that device current, and only that address is
// ever passed to a kernel.  All calls on one GPU share the array: calls that
// overlap on one GPU (two streams, two threads) race.  Nothing needs clearing:
// a call writes every partial and window score it reads.
// ---------------------------------------------------------------------------
static __device__ __align__(256) uint8_t scratch[BMX_K2B_DECODE_SCRATCH_BYTES];

constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxScratchDevices];

static int scratch_address(void** out, std::string& err) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxScratchDevices) {
    err = std::string("no current HIP device in range: ") + hipGetErrorString(e);
    return BMX_E_HIP;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      err = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
      return BMX_E_HIP;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return BMX_OK;
}

extern "C" int bmx_k2b_decode_noalloc(const bmx_k2b_decode_args* a, void* stream) {
  if (!a) return fail(BMX_E_INVALID, "bmx_k2b_decode_noalloc: args is NULL");
  // the arguments first: an invalid geometry must not size the scratch
  if (const int rc = check_decode_args(a, "bmx_k2b_decode_noalloc")) return rc;
  const size_t need = bmx_k2b_decode_workspace_bytes(a);
  if (need > (size_t)BMX_K2B_DECODE_SCRATCH_BYTES)
    return fail(BMX_E_WORKSPACE, "bmx_k2b_decode_noalloc: this call needs " + std::to_string(need) +
                                     " bytes of partials, above the static scratch's " +
                                     std::to_string((size_t)BMX_K2B_DECODE_SCRATCH_BYTES) +
                                     " (use bmx_k2b_decode with a workspace)");
  void* ptr = nullptr;
  std::string err;
  const int rc = scratch_address(&ptr, err);
  if (rc != BMX_OK) return fail(rc, "bmx_k2b_decode_noalloc: " + err);
  return decode_launch(a, stream, ptr, (size_t)BMX_K2B_DECODE_SCRATCH_BYTES, "bmx_k2b_decode_noalloc");
}

// The argument checks of a decode call (before any sizing or launch); 0 or a
// BMX_E_INVALID code with the message set.
static int check_decode_args(const bmx_k2b_decode_args* a, const std::string& name) {
  const bmx_k2b_geom& g = a->geom;
  if (Geo::from(g).general) {   // the general page: its own geometry limits
    const std::string why = gen_decode_check(a);
    if (!why.empty()) return fail(BMX_E_INVALID, name + ": " + why);
  } else {
    if (g.h_kv < 1 || g.h_kv > kWaves) return fail(BMX_E_INVALID, name + ": h_kv must be 1..8");
    if (g.rank != 16 && g.rank != 32) return fail(BMX_E_INVALID, name + ": rank must be 16 or 32");
  }
  if (g.n_q_groups < 1 || g.n_q_groups > 16)
    return fail(BMX_E_INVALID, name + ": n_q_groups must be 1..16");
  if (a->batch < 1) return fail(BMX_E_INVALID, name + ": batch must be >= 1");
  if (a->max_packed_len < 0 || a->max_packed_len % kCodec != 0)
    return fail(BMX_E_INVALID, name + ": max_packed_len must be a multiple of 128");
  if (a->max_packed_len > 0 && a->max_pages * kPT < a->max_packed_len)
    return fail(BMX_E_INVALID, name + ": max_pages*16 < max_packed_len");
  if (a->tail_cap < 0 || a->tail_cap > 4096)
    return fail(BMX_E_INVALID, name + ": tail_cap must be 0..4096");
  if (!(a->rope_scaling > 0.0f) || !(a->rope_scaling < 1e30f))
    return fail(BMX_E_INVALID, name + ": rope_scaling must be finite and > 0");
  if (a->split_tokens < 0 || a->split_tokens % kGroup != 0)
    return fail(BMX_E_INVALID, name + ": split_tokens must be a multiple of 64");
  if (!a->q || !a->out || !a->packed_len)
    return fail(BMX_E_INVALID, name + ": q/out/packed_len must be non-NULL");
  if (a->io_dtype < BMX_K2B_IO_F32 || a->io_dtype > BMX_K2B_IO_BF16)
    return fail(BMX_E_INVALID, name + ": io_dtype must be BMX_K2B_IO_F32, _F16 or _BF16");
  if (a->tail_dtype != BMX_K2B_TAIL_F16 && a->tail_dtype != BMX_K2B_TAIL_BF16)
    return fail(BMX_E_INVALID, name + ": tail_dtype must be BMX_K2B_TAIL_F16 or _BF16");
  if (!a->tail_len && (a->tail_len_value < 0 || a->tail_len_value > a->tail_cap))
    return fail(BMX_E_INVALID, name + ": with tail_len NULL, tail_len_value must be 0..tail_cap");
  if (a->n_new < 0 || (a->n_new > 0 && (a->tail_len || a->n_new > a->tail_len_value || !a->new_k ||
                                        !a->new_v)))
    return fail(BMX_E_INVALID, name + ": n_new rows given apart need tail_len NULL, "
                                      "n_new <= tail_len_value and new_k/new_v non-NULL");
  if (a->n_new > 0 && (a->new_stride_b % 8 != 0 || a->new_stride_h % 8 != 0 || a->new_stride_t % 8 != 0))
    return fail(BMX_E_INVALID, name + ": new_k/new_v strides must be multiples of 8 elements");
  if (a->max_packed_len > 0 && (!a->pages || !a->basis))
    return fail(BMX_E_INVALID, name + ": pages/basis must be non-NULL");
  if (a->max_packed_len > 0 && a->n_pool_pages < 1)
    return fail(BMX_E_INVALID, name + ": n_pool_pages must be >= 1");
  if (a->tail_cap > 0 && (!a->k_tail || !a->v_tail))
    return fail(BMX_E_INVALID, name + ": k_tail/v_tail must be non-NULL when tail_cap > 0");
  if (a->tail_cap > 0 && (a->tail_stride_t % 8 != 0 || a->tail_stride_h % 8 != 0 ||
                          a->tail_stride_b % 8 != 0))
    return fail(BMX_E_INVALID, name + ": tail strides must be multiples of 8 elements");
  return BMX_OK;
}

static int decode_launch(const bmx_k2b_decode_args* a, void* stream, void* ws, size_t ws_cap,
                         const std::string& name) {
  const bmx_k2b_geom& g = a->geom;
  if (const int rc = check_decode_args(a, name)) return rc;
  if (Geo::from(g).general) return gen_decode(a, (hipStream_t)stream, ws, ws_cap, name);
  const int max_splits = choose_splits(a);
  const size_t need = ws_bytes(a, max_splits);
  if (max_splits > 8192)
    return fail(BMX_E_INVALID, name + ": more than 8192 splits; use a larger split_tokens");
  if (!ws || ws_cap < need)
    return fail(BMX_E_WORKSPACE, name + ": workspace missing or smaller than "
                                 "bmx_k2b_decode_workspace_bytes()");
  hipStream_t st = (hipStream_t)stream;
  const size_t rows = (size_t)a->batch * max_splits * g.h_kv * g.n_q_groups;
  uint16_t* ws_acc = (uint16_t*)ws;
  float* ws_ml = (float*)(ws_acc + rows * kD);
  float* ws_win = ws_ml + rows * 2;
  const float qscale = a->sm_scale * 1.4426950408889634f;

  DecodeKArgs k{};
  k.h_kv = g.h_kv; k.G = g.n_q_groups;
  k.max_splits = max_splits; k.max_pages = a->max_pages;
  k.max_packed_len = a->max_packed_len; k.n_pool = a->n_pool_pages > 0 ? a->n_pool_pages : 1;
  k.L = PageLayout::make(g.h_kv, g.rank);
  k.shared_bytes = k.L.kres;   // US, VNORM, KSCALE precede KRES
  k.q = a->q; k.io_dtype = a->io_dtype; k.ws_acc = ws_acc; k.ws_ml = ws_ml;
  k.pages = a->pages; k.page_table = a->page_table; k.packed_len = a->packed_len;
  k.basis = a->basis; k.basis_stride = a->basis_stride;
  k.qscale_rope = qscale * a->rope_scaling;
  k.k_tail = a->k_tail;
  k.ts_b = a->tail_stride_b; k.ts_h = a->tail_stride_h; k.ts_t = a->tail_stride_t;
  k.tail_bf16 = a->tail_dtype == BMX_K2B_TAIL_BF16;
  k.tail_cap = a->tail_cap;
  k.win_rescale = 1.0f / a->rope_scaling;
  k.ws_win = ws_win;
  k.nw.k = a->new_k; k.nw.v = a->new_v;
  k.nw.sb = a->new_stride_b; k.nw.sh = a->new_stride_h; k.nw.st = a->new_stride_t;
  k.nw.n = a->n_new;
  k.nw.T = a->tail_len ? -1 : a->tail_len_value;
  k.nw.k_dst = const_cast<uint16_t*>(a->k_tail);
  k.nw.v_dst = const_cast<uint16_t*>(a->v_tail);
  for (int j = 0; j < 64; ++j) {
    k.inv_freq[j] = a->inv_freq[j];
    const double step = 64.0 * (double)a->inv_freq[j];  // exact: 64 * fp32
    k.step_c[j] = (float)cos(step);
    k.step_s[j] = (float)sin(step);
    k.step8_c[j] = (float)cos(step / 8.0);
    k.step8_s[j] = (float)sin(step / 8.0);
  }
  for (int j = 0; j < 4; ++j)
    if (!(a->codebook[j] == a->codebook[j]) || (j > 0 && !(a->codebook[j] > a->codebook[j - 1])))
      return fail(BMX_E_INVALID, name + ": codebook must be 4 finite ascending levels");
  const LevelMap lm = level_map(a->codebook);
  if (lm.err > 4e-6)
    return fail(BMX_E_INVALID, name + ": no fp16 level map for this codebook (error " +
                                   std::to_string(lm.err) + ")");
  for (int j = 0; j < 4; ++j) k.level_hi[j] = lm.hi[j];
  k.level_mu = lm.mu;
  // RoPE tables for every group a workgroup owns, up to kCsMaxBufs (balanced:
  // the longest sequence gets at least 1 + (CUs - B) / B workgroups)
  const bool balanced = balanced_batch(a);
  const int n_wg = balanced ? device_cu_count() : max_splits * a->batch;
  const int least_share = balanced ? 1 + (n_wg - a->batch) / a->batch : max_splits;
  const int max_groups = ((a->max_packed_len / kGroup) + least_share - 1) / least_share;
  k.cs_bufs = std::max(1, std::min(max_groups, kCsMaxBufs));
  k.balanced = balanced ? 1 : 0;
  k.n_seq = a->batch;
  {
    // magic division by max_splits (Granlund-Montgomery, all 32-bit numerators)
    const uint32_t d = (uint32_t)max_splits;
    int l = 0;
    while ((1ull << l) < d) ++l;
    k.div_magic = (uint32_t)(((1ull << 32) * ((1ull << l) - d)) / d + 1);
    k.div_sh1 = l < 1 ? l : 1;
    k.div_sh2 = l > 1 ? l - 1 : 0;
    const uint64_t groups = (uint64_t)(a->max_packed_len / kGroup);
    k.div_ok = (uint64_t)d * (groups + 1) < (1ull << 32) ? 1 : 0;
  }
  const size_t smem = (size_t)k.cs_bufs * kCsBuf * 4 + (size_t)kRingSlots * kGroupPages * k.shared_bytes;
  const dim3 grid = balanced ? dim3(n_wg, 1) : dim3(max_splits, a->batch);
  hipError_t e = g.rank == 32 ? launch_split<32>(k, grid, smem, st)
                              : launch_split<16>(k, grid, smem, st);
  if (e != hipSuccess)
    return fail(BMX_E_HIP, name + std::string(": split kernel launch: ") + hipGetErrorString(e));
  if (a->split_end_event) {
    e = hipEventRecord((hipEvent_t)a->split_end_event, st);
    if (e != hipSuccess)
      return fail(BMX_E_HIP, name + std::string(": hipEventRecord: ") + hipGetErrorString(e));
  }
  CombineKArgs c{};
  c.h_kv = g.h_kv; c.G = g.n_q_groups;
  c.max_splits = max_splits; c.tail_cap = a->tail_cap;
  c.out = a->out; c.io_dtype = a->io_dtype; c.ws_acc = ws_acc; c.ws_ml = ws_ml; c.ws_win = ws_win;
  c.v_tail = a->v_tail;
  c.ts_b = a->tail_stride_b; c.ts_h = a->tail_stride_h; c.ts_t = a->tail_stride_t;
  c.tail_bf16 = k.tail_bf16;
  c.tail_len = a->tail_len;
  c.nw = k.nw;
  for (int j = 0; j < 4; ++j) c.v_sign_bits[j] = a->v_sign_bits[j];
  c.packed_scale = (float)(1.0 / (kD * (double)lm.kappa));
  c.balanced = k.balanced; c.n_wg = n_wg;
  c.packed_len = a->packed_len; c.max_packed_len = a->max_packed_len;
  launch_combine<true>(c, g.h_kv * g.n_q_groups, a->batch, st);
  e = hipGetLastError();
  if (e != hipSuccess)
    return fail(BMX_E_HIP, name + std::string(": combine kernel launch: ") + hipGetErrorString(e));
  return BMX_OK;
}
