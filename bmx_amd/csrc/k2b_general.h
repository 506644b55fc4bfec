// General k2b geometry: head_dim, rank, residual group and key bits other than
// the reference recipe's (128, 16|32, 64, 3), on the general page
// (include/bmx_k2b.h).  Host and device helpers shared by the page queries,
// the entry points' dispatch and the kernels of k2b_general.hip.
#pragma once

#include <string>

#include "k2b_common.h"

namespace bmx {

// A bmx_k2b_geom with its defaults filled in.
struct Geo {
  int h, R, G, d, group, bits;
  bool general;   // not the recipe's page format

  static Geo from(const bmx_k2b_geom& g) {
    Geo o;
    o.h = g.h_kv;
    o.R = g.rank;
    o.G = g.n_q_groups;
    o.d = g.head_dim ? g.head_dim : kD;
    o.group = g.k_group ? g.k_group : kGroup;
    o.bits = g.k_bits ? g.k_bits : 3;
    o.general = !(o.d == kD && o.group == kGroup && o.bits == 3 && (o.R == 16 || o.R == 32));
    return o;
  }
  int C() const { return d * h; }
  // an empty string when the geometry is one this library takes for pages and
  // append (decode adds its own limits)
  std::string check() const {
    if (h < 1 || h > 16) return "h_kv must be 1..16";
    if (!general) return "";
    if (d != 32 && d != 64 && d != 128) return "head_dim must be 32, 64 or 128";
    if (R != 16 && R != 32 && R != 64 && R != 128) return "rank must be 16, 32, 64 or 128";
    if (R > d * h) return "rank must not exceed C = head_dim * h_kv";
    if (group != 16 && group != 32 && group != 64 && group != 128) return "k_group must be 16, 32, 64 or 128";
    if (bits < 2 || bits > 4) return "k_bits must be 2, 3 or 4";
    return "";
  }
};

__host__ __device__ constexpr int gen_align16(int x) { return (x + 15) & ~15; }

// Byte offsets of the general page's sections.
struct GenLayout {
  int32_t us, vnorm, kscale, kres, vcode, bytes;
  int32_t d, h, R, group, bits, C, slots, per_slot;   // slots = group / 16 pages share a group's scales
  __host__ __device__ static GenLayout make(int h, int R, int d, int group, int bits) {
    GenLayout L;
    L.d = d; L.h = h; L.R = R; L.group = group; L.bits = bits;
    L.C = d * h;
    L.slots = group / kPT;
    L.per_slot = L.C / L.slots;
    L.us = 0;
    L.vnorm = gen_align16(L.us + kPT * R * 2);
    L.kscale = gen_align16(L.vnorm + h * kPT * 2);
    L.kres = gen_align16(L.kscale + L.per_slot * 2);
    L.vcode = gen_align16(L.kres + h * kPT * (d / 2));
    L.bytes = gen_align16(L.vcode + h * 4 * d);
    return L;
  }
  static GenLayout of(const Geo& g) { return make(g.h, g.R, g.d, g.group, g.bits); }
};

// Entry points on the general page (k2b_general.hip), called by bmx_k2b_append,
// bmx_k2b_decode(_noalloc), bmx_k2b_decode_workspace_bytes and bmx_k2b_dequant
// after their common argument checks; the geometry-specific checks are theirs.
int gen_append(const bmx_k2b_append_args* a, hipStream_t st);
std::string gen_decode_check(const bmx_k2b_decode_args* a);
size_t gen_decode_workspace(const bmx_k2b_decode_args* a);
int gen_decode(const bmx_k2b_decode_args* a, hipStream_t st, void* ws, size_t ws_cap, const std::string& name);
int gen_dequant(const bmx_k2b_dequant_args* a, hipStream_t st);

}  // namespace bmx
