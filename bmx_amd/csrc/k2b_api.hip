// Host-side helpers of the C-ABI: error channel and page geometry queries.

#include "k2b_common.h"

static thread_local std::string g_last_error;

void bmx_set_error(const std::string& msg) { g_last_error = msg; }

extern "C" const char* bmx_last_error(void) { return g_last_error.c_str(); }

static bool geom_ok(const bmx_k2b_geom* g) {
  return g && g->h_kv >= 1 && g->h_kv <= 16 && (g->rank == 16 || g->rank == 32);
}

extern "C" size_t bmx_k2b_page_bytes(const bmx_k2b_geom* g) {
  if (!geom_ok(g)) {
    bmx_set_error("bmx_k2b_page_bytes: unsupported geometry (h_kv 1..16, rank 16|32)");
    return 0;
  }
  return (size_t)bmx::PageLayout::make(g->h_kv, g->rank).bytes;
}

extern "C" int bmx_k2b_page_section(const bmx_k2b_geom* g, int section, size_t* offset,
                                    size_t* bytes) {
  if (!geom_ok(g) || !offset || !bytes) {
    bmx_set_error("bmx_k2b_page_section: bad geometry or NULL output");
    return BMX_E_INVALID;
  }
  const bmx::PageLayout L = bmx::PageLayout::make(g->h_kv, g->rank);
  const int32_t starts[6] = {L.us, L.vnorm, L.kscale, L.kres, L.vcode, L.bytes};
  if (section < 0 || section > 4) {
    bmx_set_error("bmx_k2b_page_section: section must be 0..4");
    return BMX_E_INVALID;
  }
  *offset = (size_t)starts[section];
  *bytes = (size_t)(starts[section + 1] - starts[section]);
  return BMX_OK;
}
