// Host-side helpers of the C-ABI: error channel, per-device launcher state and
// page geometry queries.

#include "k2b_common.h"
#include "k2b_general.h"

#include <mutex>

static thread_local std::string g_last_error;

void bmx_set_error(const std::string& msg) { g_last_error = msg; }

extern "C" const char* bmx_last_error(void) { return g_last_error.c_str(); }

// Launcher state per device: every GPU of a process (a device id up to
// kMaxDevices - 1) has its own CU count and its own raised LDS limits.
namespace {
constexpr int kMaxDevices = 64;
constexpr int kMaxLdsKernels = 64;
std::mutex g_dev_mu;
int g_cu_count[kMaxDevices];
struct LdsEntry {
  int dev;
  const void* kernel;
  size_t bytes;
};
LdsEntry g_lds[kMaxLdsKernels];
int g_n_lds = 0;

int current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
  return dev;
}
}  // namespace

int bmx_device_cu_count() {
  const int dev = current_device();
  std::lock_guard<std::mutex> lock(g_dev_mu);
  if (dev < kMaxDevices && g_cu_count[dev] > 0) return g_cu_count[dev];
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;   // MI355X
  if (dev < kMaxDevices) g_cu_count[dev] = cus;
  return cus;
}

hipError_t bmx_ensure_dynamic_lds(const void* kernel, size_t bytes) {
  const int dev = current_device();
  std::lock_guard<std::mutex> lock(g_dev_mu);
  int slot = -1;
  for (int i = 0; i < g_n_lds; ++i)
    if (g_lds[i].dev == dev && g_lds[i].kernel == kernel) slot = i;
  if (slot >= 0 && g_lds[slot].bytes >= bytes) return hipSuccess;
  const hipError_t e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (e != hipSuccess) return e;
  if (slot < 0 && g_n_lds < kMaxLdsKernels) slot = g_n_lds++;
  if (slot >= 0) g_lds[slot] = LdsEntry{dev, kernel, bytes};
  return hipSuccess;
}

// The geometry's page sections: (offset, size) of US, VNORM, KSCALE, KRES,
// VCODE and the page size; an error message when the geometry is not taken.
static std::string page_sections(const bmx_k2b_geom* g, int32_t starts[6], int32_t sizes[5]) {
  if (!g) return "geometry is NULL";
  const bmx::Geo geo = bmx::Geo::from(*g);
  const std::string why = geo.check();
  if (!why.empty()) return why;
  if (!geo.general) {
    const bmx::PageLayout L = bmx::PageLayout::make(geo.h, geo.R);
    const int32_t st[6] = {L.us, L.vnorm, L.kscale, L.kres, L.vcode, L.bytes};
    for (int i = 0; i < 6; ++i) starts[i] = st[i];
    for (int i = 0; i < 5; ++i) sizes[i] = st[i + 1] - st[i];
    return "";
  }
  const bmx::GenLayout L = bmx::GenLayout::of(geo);
  const int32_t st[6] = {L.us, L.vnorm, L.kscale, L.kres, L.vcode, L.bytes};
  const int32_t sz[5] = {bmx::kPT * geo.R * 2, geo.h * bmx::kPT * 2, L.per_slot * 2,
                         geo.h * bmx::kPT * (geo.d / 2), geo.h * 4 * geo.d};
  for (int i = 0; i < 6; ++i) starts[i] = st[i];
  for (int i = 0; i < 5; ++i) sizes[i] = sz[i];
  return "";
}

extern "C" size_t bmx_k2b_page_bytes(const bmx_k2b_geom* g) {
  int32_t starts[6], sizes[5];
  const std::string why = page_sections(g, starts, sizes);
  if (!why.empty()) {
    bmx_set_error("bmx_k2b_page_bytes: unsupported geometry: " + why);
    return 0;
  }
  return (size_t)starts[5];
}

extern "C" int bmx_k2b_page_section(const bmx_k2b_geom* g, int section, size_t* offset,
                                    size_t* bytes) {
  int32_t starts[6], sizes[5];
  const std::string why = page_sections(g, starts, sizes);
  if (!why.empty() || !offset || !bytes) {
    bmx_set_error("bmx_k2b_page_section: " + (why.empty() ? std::string("NULL output") : why));
    return BMX_E_INVALID;
  }
  if (section < 0 || section > 4) {
    bmx_set_error("bmx_k2b_page_section: section must be 0..4");
    return BMX_E_INVALID;
  }
  *offset = (size_t)starts[section];
  *bytes = (size_t)sizes[section];
  return BMX_OK;
}
