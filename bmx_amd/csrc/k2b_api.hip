// Host-side helpers of the C-ABI: error channel, per-device launcher state and
// page geometry queries.

#include "k2b_common.h"

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
