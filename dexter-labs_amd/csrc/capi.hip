// Error slot, version query and launch-schedule overrides of the C ABI
// (include/dexter_gfx950.h).
#include "dx_common.h"

#include <stdarg.h>
#include <stdio.h>

#include <atomic>

namespace dx {

namespace {
thread_local char g_error[512] = "";
}

namespace {
std::atomic<int> g_tuning[DX_TUNE_KEYS];  // zero-initialised: the library's own choices
}

int tuning(int key) { return g_tuning[key].load(std::memory_order_relaxed); }

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

}  // namespace dx

extern "C" const char* dx_last_error(void) { return dx::g_error; }

extern "C" int dx_abi_version(void) { return DX_ABI_VERSION; }

extern "C" int dx_set_tuning(int key, int value) {
  // Largest value per key: splits 16, attention kernel 4, norm waves 16,
  // QKV splits 16, QKV waves 4, decode merge 2, split merge of the paired
  // and dual-stream kernels 3.
  static const int kMax[DX_TUNE_KEYS] = {16, 4, 16, 16, 4, 2, 3};
  DX_CHECK_ARG(key >= 0 && key < DX_TUNE_KEYS, "set_tuning: unknown key %d", key);
  DX_CHECK_ARG(value >= 0 && value <= kMax[key], "set_tuning: value %d out of range for key %d",
               value, key);
  dx::g_tuning[key].store(value, std::memory_order_relaxed);
  return DX_OK;
}
