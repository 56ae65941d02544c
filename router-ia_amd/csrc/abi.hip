// Library-wide C ABI plumbing: version, thread-local last-error string.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "ria_common.h"

namespace ria {

static thread_local char g_last_error[1024] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return set_error(RIA_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  }
  return RIA_OK;
}

}  // namespace ria

extern "C" int ria_abi_version(void) { return RIA_ABI_VERSION; }

extern "C" const char* ria_last_error(void) { return ria::g_last_error; }

extern "C" int ria_device_info(int device, ria_device_record* out) {
  if (!out) return ria::set_error(RIA_ERR_INVALID, "ria_device_info: null record");
  hipDeviceProp_t p;
  const hipError_t e = hipGetDeviceProperties(&p, device);
  if (e != hipSuccess) return ria::set_error(RIA_ERR_LAUNCH, "ria_device_info: %s", hipGetErrorString(e));
  memset(out, 0, sizeof(*out));
  snprintf(out->name, sizeof(out->name), "%s", p.name);
  snprintf(out->arch, sizeof(out->arch), "%s", p.gcnArchName);
  out->compute_units = p.multiProcessorCount;
  out->clock_khz = p.clockRate;
  out->memory_clock_khz = p.memoryClockRate;
  out->memory_bus_bits = p.memoryBusWidth;
  out->memory_bytes = static_cast<int64_t>(p.totalGlobalMem);
  out->l2_bytes = p.l2CacheSize;
  out->lds_bytes_per_cu = static_cast<int>(p.maxSharedMemoryPerMultiProcessor);
  out->wavefront_size = p.warpSize;
  return RIA_OK;
}
