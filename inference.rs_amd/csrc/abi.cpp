// Library identity and the per-thread error slot of the C ABI.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "inferencequant.h"

#ifndef QMM_BUILD_ID
#define QMM_BUILD_ID "qmm-gfx950-dev"
#endif

extern "C" {

// kernel_library.rs:8, 288-297: every kernel library exports the id of the build it belongs to
__attribute__((visibility("default"))) const char inference_kernel_build_id[] = QMM_BUILD_ID;

}

namespace {
thread_local char g_error[512] = {0};
}

void qmm_set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof g_error, fmt, ap);
  va_end(ap);
}

int qmm_device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

extern "C" const char *qmm_last_error(void) { return g_error; }
extern "C" void qmm_clear_error(void) { g_error[0] = 0; }
