// Thread-local error messages and reading back the per-device error word
// (device_word.hip holds the word itself).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "common.hpp"

namespace flare {

namespace {
thread_local char g_message[512] = "";
}  // namespace

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_message, sizeof(g_message), fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t err, const char *what) {
  return fail(FLARE_ERR_HIP, "%s failed: %s", what, hipGetErrorString(err));
}

}  // namespace flare

extern "C" const char *flare_last_error(void) { return flare::g_message; }

extern "C" int32_t flare_abi_version(void) { return FLARE_ABI_VERSION; }

extern "C" int32_t flare_take_device_errors(void *stream) {
  int status = FLARE_OK;
  int *word = flare::device_error_word(&status);
  if (!word) return -1;
  hipStream_t s = flare::as_stream(stream);
  int value = 0;
  if (hipMemcpyAsync(&value, word, sizeof(int), hipMemcpyDeviceToHost, s) != hipSuccess) return -1;
  if (hipMemsetAsync(word, 0, sizeof(int), s) != hipSuccess) return -1;
  if (hipStreamSynchronize(s) != hipSuccess) return -1;
  return value;
}
