// Thread-local error messages and the per-device error word.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <mutex>

#include "common.hpp"

namespace flare {

namespace {
thread_local char g_message[512] = "";
std::mutex g_word_mutex;
int *g_words[64] = {};
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

int *device_error_word(int *status) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= 64) {
    *status = hip_fail(e == hipSuccess ? hipErrorInvalidDevice : e, "hipGetDevice");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_word_mutex);
  if (!g_words[dev]) {
    int *p = nullptr;
    e = hipMalloc(&p, sizeof(int));
    if (e == hipSuccess) e = hipMemset(p, 0, sizeof(int));
    if (e != hipSuccess) {
      *status = hip_fail(e, "allocating the device error word");
      return nullptr;
    }
    g_words[dev] = p;
  }
  *status = FLARE_OK;
  return g_words[dev];
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
