// The per-device error word that kernels OR their error bits into.  It is a
// __device__ variable: every GPU the library runs on holds its own copy,
// zero when the code object loads, so no call allocates it (entry points stay
// usable by callers that cannot allocate).  Host code reaches it through the
// address hipGetSymbolAddress returns for the current device, never through
// the variable's name.
#include <hip/hip_runtime.h>

#include <mutex>

#include "common.hpp"

namespace flare {

static __device__ int error_word;

namespace {
std::mutex g_word_mutex;
int *g_words[64] = {};
}  // namespace

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
    e = hipGetSymbolAddress(reinterpret_cast<void **>(&p), HIP_SYMBOL(error_word));
    if (e != hipSuccess || p == nullptr) {
      *status = hip_fail(e == hipSuccess ? hipErrorInvalidSymbol : e, "hipGetSymbolAddress(error word)");
      return nullptr;
    }
    g_words[dev] = p;
  }
  *status = FLARE_OK;
  return g_words[dev];
}

}  // namespace flare
