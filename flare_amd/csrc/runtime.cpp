// Streams for callers that hold no HIP runtime binding of their own (a host
// in another language over the C ABI).
#include <hip/hip_runtime.h>

#include "common.hpp"

using namespace flare;

extern "C" int flare_stream_create(void **stream_out) {
  if (!stream_out) return fail(FLARE_ERR_ARGUMENT, "stream_out is null");
  hipStream_t s = nullptr;
  // default priority: every stream of the library runs at the same priority
  const hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
  if (e != hipSuccess) return hip_fail(e, "hipStreamCreateWithFlags");
  *stream_out = s;
  return FLARE_OK;
}

extern "C" int flare_stream_synchronize(void *stream) {
  const hipError_t e = hipStreamSynchronize(as_stream(stream));
  return e == hipSuccess ? FLARE_OK : hip_fail(e, "hipStreamSynchronize");
}

extern "C" int flare_stream_destroy(void *stream) {
  if (!stream) return fail(FLARE_ERR_ARGUMENT, "the null (default) stream cannot be destroyed");
  const hipError_t e = hipStreamDestroy(as_stream(stream));
  return e == hipSuccess ? FLARE_OK : hip_fail(e, "hipStreamDestroy");
}
