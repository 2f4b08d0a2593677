// Raw byte movement.  Row copies between device tables: gather (dst_index
// NULL), scatter (src_index NULL) or both, used by the stores' assign and
// checkpoint page-image export / import; rows move as raw bytes, so every
// dtype (storage values, fp32 optimizer state, int32 step counters) shares
// it.  And a zero fill: a kernel, not hipMemsetAsync, so that a caller may
// capture it in a HIP graph.
#include "common.hpp"

#include <algorithm>

namespace flare {
namespace {

constexpr int kThreads = 256;

template <typename U>
__global__ __launch_bounds__(kThreads) void copy_rows_kernel(const U *__restrict__ src, int64_t src_rows,
                                                             U *__restrict__ dst, int64_t dst_rows,
                                                             int64_t units, const int32_t *__restrict__ src_index,
                                                             const int32_t *__restrict__ dst_index, int64_t n,
                                                             int *err) {
  const int64_t total = n * units;
  for (int64_t t = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; t < total;
       t += static_cast<int64_t>(gridDim.x) * kThreads) {
    const int64_t i = t / units;
    const int64_t u = t - i * units;
    const int64_t s = src_index ? src_index[i] : i;
    const int64_t d = dst_index ? dst_index[i] : i;
    if (s < 0 || s >= src_rows || d < 0 || d >= dst_rows) {
      if (u == 0) record_error(err, kErrIndexOutOfRange);
      continue;
    }
    dst[d * units + u] = src[s * units + u];
  }
}

template <typename U>
__global__ __launch_bounds__(kThreads) void fill_zero_kernel(U *__restrict__ dst, int64_t units) {
  for (int64_t t = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; t < units;
       t += static_cast<int64_t>(gridDim.x) * kThreads)
    dst[t] = U{};
}

// Contiguous copy of `units` U-sized units: one unit per thread over a full
// grid of short blocks.  At any moment the blocks in flight cover one compact
// window of the source and the destination, which keeps HBM streaming; the
// same copy written as a grid-stride loop over a capped grid moved 10-25%
// less on this GPU (blocks drift apart and spread over many DRAM pages).
template <typename U>
__global__ __launch_bounds__(kThreads) void copy_contiguous_kernel(const U *__restrict__ src, U *__restrict__ dst,
                                                                   int64_t units) {
  const int64_t t = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x;
  if (t < units) dst[t] = src[t];
}

// dst[i] = src[i] converted through float32 (exact widening, round-to-nearest-
// even narrowing); four elements per thread.
template <typename SrcTag, typename DstTag>
__global__ __launch_bounds__(kThreads) void convert_kernel(const typename SrcTag::elem *__restrict__ src,
                                                           typename DstTag::elem *__restrict__ dst, int64_t count) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads * 4;
  for (int64_t i = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) * 4; i < count; i += stride) {
    if (i + 4 <= count) {
      typename SrcTag::elem v[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) v[k] = src[i + k];
#pragma unroll
      for (int k = 0; k < 4; ++k) dst[i + k] = DstTag::from_f32(SrcTag::to_f32(v[k]));
    } else {
      for (int64_t k = i; k < count; ++k) dst[k] = DstTag::from_f32(SrcTag::to_f32(src[k]));
    }
  }
}

template <typename SrcTag>
int launch_convert(const void *src, void *dst, int32_t dst_dtype, int64_t count, hipStream_t s) {
  const int grid = static_cast<int>(std::min<int64_t>(std::max<int64_t>(ceil_div(count, kThreads * 4), 1), 1 << 16));
  const auto *in = static_cast<const typename SrcTag::elem *>(src);
  switch (dst_dtype) {
    case FLARE_FLOAT32: convert_kernel<SrcTag, TagF32><<<grid, kThreads, 0, s>>>(in, static_cast<float *>(dst), count); break;
    case FLARE_FLOAT16: convert_kernel<SrcTag, TagF16><<<grid, kThreads, 0, s>>>(in, static_cast<_Float16 *>(dst), count); break;
    case FLARE_BFLOAT16: convert_kernel<SrcTag, TagBF16><<<grid, kThreads, 0, s>>>(in, static_cast<uint16_t *>(dst), count); break;
    default: return fail(FLARE_ERR_DTYPE, "conversion target must be float32, float16 or bfloat16, got dtype code %d", dst_dtype);
  }
  FLARE_TRY_HIP(hipGetLastError());
  return FLARE_OK;
}

}  // namespace
}  // namespace flare

using namespace flare;

extern "C" int flare_convert(const void *src, int32_t src_dtype, void *dst, int32_t dst_dtype, int64_t count,
                             void *stream) {
  if (count < 0) return fail(FLARE_ERR_SHAPE, "element count %lld is negative", static_cast<long long>(count));
  if (storage_bytes(src_dtype) == 0 || storage_bytes(dst_dtype) == 0)
    return fail(FLARE_ERR_DTYPE, "conversion supports float32, float16 and bfloat16, got dtype codes %d -> %d",
                src_dtype, dst_dtype);
  if (count == 0) return FLARE_OK;
  if (!src || !dst) return fail(FLARE_ERR_ARGUMENT, "conversion buffers are null");
  hipStream_t s = as_stream(stream);
  switch (src_dtype) {
    case FLARE_FLOAT32: return launch_convert<TagF32>(src, dst, dst_dtype, count, s);
    case FLARE_FLOAT16: return launch_convert<TagF16>(src, dst, dst_dtype, count, s);
    default: return launch_convert<TagBF16>(src, dst, dst_dtype, count, s);
  }
}

extern "C" int flare_zero_bytes(void *dst, int64_t bytes, void *stream) {
  if (bytes < 0) return fail(FLARE_ERR_SHAPE, "byte count %lld is negative", static_cast<long long>(bytes));
  if (bytes == 0) return FLARE_OK;
  if (!dst) return fail(FLARE_ERR_ARGUMENT, "zero fill buffer is null");
  hipStream_t s = as_stream(stream);
  int unit = 1;
  for (int c : {16, 4}) {
    if (bytes % c == 0 && aligned(dst, c)) {
      unit = c;
      break;
    }
  }
  const int64_t units = bytes / unit;
  // one unit per thread (a full grid of short blocks) up to 2^31 - 1 blocks
  const int grid = static_cast<int>(std::min<int64_t>(ceil_div(units, kThreads), 0x7fffffff));
  if (unit == 16) fill_zero_kernel<uint4><<<grid, kThreads, 0, s>>>(static_cast<uint4 *>(dst), units);
  else if (unit == 4) fill_zero_kernel<uint32_t><<<grid, kThreads, 0, s>>>(static_cast<uint32_t *>(dst), units);
  else fill_zero_kernel<uint8_t><<<grid, kThreads, 0, s>>>(static_cast<uint8_t *>(dst), units);
  FLARE_TRY_HIP(hipGetLastError());
  return FLARE_OK;
}

extern "C" int flare_copy_rows(const void *src, int64_t src_rows, void *dst, int64_t dst_rows, int64_t row_bytes,
                               const int32_t *src_index, const int32_t *dst_index, int64_t n, void *stream) {
  if (row_bytes <= 0 || row_bytes % 2 != 0 || src_rows < 0 || dst_rows < 0 || n < 0)
    return fail(FLARE_ERR_SHAPE, "invalid row copy sizes (row_bytes %lld must be a positive multiple of 2)",
                static_cast<long long>(row_bytes));
  if (n == 0) return FLARE_OK;
  if (!src || !dst) return fail(FLARE_ERR_ARGUMENT, "row copy buffers are null");
  if (!src_index && n > src_rows) return fail(FLARE_ERR_SHAPE, "more rows than the source holds");
  if (!dst_index && n > dst_rows) return fail(FLARE_ERR_SHAPE, "more rows than the destination holds");
  int st = FLARE_OK;
  int *err = device_error_word(&st);
  if (!err) return st;
  hipStream_t s = as_stream(stream);
  int unit = 2;
  for (int c : {16, 8, 4}) {
    if (row_bytes % c == 0 && aligned(src, c) && aligned(dst, c)) {
      unit = c;
      break;
    }
  }
  const int64_t units = row_bytes / unit;
  if (!src_index && !dst_index && ceil_div(n * units, kThreads) <= 0x7fffffff) {
    // rows 0 .. n-1 onto rows 0 .. n-1: one contiguous block of n * row_bytes bytes
    const int cgrid = static_cast<int>(ceil_div(n * units, kThreads));
    switch (unit) {
      case 16: copy_contiguous_kernel<uint4><<<cgrid, kThreads, 0, s>>>(static_cast<const uint4 *>(src),
                                                                        static_cast<uint4 *>(dst), n * units); break;
      case 8: copy_contiguous_kernel<uint2><<<cgrid, kThreads, 0, s>>>(static_cast<const uint2 *>(src),
                                                                       static_cast<uint2 *>(dst), n * units); break;
      case 4: copy_contiguous_kernel<uint32_t><<<cgrid, kThreads, 0, s>>>(static_cast<const uint32_t *>(src),
                                                                          static_cast<uint32_t *>(dst), n * units);
        break;
      default: copy_contiguous_kernel<uint16_t><<<cgrid, kThreads, 0, s>>>(static_cast<const uint16_t *>(src),
                                                                           static_cast<uint16_t *>(dst), n * units);
        break;
    }
    FLARE_TRY_HIP(hipGetLastError());
    return FLARE_OK;
  }
  const int grid = static_cast<int>(std::min<int64_t>(ceil_div(n * units, kThreads), 1 << 16));
  switch (unit) {
    case 16:
      copy_rows_kernel<uint4><<<grid, kThreads, 0, s>>>(static_cast<const uint4 *>(src), src_rows,
                                                        static_cast<uint4 *>(dst), dst_rows, units, src_index,
                                                        dst_index, n, err);
      break;
    case 8:
      copy_rows_kernel<uint2><<<grid, kThreads, 0, s>>>(static_cast<const uint2 *>(src), src_rows,
                                                        static_cast<uint2 *>(dst), dst_rows, units, src_index,
                                                        dst_index, n, err);
      break;
    case 4:
      copy_rows_kernel<uint32_t><<<grid, kThreads, 0, s>>>(static_cast<const uint32_t *>(src), src_rows,
                                                           static_cast<uint32_t *>(dst), dst_rows, units,
                                                           src_index, dst_index, n, err);
      break;
    default:
      copy_rows_kernel<uint16_t><<<grid, kThreads, 0, s>>>(static_cast<const uint16_t *>(src), src_rows,
                                                           static_cast<uint16_t *>(dst), dst_rows, units,
                                                           src_index, dst_index, n, err);
      break;
  }
  FLARE_TRY_HIP(hipGetLastError());
  return FLARE_OK;
}
