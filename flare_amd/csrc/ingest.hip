// CSR-native ingest: global dense positions of the unique ids' first
// occurrences, computed on the device from the ragged batch itself.
//
// A ragged batch of L nested levels: splits[0] maps each local row r0 to a
// range of level-1 entries, ..., splits[L-1] maps the last level's entries to
// ranges of flat values.  Flat value i therefore has a path (r0, j1, ..., jL):
// j_k is the entry's index inside its parent's range.  Its dense position is
// origin[r0] * S_0 + j1 * S_1 + ... + jL * S_L, where S_k are the suffix
// products of widths (the dense shape after the row axis), i.e. the row-major
// offset in [global_rows, widths...].
#include "common.hpp"

#include <algorithm>

namespace flare {
namespace {

constexpr int kMaxLevels = 4;
constexpr int kThreads = 256;

struct Nested {
  const int64_t *splits[kMaxLevels];
  int64_t entries[kMaxLevels];  // splits[k] has entries[k] + 1 values
  int64_t strides[kMaxLevels + 1];
  int64_t widths[kMaxLevels];
  int levels;
  int64_t rows;  // origin entries
};

// Index e with splits[e] <= v < splits[e + 1] (the last such e when ranges are
// empty), or -1 when v lies outside [splits[0], splits[entries]).
__device__ __forceinline__ int64_t owner(const int64_t *splits, int64_t entries, int64_t v) {
  if (entries <= 0 || v < splits[0] || v >= splits[entries]) return -1;
  int64_t lo = 0, hi = entries;  // splits[lo] <= v < splits[hi]
  while (hi - lo > 1) {
    const int64_t mid = lo + (hi - lo) / 2;
    if (splits[mid] <= v) lo = mid;
    else hi = mid;
  }
  return lo;
}

__global__ __launch_bounds__(kThreads) void positions_kernel(const int64_t *__restrict__ first, int64_t count,
                                                             Nested nest, const int64_t *__restrict__ origin,
                                                             int32_t *__restrict__ out, int *err) {
  for (int64_t u = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; u < count;
       u += static_cast<int64_t>(gridDim.x) * kThreads) {
    int64_t v = first[u];
    int64_t pos = 0;
    bool ok = true;
    // innermost level first: the entry holding v, then that entry inside its parent, ...
    for (int k = nest.levels - 1; k >= 0 && ok; --k) {
      const int64_t e = owner(nest.splits[k], nest.entries[k], v);
      if (e < 0) {
        ok = false;
        break;
      }
      const int64_t j = v - nest.splits[k][e];
      if (j >= nest.widths[k]) {
        ok = false;
        break;
      }
      pos += j * nest.strides[k + 1];
      v = e;
    }
    if (ok) {
      if (v < 0 || v >= nest.rows) ok = false;
      else pos += origin[v] * nest.strides[0];
    }
    if (!ok || pos < 0 || pos > 0x7fffffffll) {
      record_error(err, kErrIndexOutOfRange);
      pos = -1;
    }
    out[u] = static_cast<int32_t>(pos);
  }
}

}  // namespace
}  // namespace flare

using namespace flare;

extern "C" int flare_nested_global_positions(const int64_t *first_indices, int64_t count, int32_t levels,
                                             const int64_t *const *splits, const int64_t *split_lengths,
                                             const int64_t *origin_indices, int64_t origin_rows,
                                             const int64_t *widths, int32_t *out, void *stream) {
  if (levels < 1 || levels > kMaxLevels)
    return fail(FLARE_ERR_ARGUMENT, "nested levels must be in [1, %d], got %d", kMaxLevels, levels);
  if (count < 0 || origin_rows < 0) return fail(FLARE_ERR_SHAPE, "invalid nested position sizes");
  if (!splits || !split_lengths || !widths) return fail(FLARE_ERR_ARGUMENT, "nested splits and widths are required");
  Nested nest{};
  nest.levels = levels;
  nest.rows = origin_rows;
  for (int k = 0; k < levels; ++k) {
    if (split_lengths[k] < 1 || !splits[k]) return fail(FLARE_ERR_SHAPE, "nested level %d has no splits", k);
    if (widths[k] <= 0) return fail(FLARE_ERR_SHAPE, "dense width %d must be positive, got %lld", k,
                                    static_cast<long long>(widths[k]));
    nest.splits[k] = splits[k];
    nest.entries[k] = split_lengths[k] - 1;
    nest.widths[k] = widths[k];
  }
  nest.strides[levels] = 1;
  for (int k = levels - 1; k >= 0; --k) nest.strides[k] = nest.strides[k + 1] * widths[k];
  if (count == 0) return FLARE_OK;
  if (!first_indices || !out || (origin_rows > 0 && !origin_indices))
    return fail(FLARE_ERR_ARGUMENT, "nested position buffers are null");
  int st = FLARE_OK;
  int *err = device_error_word(&st);
  if (!err) return st;
  const int grid = static_cast<int>(std::min<int64_t>(ceil_div(count, kThreads), 65536));
  positions_kernel<<<grid, kThreads, 0, as_stream(stream)>>>(first_indices, count, nest, origin_indices, out, err);
  FLARE_TRY_HIP(hipGetLastError());
  return FLARE_OK;
}
