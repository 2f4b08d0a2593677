// Backward engine: stable radix sort of (key, occurrence) pairs, first-
// occurrence dedup, deterministic segment reduction and the fused sparse
// optimizer row update.
//
// Kernel sequence of one call (all on the caller's stream):
//   zero        clear histograms, tile tickets, look-back status, counters and
//               the first-occurrence bitmap
//   prepare     build the 32/64-bit sort key of every occurrence (invalid ->
//               sentinel) and the digit histograms of every radix pass
//   onesweep    one launch per 8-bit digit: stable in-tile ranking with wave64
//               ballots, decoupled look-back across tiles, LDS-staged scatter
//   head_count  key heads per tile of sorted keys, scanned by scan_counts
//   runs        run ids, run starts / keys, each key's first occurrence set in
//               the bitmap, gradient rows gathered into sorted order
//   first_count first occurrences per tile of occurrences, scanned
//   rank        first-occurrence order: unique / first_indices / run -> rank
//   sums        long keys: per 64-position unit, sequential fp32 sums of the
//               key's gradient rows in occurrence order (per-key sums, or
//               unit partials for keys that span units)
//   fold        keys spanning many units: one block folds the unit partials
//   apply       per key: short keys summed here; then the optimizer update
//               (or the reduced gradient) written once per unique key
// The last three are in update.hpp, instantiated per value dtype in the
// update_*.hip files.
#include "backward.hpp"
#include "update.hpp"

#include <mutex>

#include <algorithm>
#include <cmath>
#include <type_traits>

namespace flare {

int bits_for(uint64_t max_value) {
  int b = 0;
  while (b < 64 && (max_value >> b) != 0) ++b;
  return b;
}

static size_t align_up(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

// Timing markers of the calling thread (flare_set_update_events).
thread_local hipEvent_t t_update_events[4] = {};
thread_local int t_update_event_count = 0;

Workspace layout_workspace(void *base, int64_t n, int key_bytes, int dim, bool need_grad_row,
                           bool need_aux, bool need_partials, bool need_sums) {
  Workspace w{};
  w.n = n;
  w.key_bytes = key_bytes;
  w.tiles = static_cast<uint32_t>(ceil_div(std::max<int64_t>(n, 1), kSortTile));
  w.sort_tiles = static_cast<uint32_t>(ceil_div(std::max<int64_t>(n, 1), kOneTile));
  w.units = static_cast<uint32_t>(ceil_div(std::max<int64_t>(n, 1), kReduceUnit));
  const size_t un = static_cast<size_t>(std::max<int64_t>(n, 1));
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off = align_up(off + bytes);
    return at;
  };
  const size_t o_hist = take(static_cast<size_t>(kHistCopies) * kMaxPasses * kMaxRadix * 4);
  const size_t o_tickets = take(16 * 4);
  const size_t o_meta = take(8 * 4);
  const size_t o_scan_status = take(static_cast<size_t>(2) * w.tiles * 4);
  // whole tiles, so first_count_kernel reads 16-byte vectors without a tail
  const size_t o_head_flag = take(static_cast<size_t>(w.tiles) * kSortTile);
  // per tile: every plan's passes x 2^digit bits (8 x 256 for 64-bit keys, 3 x 1024 at most for 32-bit)
  const size_t status_per_tile = std::max<size_t>(kMaxPasses * 256, 3 * kMaxRadix);
  const size_t o_sort_status = take(status_per_tile * w.sort_tiles * 4);
  w.sort_status_offset = o_sort_status;
  w.zero_bytes = off;
  const size_t o_k0 = take(un * key_bytes);
  const size_t o_k1 = take(un * key_bytes);
  const size_t o_v0 = take(un * 4);
  const size_t o_v1 = take(un * 4);
  const size_t o_grow = need_grad_row ? take(un * 4) : 0;
  const size_t o_sgr = need_grad_row ? take(un * 4) : 0;
  const size_t o_rgr = need_grad_row ? take(un * 4) : 0;
  const size_t o_aux = need_aux ? take(un * 4) : 0;
  const size_t o_ssc = need_aux ? take(un * 4) : 0;
  const size_t o_rsc = need_aux ? take(un * 4) : 0;
  const size_t o_head_run = take(un * 8);
  const size_t o_rs = take((un + 1) * 4);
  const size_t o_rr = take(un * 4);
  const size_t o_rk = take(un * 4);
  const size_t o_ufr = take(static_cast<size_t>(w.units) * 4);
  const size_t o_hot = take(static_cast<size_t>(w.units) * 4);
  const size_t o_part = need_partials ? take(static_cast<size_t>(w.units) * 2 * dim * 4) : 0;
  const size_t o_sums = need_sums ? take(un * static_cast<size_t>(dim) * 4) : 0;
  w.total_bytes = off;
  if (base) {
    char *b = static_cast<char *>(base);
    w.hist = reinterpret_cast<uint32_t *>(b + o_hist);
    w.tickets = reinterpret_cast<uint32_t *>(b + o_tickets);
    w.meta = reinterpret_cast<uint32_t *>(b + o_meta);
    w.sort_status = reinterpret_cast<uint32_t *>(b + o_sort_status);
    w.scan_status = reinterpret_cast<uint32_t *>(b + o_scan_status);
    w.keys[0] = b + o_k0;
    w.keys[1] = b + o_k1;
    w.vals[0] = reinterpret_cast<uint32_t *>(b + o_v0);
    w.vals[1] = reinterpret_cast<uint32_t *>(b + o_v1);
    w.grad_row = need_grad_row ? reinterpret_cast<uint32_t *>(b + o_grow) : nullptr;
    w.aux = need_aux ? reinterpret_cast<float *>(b + o_aux) : nullptr;
    w.sorted_grad_row = need_grad_row ? reinterpret_cast<uint32_t *>(b + o_sgr) : nullptr;
    w.sorted_scale = need_aux ? reinterpret_cast<float *>(b + o_ssc) : nullptr;
    w.run_grad_row = need_grad_row ? reinterpret_cast<uint32_t *>(b + o_rgr) : nullptr;
    w.run_scale = need_aux ? reinterpret_cast<float *>(b + o_rsc) : nullptr;
    w.head_flag = reinterpret_cast<uint8_t *>(b + o_head_flag);
    w.head_run = reinterpret_cast<uint2 *>(b + o_head_run);
    w.run_start = reinterpret_cast<uint32_t *>(b + o_rs);
    w.run_rank = reinterpret_cast<uint32_t *>(b + o_rr);
    w.run_key = reinterpret_cast<uint32_t *>(b + o_rk);
    w.unit_first_run = reinterpret_cast<uint32_t *>(b + o_ufr);
    w.hot_runs = reinterpret_cast<uint32_t *>(b + o_hot);
    w.partial = need_partials ? reinterpret_cast<float *>(b + o_part) : nullptr;
    w.sums = need_sums ? reinterpret_cast<float *>(b + o_sums) : nullptr;
  }
  return w;
}

RadixPlan radix_plan(int bits, int key_bytes) {
  const int p8 = std::max(1, (bits + 7) / 8);
  if (key_bytes == 4) {
    for (int d = 9; d <= kMaxDigitBits; ++d) {
      const int p = std::max(1, (bits + d - 1) / d);
      if (p < p8) return {d, p};
    }
  }
  return {8, p8};
}

size_t zero_bytes_for(const Workspace &w, const RadixPlan &plan) {
  const size_t status = static_cast<size_t>(plan.passes) * w.sort_tiles * (size_t{1} << plan.digit_bits) * 4;
  return std::min(w.zero_bytes, align_up(w.sort_status_offset + status));
}

namespace {

// ----------------------------------------------------------------------------
// zero
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(256) void zero_kernel(uint4 *p, size_t n16) {
  for (size_t i = blockIdx.x * 256ull + threadIdx.x; i < n16; i += gridDim.x * 256ull)
    p[i] = make_uint4(0, 0, 0, 0);
}

__global__ __launch_bounds__(256) void zero_f32_kernel(float *p, size_t n) {
  for (size_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += gridDim.x * 256ull) p[i] = 0.0f;
}

// ----------------------------------------------------------------------------
// finite check of a gradient (or any storage-dtype array)
// ----------------------------------------------------------------------------
__global__ void zero_count_kernel(int64_t *count) {
  if (threadIdx.x == 0) *count = 0;
}

// A zero count written by a kernel (not a memset node), so that the call
// can be captured in a graph.
int launch_zero_count(int64_t *count, hipStream_t s) {
  zero_count_kernel<<<1, 64, 0, s>>>(count);
  FLARE_TRY_HIP(hipGetLastError());
  return FLARE_OK;
}

__global__ void clear_flags_kernel(uint32_t *flag, int32_t *flag_out) {
  if (threadIdx.x == 0) {
    if (flag) *flag = 0;
    if (flag_out) *flag_out = 0;
  }
}

// Sets *flag / *flag_out to 1 (and error bit kErrNonFinite) when any of the
// `count` elements is inf or NaN: exponent bits all ones.
__global__ __launch_bounds__(256) void nonfinite_kernel(const void *values, int elem_bytes, uint32_t exp_mask,
                                                        uint64_t count, uint32_t *flag, int32_t *flag_out, int *err) {
  bool bad = false;
  const uint64_t tid = blockIdx.x * 256ull + threadIdx.x;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * 256ull;
  const uint64_t per16 = 16 / elem_bytes;
  const uint64_t n16 = (reinterpret_cast<uintptr_t>(values) % 16 == 0) ? count / per16 : 0;
  const uint4 *v16 = static_cast<const uint4 *>(values);
  for (uint64_t i = tid; i < n16; i += stride) {
    const uint4 q = v16[i];
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (elem_bytes == 4) bad |= (w[k] & exp_mask) == exp_mask;
      else bad |= ((w[k] & exp_mask) == exp_mask) || (((w[k] >> 16) & exp_mask) == exp_mask);
    }
  }
  for (uint64_t i = n16 * per16 + tid; i < count; i += stride) {
    const uint32_t x = elem_bytes == 4 ? static_cast<const uint32_t *>(values)[i]
                                       : static_cast<const uint16_t *>(values)[i];
    bad |= (x & exp_mask) == exp_mask;
  }
  if (__ballot(bad) && (threadIdx.x & 63) == 0) {
    if (flag) *flag = 1;
    if (flag_out) *flag_out = 1;
    record_error(err, kErrNonFinite);
  }
}

// Clears the flags, then checks `count` elements of a float32, float16 or
// bfloat16 array.
int launch_finite_check(const void *values, int dtype, int64_t count, uint32_t *flag, int32_t *flag_out, int *err,
                        hipStream_t s) {
  uint32_t mask = 0;
  int bytes = 0;
  switch (dtype) {
    case FLARE_FLOAT32: mask = 0x7f800000u; bytes = 4; break;
    case FLARE_FLOAT16: mask = 0x7c00u; bytes = 2; break;
    case FLARE_BFLOAT16: mask = 0x7f80u; bytes = 2; break;
    default: return fail(FLARE_ERR_DTYPE, "finite check requires float16, bfloat16 or float32, got dtype code %d", dtype);
  }
  clear_flags_kernel<<<1, 64, 0, s>>>(flag, flag_out);
  if (count > 0) {
    const int grid = static_cast<int>(std::min<int64_t>(std::max<int64_t>(1, ceil_div(count, 256 * 16 / bytes)), 8192));
    nonfinite_kernel<<<grid, 256, 0, s>>>(values, bytes, mask, static_cast<uint64_t>(count), flag, flag_out, err);
  }
  FLARE_TRY_HIP(hipGetLastError());
  return FLARE_OK;
}

int launch_zero(void *p, size_t bytes, hipStream_t s) {
  if (bytes == 0) return FLARE_OK;
  const size_t n16 = bytes / 16;  // every zeroed region is 256-byte aligned
  const int grid = static_cast<int>(std::min<size_t>((n16 + 255) / 256, 4096));
  zero_kernel<<<std::max(grid, 1), 256, 0, s>>>(static_cast<uint4 *>(p), n16);
  FLARE_TRY_HIP(hipGetLastError());
  return FLARE_OK;
}

// ----------------------------------------------------------------------------
// prepare: keys + histograms
// ----------------------------------------------------------------------------
template <typename K>
__device__ __forceinline__ void add_histograms(uint32_t *s_hist, K key, int passes, int digit) {
  const uint32_t mask = (1u << digit) - 1;
  for (int p = 0; p < passes; ++p) {
    const uint32_t d = static_cast<uint32_t>(key >> (p * digit)) & mask;
    atomicAdd(&s_hist[(p << digit) + d], 1u);
  }
}

__device__ __forceinline__ void flush_histograms(const uint32_t *s_hist, uint32_t *hist, int passes,
                                                 int digit) {
  uint32_t *copy = hist + static_cast<size_t>(blockIdx.x % kHistCopies) * kMaxPasses * kMaxRadix;
  for (int i = threadIdx.x; i < (passes << digit); i += blockDim.x) {
    const uint32_t c = s_hist[i];
    if (c) atomicAdd(&copy[(i >> digit) * kMaxRadix + (i & ((1 << digit) - 1))], c);
  }
}

// Global count of digit d of pass p: sum of the histogram copies.
__device__ __forceinline__ uint32_t digit_total(const uint32_t *hist, int pass, int d) {
  uint32_t sum = 0;
#pragma unroll
  for (int c = 0; c < kHistCopies; ++c) sum += hist[(static_cast<size_t>(c) * kMaxPasses + pass) * kMaxRadix + d];
  return sum;
}

// Keys from a row-index array (int64 store keys or int32 padded inverse).
// valid: 0 <= key < key_limit and key != pad (when has_pad); else sentinel.
template <typename SrcT>
__global__ __launch_bounds__(256) void prepare_rows_kernel(const SrcT *__restrict__ src, int64_t n,
                                                          int64_t key_limit, int has_pad,
                                                          int64_t pad, int passes, int digit,
                                                          uint32_t *__restrict__ keys,
                                                          uint32_t *__restrict__ hist, int *err) {
  __shared__ uint32_t s_hist[kMaxHistBins];
  for (int i = threadIdx.x; i < (passes << digit); i += 256) s_hist[i] = 0;
  __syncthreads();
  const uint32_t sentinel = static_cast<uint32_t>(key_limit);
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += gridDim.x * 256ll) {
    const int64_t v = static_cast<int64_t>(src[i]);
    uint32_t k = sentinel;
    if (!(has_pad && v == pad)) {
      if (v >= 0 && v < key_limit) {
        k = static_cast<uint32_t>(v);
      } else {
        record_error(err, kErrIndexOutOfRange);
      }
    }
    keys[i] = k;
    add_histograms(s_hist, k, passes, digit);
  }
  __syncthreads();
  flush_histograms(s_hist, hist, passes, digit);
}

// Keys from CSR bags (table-major, bag k = t*batch + b).  The block's bag
// boundaries are staged in LDS; each occurrence finds its bag by binary
// search there.  Also writes the gradient row (b*T + t for [B, T, D] pooled
// gradients, the bag k itself for [T, B, D]) and, for mean pooling, the bag
// length of every occurrence.
constexpr int kPrepMaxBags = 4096;
// Threads of a prepare block: about 512 blocks of 16 waves walk the bags, so
// that each thread has few bags and the whole GPU has its loads in flight.
constexpr int kPrepThreads = 1024;

// Bags per prepare block: about 512 blocks (fewer histogram flushes), at most kPrepMaxBags bags each.
constexpr int64_t kPerBagLength = 8;
// In the per-bag walk: bags longer than kPrepWalk ids go to a block-wide walk
// (at most kPrepLongBags of them per block; more are walked by their thread).
constexpr int64_t kPrepWalk = 32;
constexpr int kPrepLongBags = 256;

int prep_bags_per_block(int64_t bags) {
  return static_cast<int>(std::min<int64_t>(kPrepMaxBags, std::max<int64_t>(64, ceil_div(bags, 512))));
}

template <typename IdT>
__global__ __launch_bounds__(kPrepThreads) void prepare_csr_kernel(
    const IdT *__restrict__ ids, int64_t n, const int64_t *__restrict__ offsets, int64_t bags,
    int bags_per_block, const int64_t *__restrict__ row_base, int32_t num_tables, int64_t batch,
    int64_t key_limit, int passes, int digit, uint32_t *__restrict__ keys, uint32_t *__restrict__ grad_row,
    float *__restrict__ aux, uint32_t *__restrict__ hist, uint32_t *__restrict__ reject, int per_bag,
    int table_major, int one_id, uint32_t *__restrict__ ident_flag, int *err) {
  __shared__ uint32_t s_hist[kMaxHistBins];
  __shared__ int64_t s_off[kPrepMaxBags + 1];
  for (int i = threadIdx.x; i < (passes << digit); i += kPrepThreads) s_hist[i] = 0;
  const int64_t bag0 = static_cast<int64_t>(blockIdx.x) * bags_per_block;
  const int nb = static_cast<int>(std::min<int64_t>(bags_per_block, bags - bag0));
  for (int i = threadIdx.x; i <= nb; i += kPrepThreads) {
    const int64_t o = offsets[bag0 + i];
    s_off[i] = o < 0 ? 0 : (o > n ? n : o);
    // offsets must start at 0, end at n and never decrease; otherwise some
    // occurrences belong to no bag (or to two), so the batch is rejected
    if (o < 0 || o > n || (bag0 + i == 0 && o != 0) || (bag0 + i == bags && o != n)) {
      record_error(err, kErrIndexOutOfRange);
      *reject = 1;
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < nb; i += kPrepThreads)
    if (s_off[i + 1] < s_off[i] || (one_id && s_off[i + 1] - s_off[i] != 1)) {
      record_error(err, kErrIndexOutOfRange);
      *reject = 1;
    }
  // one id per bag in table-major order: occurrence i is pooled row i, which the
  // update kernels use in place of a stored gradient row (workspace word 6)
  const bool ident = one_id && table_major;
  if (ident && blockIdx.x == 0 && threadIdx.x == 0) *ident_flag = 1;
  const int64_t first = s_off[0];
  const int64_t last = s_off[nb];
  const uint32_t sentinel = static_cast<uint32_t>(key_limit);
  // occurrence i of block-local bag lo
  auto emit = [&](int64_t i, int lo) {
    const int64_t bag = bag0 + lo;
    const int64_t t = bag / batch;
    const int64_t b = bag - t * batch;
    const int64_t id = static_cast<int64_t>(ids[i]);
    const int64_t lo_row = row_base[t];
    uint32_t k = sentinel;
    if (id >= 0 && id < row_base[t + 1] - lo_row) {
      k = static_cast<uint32_t>(lo_row + id);
    } else {
      record_error(err, kErrIndexOutOfRange);
    }
    keys[i] = k;
    if (!ident) grad_row[i] = static_cast<uint32_t>(table_major ? bag : b * num_tables + t);
    if (aux) aux[i] = static_cast<float>(s_off[lo + 1] - s_off[lo]);
    add_histograms(s_hist, k, passes, digit);
  };
  if (per_bag) {
    // short bags: one thread per bag walks its few occurrences (no search);
    // bags longer than kPrepWalk are listed and then walked by the whole block
    __shared__ int s_long[kPrepLongBags];
    __shared__ int s_nlong;
    if (threadIdx.x == 0) s_nlong = 0;
    __syncthreads();
    for (int lo = threadIdx.x; lo < nb; lo += kPrepThreads) {
      const int64_t b0 = s_off[lo], b1 = s_off[lo + 1];
      if (b1 - b0 > kPrepWalk) {
        const int slot = atomicAdd(&s_nlong, 1);
        if (slot < kPrepLongBags) {
          s_long[slot] = lo;
          continue;
        }
      }
      for (int64_t i = b0; i < b1; ++i) emit(i, lo);
    }
    __syncthreads();
    const int nlong = s_nlong < kPrepLongBags ? s_nlong : kPrepLongBags;
    for (int j = 0; j < nlong; ++j) {
      const int lo = s_long[j];
      for (int64_t i = s_off[lo] + threadIdx.x; i < s_off[lo + 1]; i += kPrepThreads) emit(i, lo);
    }
  } else {
    for (int64_t i = first + threadIdx.x; i < last; i += kPrepThreads) {
      int lo = 0, hi = nb;  // find bag: s_off[lo] <= i < s_off[lo+1]
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (s_off[mid] <= i) lo = mid; else hi = mid;
      }
      emit(i, lo);
    }
  }
  __syncthreads();
  flush_histograms(s_hist, hist, passes, digit);
}

// Keys of bags of exactly one id in table-major order (the caller's
// FLARE_LAYOUT_ONE_ID_PER_BAG, n == bags): occurrence i is bag i of table
// i / batch, so no bag boundaries are staged or searched.  Four consecutive
// occurrences per thread; the claim is checked as offsets[i] == i for every
// i <= n (otherwise error bit 1 and the batch is rejected, as in
// prepare_csr_kernel).  Mean pooling divides by a bag length of 1.
constexpr int kPrepOneItems = 4;

template <typename IdT>
__global__ __launch_bounds__(kPrepThreads) void prepare_one_kernel(
    const IdT *__restrict__ ids, uint32_t n, const int64_t *__restrict__ offsets,
    const int64_t *__restrict__ row_base, uint32_t batch, int64_t key_limit, int passes, int digit,
    uint32_t *__restrict__ keys, float *__restrict__ aux, uint32_t *__restrict__ hist,
    uint32_t *__restrict__ reject, uint32_t *__restrict__ ident_flag, int *err) {
  __shared__ uint32_t s_hist[kMaxHistBins];
  for (int i = threadIdx.x; i < (passes << digit); i += kPrepThreads) s_hist[i] = 0;
  if (blockIdx.x == 0 && threadIdx.x == 0) *ident_flag = 1;
  __syncthreads();
  const uint32_t i0 = (blockIdx.x * kPrepThreads + threadIdx.x) * kPrepOneItems;
  const uint32_t sentinel = static_cast<uint32_t>(key_limit);
  if (i0 < n) {
    IdT id[kPrepOneItems];
    int64_t off[kPrepOneItems];
#pragma unroll
    for (int k = 0; k < kPrepOneItems; ++k) {
      const uint32_t i = i0 + k;
      id[k] = i < n ? ids[i] : IdT(0);
      off[k] = i < n ? offsets[i] : 0;
    }
    bool claim = true;
#pragma unroll
    for (int k = 0; k < kPrepOneItems; ++k)
      if (i0 + k < n && off[k] != static_cast<int64_t>(i0 + k)) claim = false;
    if (i0 + kPrepOneItems >= n && i0 <= n && offsets[n] != static_cast<int64_t>(n)) claim = false;
    if (!claim) {
      record_error(err, kErrIndexOutOfRange);
      *reject = 1;
    }
    uint32_t key[kPrepOneItems];
#pragma unroll
    for (int k = 0; k < kPrepOneItems; ++k) {
      const uint32_t i = i0 + k;
      key[k] = sentinel;
      if (i >= n) continue;
      const uint32_t t = i / batch;
      const int64_t lo = row_base[t];
      const int64_t v = static_cast<int64_t>(id[k]);
      if (v >= 0 && v < row_base[t + 1] - lo) {
        key[k] = static_cast<uint32_t>(lo + v);
      } else {
        record_error(err, kErrIndexOutOfRange);
      }
      add_histograms(s_hist, key[k], passes, digit);
      if (aux) aux[i] = 1.0f;
    }
    if (i0 + kPrepOneItems <= n) {
      *reinterpret_cast<uint4 *>(keys + i0) = make_uint4(key[0], key[1], key[2], key[3]);
    } else {
#pragma unroll
      for (int k = 0; k < kPrepOneItems; ++k)
        if (i0 + k < n) keys[i0 + k] = key[k];
    }
  }
  __syncthreads();
  flush_histograms(s_hist, hist, passes, digit);
}

// Keys for generic dedup: (value - minimum) as unsigned, 32 or 64 bits.
template <typename SrcT, typename K>
__global__ __launch_bounds__(256) void prepare_generic_kernel(const SrcT *__restrict__ src,
                                                             int64_t n,
                                                             const uint64_t *__restrict__ minimum,
                                                             uint64_t key_bound, int passes, int digit,
                                                             K *__restrict__ keys,
                                                             uint32_t *__restrict__ hist, int *err) {
  // minimum != nullptr: keys are mapped to their order-preserving unsigned
  // image and offset by the measured minimum; otherwise the caller promised
  // 0 <= key < key_bound and the raw value is the key: a key outside that
  // range (the sort only covers the bits of key_bound - 1, so its run could
  // split) sets the index error bit.
  __shared__ uint32_t s_hist[kMaxHistBins];
  for (int i = threadIdx.x; i < (passes << digit); i += 256) s_hist[i] = 0;
  __syncthreads();
  const uint64_t lo = minimum ? *minimum : 0;
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += gridDim.x * 256ll) {
    uint64_t ord;
    if constexpr (std::is_signed<SrcT>::value) {
      ord = static_cast<uint64_t>(static_cast<int64_t>(src[i]));
      if (minimum) ord ^= 0x8000000000000000ull;
    } else {
      ord = static_cast<uint64_t>(src[i]);
    }
    if (!minimum) {
      const bool negative = std::is_signed<SrcT>::value && static_cast<int64_t>(src[i]) < 0;
      if (negative || ord >= key_bound) record_error(err, kErrIndexOutOfRange);
    }
    const K k = static_cast<K>(ord - lo);
    keys[i] = k;
    add_histograms(s_hist, k, passes, digit);
  }
  __syncthreads();
  flush_histograms(s_hist, hist, passes, digit);
}

// Order-preserving unsigned image of the keys: min and max (for the bit width).
template <typename SrcT>
__global__ __launch_bounds__(256) void minmax_kernel(const SrcT *__restrict__ src, int64_t n,
                                                    unsigned long long *__restrict__ out) {
  unsigned long long lo = ~0ull, hi = 0;
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += gridDim.x * 256ll) {
    unsigned long long ord;
    if constexpr (std::is_signed<SrcT>::value)
      ord = static_cast<unsigned long long>(static_cast<int64_t>(src[i])) ^ 0x8000000000000000ull;
    else
      ord = static_cast<unsigned long long>(src[i]);
    lo = ord < lo ? ord : lo;
    hi = ord > hi ? ord : hi;
  }
  for (int off = 32; off > 0; off >>= 1) {
    const unsigned long long a = __shfl_xor(lo, off, 64);
    const unsigned long long b = __shfl_xor(hi, off, 64);
    lo = a < lo ? a : lo;
    hi = b > hi ? b : hi;
  }
  if ((threadIdx.x & 63) == 0) {
    atomicMin(&out[0], lo);
    atomicMax(&out[1], hi);
  }
}

__global__ void init_minmax_kernel(unsigned long long *out) {
  out[0] = ~0ull;
  out[1] = 0;
}

// ----------------------------------------------------------------------------
// onesweep radix pass (stable)
// ----------------------------------------------------------------------------
// kCarry: a second 32-bit value (the gradient row of each occurrence) moves
// with the key, so that the last pass leaves it in sorted order.
template <typename K, int DIGIT, bool kCarry>
__global__ __launch_bounds__(kOneThreads) void onesweep_kernel(
    const K *__restrict__ kin, const uint32_t *__restrict__ vin, K *__restrict__ kout,
    uint32_t *__restrict__ vout, const uint32_t *__restrict__ gin, uint32_t *__restrict__ gout,
    uint32_t n, int pass, const uint32_t *__restrict__ hist, uint32_t *status, uint32_t *ticket,
    int *err) {
  constexpr int kWaves = kOneThreads / 64;
  constexpr int kRadix = 1 << DIGIT;
  static_assert(kOneThreads >= kRadix, "one thread per digit");
  const int shift = pass * DIGIT;
  __shared__ uint32_t s_tile;
  __shared__ uint32_t s_wcnt[kWaves][kRadix];
  __shared__ uint32_t s_tile_start[kRadix];
  __shared__ uint32_t s_gbase[kRadix];
  __shared__ uint32_t s_scan[2][kWaves];
  __shared__ K s_keys[kOneTile];
  __shared__ uint32_t s_vals[kOneTile];
  __shared__ uint32_t s_gvals[kCarry ? kOneTile : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  if (tid == 0) s_tile = atomicAdd(ticket, 1u);
  for (int i = tid; i < kWaves * kRadix; i += kOneThreads) (&s_wcnt[0][0])[i] = 0;
  __syncthreads();
  const uint32_t tile = s_tile;
  const uint32_t base = tile * kOneTile;

  K key[kOneItems];
  uint32_t val[kOneItems];
  uint32_t gval[kCarry ? kOneItems : 1];
  uint32_t rank[kOneItems];
#pragma unroll
  for (int k = 0; k < kOneItems; ++k) {
    const uint32_t e = base + wave * (kOneItems * 64) + k * 64 + lane;
    if (e < n) {
      key[k] = kin[e];
      val[k] = vin ? vin[e] : e;
      if constexpr (kCarry) gval[k] = gin[e];
    } else {
      key[k] = 0;
      val[k] = 0;
      if constexpr (kCarry) gval[k] = 0;
    }
  }
  // Stable rank inside the tile: for every item the lanes holding the same
  // digit are found with wave64 ballots; the lowest of them advances the
  // wave's LDS counter of that digit by the group's size.  The counter reads
  // and writes of one wave stay in program order, so item k's groups precede
  // item k+1's.
  const uint64_t lt = lanemask_lt();
#pragma unroll
  for (int k = 0; k < kOneItems; ++k) {
    const uint32_t e = base + wave * (kOneItems * 64) + k * 64 + lane;
    const bool valid = e < n;
    const uint32_t d = valid ? (static_cast<uint32_t>(key[k] >> shift) & (kRadix - 1)) : 0;
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < DIGIT; ++b) {
      const bool bit = (d >> b) & 1u;
      const uint64_t bb = __ballot(bit);
      peers &= bit ? bb : ~bb;
    }
    const uint32_t before = __popcll(peers & lt);
    const uint32_t c = valid ? s_wcnt[wave][d] : 0;
    rank[k] = c + before;
    if (valid && before == 0) s_wcnt[wave][d] = c + static_cast<uint32_t>(__popcll(peers));
  }
  __syncthreads();

  // per digit (thread d < kRadix): wave-exclusive prefixes, tile totals,
  // tile-local and global bases
  const int d = tid;
  uint32_t total = 0;
  if (d < kRadix) {
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const uint32_t c = s_wcnt[w][d];
      s_wcnt[w][d] = total;
      total += c;
    }
  }
  const uint32_t tile_start = block_exclusive_scan<kOneThreads>(total, s_scan[0]);
  const uint32_t digit_base =
      block_exclusive_scan<kOneThreads>(d < kRadix ? digit_total(hist, pass, d) : 0u, s_scan[1]);
  if (d < kRadix) {
    const uint32_t prefix = lookback_exclusive(status, tile, kRadix, d, total, err);
    s_tile_start[d] = tile_start;
    s_gbase[d] = digit_base + prefix;
  }
  __syncthreads();

#pragma unroll
  for (int k = 0; k < kOneItems; ++k) {
    const uint32_t e = base + wave * (kOneItems * 64) + k * 64 + lane;
    if (e < n) {
      const uint32_t dk = static_cast<uint32_t>(key[k] >> shift) & (kRadix - 1);
      const uint32_t pos = s_tile_start[dk] + s_wcnt[wave][dk] + rank[k];
      s_keys[pos] = key[k];
      s_vals[pos] = val[k];
      if constexpr (kCarry) s_gvals[pos] = gval[k];
    }
  }
  __syncthreads();
  const uint32_t count = (n - base) < static_cast<uint32_t>(kOneTile) ? (n - base) : kOneTile;
  for (uint32_t p = tid; p < count; p += kOneThreads) {
    const K kk = s_keys[p];
    const uint32_t dk = static_cast<uint32_t>(kk >> shift) & (kRadix - 1);
    const uint32_t out = s_gbase[dk] + (p - s_tile_start[dk]);
    if (out < n) {  // always true unless a spin guard tripped
      kout[out] = kk;
      vout[out] = s_vals[p];
      if constexpr (kCarry) gout[out] = s_gvals[p];
    }
  }
}

// ----------------------------------------------------------------------------
// Block-wide inclusive count of per-element flags for a striped tile
// (element of item k, thread t = base + k*256 + t).  Returns per item the
// inclusive count within the tile; *tile_total gets the tile's count.
// ----------------------------------------------------------------------------
struct FlagScan {
  uint32_t incl[kSortItems];
};

__device__ __forceinline__ void tile_flag_scan(const bool (&flag)[kSortItems], uint32_t *s_cnt,
                                               FlagScan &out, uint32_t *tile_total) {
  constexpr int kWaves = kSortThreads / 64;
  static_assert(kSortItems * kWaves == 64, "one count per (item, wave) pair, scanned by one wave");
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const uint64_t le = lanemask_lt() | (1ull << lane);
  uint32_t within[kSortItems];
#pragma unroll
  for (int k = 0; k < kSortItems; ++k) {
    const uint64_t b = __ballot(flag[k]);
    within[k] = __popcll(b & le);
    if (lane == 0) s_cnt[k * kWaves + wave] = __popcll(b);
  }
  __syncthreads();
  if (tid < 64) {  // 64 counts in (item, wave) order -> exclusive scan
    const uint32_t v = s_cnt[tid];
    uint32_t incl = v;
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t y = __shfl_up(incl, off, 64);
      if (tid >= off) incl += y;
    }
    s_cnt[64 + tid] = incl - v;
    if (tid == 63) s_cnt[128] = incl;
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kSortItems; ++k) out.incl[k] = s_cnt[64 + k * kWaves + wave] + within[k];
  *tile_total = s_cnt[128];
}

// ----------------------------------------------------------------------------
// runs: segment heads of the sorted keys
// ----------------------------------------------------------------------------
// Number of key heads (first position of each distinct valid key) in each
// kSortTile tile of the sorted keys; the counts are then scanned by
// scan_counts_kernel so that every tile of runs_kernel knows its first run.
template <typename K>
__global__ __launch_bounds__(kSortThreads) void head_count_kernel(const K *__restrict__ sk,
                                                                 uint32_t n, K sentinel,
                                                                 int use_sentinel,
                                                                 uint32_t *__restrict__ counts) {
  __shared__ uint32_t s_sum[kSortThreads / 64];
  const uint32_t base = blockIdx.x * kSortTile;
  uint32_t c = 0;
#pragma unroll
  for (int k = 0; k < kSortItems; ++k) {
    const uint32_t j = base + k * kSortThreads + threadIdx.x;
    if (j < n) {
      const K key = sk[j];
      const bool valid = !(use_sentinel && key >= sentinel);
      c += (valid && (j == 0 || sk[j - 1] != key)) ? 1u : 0u;
    }
  }
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) c += __shfl_xor(c, m, 64);
  if ((threadIdx.x & 63) == 0) s_sum[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t t = 0;
#pragma unroll
    for (int w = 0; w < kSortThreads / 64; ++w) t += s_sum[w];
    counts[blockIdx.x] = t;
  }
}

// Up to this many tiles, runs_kernel and rank_kernel add up the per-tile
// counts of the tiles before theirs themselves (at most 8 L2-resident loads
// per thread) instead of waiting for a separate scan launch.
constexpr uint32_t kFusedPrefixTiles = 2048;

// Sum of counts[0 .. tile) over the block; every thread of the block calls it
// once, at the same point.
__device__ __forceinline__ uint32_t block_prefix_of_counts(const uint32_t *__restrict__ counts, uint32_t tile) {
  __shared__ uint32_t s_part[kSortThreads / 64];
  uint32_t v = 0;
  for (uint32_t i = threadIdx.x; i < tile; i += kSortThreads) v += counts[i];
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) v += __shfl_xor(v, m, 64);
  if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = v;
  __syncthreads();
  uint32_t t = 0;
#pragma unroll
  for (int w = 0; w < kSortThreads / 64; ++w) t += s_part[w];
  return t;
}

// First occurrences (head_flag bytes, 0 or 1) in each kSortTile tile of
// occurrences: 4 flags per thread (the flag array holds whole tiles).
__global__ __launch_bounds__(kSortThreads) void first_count_kernel(const uint8_t *__restrict__ head_flag,
                                                                  uint32_t *__restrict__ counts) {
  static_assert(kSortTile == kSortThreads * 4, "one 4-byte word of flags per thread");
  const uint32_t f = reinterpret_cast<const uint32_t *>(head_flag)[blockIdx.x * kSortThreads + threadIdx.x];
  uint32_t c = __popc(f);
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) c += __shfl_xor(c, m, 64);
  __shared__ uint32_t s_sum[kSortThreads / 64];
  if ((threadIdx.x & 63) == 0) s_sum[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t t = 0;
#pragma unroll
    for (int w = 0; w < kSortThreads / 64; ++w) t += s_sum[w];
    counts[blockIdx.x] = t;
  }
}

// In-place exclusive scan of per-tile counts: one block of 1024 threads.
__global__ __launch_bounds__(1024) void scan_counts_kernel(uint32_t *counts, uint32_t tiles) {
  __shared__ uint32_t s_scan[16];
  __shared__ uint32_t s_carry;
  if (threadIdx.x == 0) s_carry = 0;
  __syncthreads();
  for (uint32_t b = 0; b < tiles; b += 1024) {
    const uint32_t i = b + threadIdx.x;
    const uint32_t v = i < tiles ? counts[i] : 0u;
    const uint32_t ex = block_exclusive_scan<1024>(v, s_scan);
    const uint32_t carry = s_carry;
    if (i < tiles) counts[i] = carry + ex;
    __syncthreads();
    if (threadIdx.x == 1023) s_carry = carry + ex + v;
    __syncthreads();
  }
}

template <typename K>
__global__ __launch_bounds__(kSortThreads) void runs_kernel(
    const K *__restrict__ sk, const uint32_t *__restrict__ sv, uint32_t n, K sentinel,
    int use_sentinel, uint32_t *__restrict__ run_start, uint32_t *__restrict__ unit_first_run,
    uint8_t *__restrict__ head_flag, uint2 *__restrict__ head_run,
    uint32_t *__restrict__ meta, const uint32_t *__restrict__ head_prefix, int fused_prefix,
    uint32_t *__restrict__ run_key,
    const uint32_t *__restrict__ grad_row, int grad_sorted, int grad_ident, const float *__restrict__ scale,
    uint32_t *__restrict__ sorted_grad_row, float *__restrict__ sorted_scale,
    uint32_t *__restrict__ run_grad_row, float *__restrict__ run_scale, const uint32_t *reject) {
  __shared__ uint32_t s_cnt[160];
  const int tid = threadIdx.x;
  const uint32_t tile = blockIdx.x;
  const uint32_t base = tile * kSortTile;
  if (*reject) {  // a rejected batch has no runs: everything after the sort does nothing
    if (tile == 0 && tid == 0) {
      meta[0] = 0;
      meta[1] = 0;
      run_start[0] = 0;
    }
    return;
  }
  bool valid[kSortItems], head[kSortItems];
  K key[kSortItems];
#pragma unroll
  for (int k = 0; k < kSortItems; ++k) {
    const uint32_t j = base + k * kSortThreads + tid;
    valid[k] = false;
    head[k] = false;
    if (j < n) {
      key[k] = sk[j];
      valid[k] = !(use_sentinel && key[k] >= sentinel);
      head[k] = valid[k] && (j == 0 || sk[j - 1] != key[k]);
    }
  }
  FlagScan fs;
  uint32_t total;
  tile_flag_scan(head, s_cnt, fs, &total);
  // heads before this tile: scanned counts, or the raw counts added up here
  const uint32_t prefix = fused_prefix ? block_prefix_of_counts(head_prefix, tile) : head_prefix[tile];
#pragma unroll
  for (int k = 0; k < kSortItems; ++k) {
    const uint32_t j = base + k * kSortThreads + tid;
    if (!valid[k]) {
      if (j == 0 && j < n) {  // nothing valid at all
        meta[0] = 0;
        meta[1] = 0;
        run_start[0] = 0;
      }
      continue;
    }
    const uint32_t r = prefix + fs.incl[k] - 1;
    if (r >= n) continue;
    if (head[k]) {
      run_start[r] = j;
      if (run_key) run_key[r] = static_cast<uint32_t>(key[k]);
    }
    if ((j % kReduceUnit) == 0) unit_first_run[j / kReduceUnit] = r;
    const uint32_t o = sv[j];
    if (o < n) {
      if (head[k]) {
        // first occurrence of the key (the sort is stable): mark it for rank_kernel
        head_flag[o] = 1;  // one sorted position per occurrence: no other writer
        // the key travels with the run, so rank_kernel reads it in occurrence
        // order instead of from run_key at random
        head_run[o] = make_uint2(r, static_cast<uint32_t>(key[k]));
      }
      // per sorted position: the gradient row and scale of its occurrence
      // (grad_sorted: the sort has already put the rows in sorted order;
      // grad_ident: the occurrence is the row)
      if (grad_ident) {
        if (head[k]) run_grad_row[r] = o;
      } else if (sorted_grad_row) {
        if (grad_sorted) {
          if (head[k]) run_grad_row[r] = sorted_grad_row[j];
        } else {
          const uint32_t gr = grad_row[o];
          sorted_grad_row[j] = gr;
          if (head[k]) run_grad_row[r] = gr;
        }
      }
      if (sorted_scale) {
        const float sc = scale[o];
        sorted_scale[j] = sc;
        if (head[k]) run_scale[r] = sc;
      }
    }
    const bool last = (j + 1 == n) || (use_sentinel && sk[j + 1] >= sentinel);
    if (last) {
      meta[0] = j + 1;
      meta[1] = r + 1;
      run_start[r + 1] = j + 1;
    }
  }
}

// ----------------------------------------------------------------------------
// rank: first-occurrence order
// ----------------------------------------------------------------------------
enum UniqueSource : int { kUniqueNone = 0, kUniqueFromValues = 1, kUniqueFromSorted = 2 };

__global__ __launch_bounds__(kSortThreads) void rank_kernel(
    const uint8_t *__restrict__ head_flag, const uint2 *__restrict__ head_run, uint32_t n,
    const uint32_t *__restrict__ first_prefix, int fused_prefix, uint32_t tiles, uint32_t *__restrict__ run_rank,
    int64_t *__restrict__ first_indices, void *__restrict__ unique_out, int unique_source,
    const void *__restrict__ values, int value_bytes, int64_t *__restrict__ unique_count) {
  __shared__ uint32_t s_cnt[160];
  const int tid = threadIdx.x;
  const uint32_t tile = blockIdx.x;
  const uint32_t base = tile * kSortTile;
  bool first[kSortItems];
#pragma unroll
  for (int k = 0; k < kSortItems; ++k) {
    const uint32_t i = base + k * kSortThreads + tid;
    first[k] = (i < n) && head_flag[i] != 0;
  }
  FlagScan fs;
  uint32_t total;
  tile_flag_scan(first, s_cnt, fs, &total);
  // first occurrences before this tile: scanned counts, or the raw counts added up here
  const uint32_t prefix = fused_prefix ? block_prefix_of_counts(first_prefix, tile) : first_prefix[tile];
  if (tid == 0 && tile == tiles - 1 && unique_count) *unique_count = static_cast<int64_t>(prefix + total);
#pragma unroll
  for (int k = 0; k < kSortItems; ++k) {
    if (!first[k]) continue;
    const uint32_t i = base + k * kSortThreads + tid;
    const uint32_t rank = prefix + fs.incl[k] - 1;
    const uint2 hr = head_run[i];
    const uint32_t r = hr.x;
    if (rank >= n || r >= n) continue;
    run_rank[r] = rank;
    if (first_indices) first_indices[rank] = i;
    if (unique_source == kUniqueFromValues) {
      if (value_bytes == 8)
        static_cast<uint64_t *>(unique_out)[rank] = static_cast<const uint64_t *>(values)[i];
      else
        static_cast<uint32_t *>(unique_out)[rank] = static_cast<const uint32_t *>(values)[i];
    } else if (unique_source == kUniqueFromSorted) {
      static_cast<int64_t *>(unique_out)[rank] = static_cast<int64_t>(hr.y);  // 32-bit row keys
    }
  }
}

// inverse[occurrence] = rank of its key, one wave64 per unit of sorted positions.
template <typename K>
__global__ __launch_bounds__(256) void inverse_kernel(const K *__restrict__ sk,
                                                     const uint32_t *__restrict__ sv, uint32_t n,
                                                     const uint32_t *__restrict__ unit_first_run,
                                                     const uint32_t *__restrict__ run_rank,
                                                     int32_t *__restrict__ inverse) {
  static_assert(kReduceUnit == 64, "one wave per unit");
  const uint32_t j = blockIdx.x * 256u + threadIdx.x;
  const int lane = threadIdx.x & 63;
  const bool valid = j < n;
  const bool head = valid && j > 0 && sk[j] != sk[j - 1];
  const uint64_t heads = __ballot(head);
  if (!valid) return;
  const uint64_t le = (lane == 63) ? ~0ull : ((2ull << lane) - 1);
  const uint32_t r = unit_first_run[j / kReduceUnit] + __popcll(heads & le & ~1ull);
  const uint32_t o = sv[j];
  if (o < n && r < n) inverse[o] = static_cast<int32_t>(run_rank[r]);
}

int launch_update(int mode, int dtype, const UpdateArgs &a, const Shape &sh, hipStream_t s) {
  if (mode == kModeRows || mode == kModeUnique) return launch_update_rows(mode, a, sh, s);
  switch (dtype) {
    case FLARE_FLOAT32: return launch_update_f32(mode, a, sh, s);
    case FLARE_FLOAT16: return launch_update_f16(mode, a, sh, s);
    case FLARE_BFLOAT16: return launch_update_bf16(mode, a, sh, s);
    default:
      return fail(FLARE_ERR_DTYPE, "sparse embedding value dtype code %d is not float16, bfloat16 or float32", dtype);
  }
}

// Sort keys[0]/implicit iota by the low `bits` bits; returns the buffer index
// holding the result (0 or 1).  kCarry: w.grad_row moves with the keys and
// ends, sorted, in w.sorted_grad_row (the passes alternate between the two
// buffers, so the pass count must be odd).
template <typename K, int DIGIT, bool kCarry>
int run_passes(const Workspace &w, int passes, int *err, hipStream_t s, int *result) {
  const uint32_t n = static_cast<uint32_t>(w.n);
  int cur = 0;
  uint32_t *g[2] = {w.grad_row, w.sorted_grad_row};
  for (int p = 0; p < passes; ++p) {
    onesweep_kernel<K, DIGIT, kCarry><<<w.sort_tiles, kOneThreads, 0, s>>>(
        static_cast<const K *>(w.keys[cur]), p == 0 ? nullptr : w.vals[cur],
        static_cast<K *>(w.keys[cur ^ 1]), w.vals[cur ^ 1], g[p & 1], g[(p & 1) ^ 1], n, p,
        w.hist, w.sort_status + (static_cast<size_t>(p) * w.sort_tiles << DIGIT),
        w.tickets + p, err);
    FLARE_TRY_HIP(hipGetLastError());
    cur ^= 1;
  }
  *result = cur;
  return FLARE_OK;
}

// Whether a sort by this plan carries the gradient rows (32-bit keys, digits
// of at most 9 bits so that the third staging array fits in LDS, and an odd
// pass count so that the rows end in w.sorted_grad_row).
bool carries_grad_rows(const Workspace &w, const RadixPlan &plan, int key_bytes) {
  return key_bytes == 4 && w.grad_row && w.sorted_grad_row && plan.digit_bits <= 9 && (plan.passes & 1);
}

template <typename K>
int run_sort(const Workspace &w, const RadixPlan &plan, int *err, hipStream_t s, int *result,
             bool carry = false) {
  if constexpr (sizeof(K) == 4) {
    if (carry) {
      if (plan.digit_bits == 9) return run_passes<K, 9, true>(w, plan.passes, err, s, result);
      return run_passes<K, 8, true>(w, plan.passes, err, s, result);
    }
    if (plan.digit_bits == 9) return run_passes<K, 9, false>(w, plan.passes, err, s, result);
    if (plan.digit_bits == 10) return run_passes<K, 10, false>(w, plan.passes, err, s, result);
  }
  return run_passes<K, 8, false>(w, plan.passes, err, s, result);
}


// Runs and first-occurrence ranks of sorted keys: head counts per tile and
// their scan, runs (run ids; each key's first occurrence marked in the
// occurrence bitmap), first occurrences per occurrence tile and their scan,
// then ranks.
struct RunsOutputs {
  uint32_t *run_key;              // or null
  const uint32_t *grad_row;       // gathered into sorted order when non-null
  int grad_sorted;                // 1: the sort carried the rows into sorted order
  int grad_ident;                 // 1: each occurrence is its own gradient row (not stored)
  const float *scale;             // gathered into sorted order when non-null
  int64_t *first_indices;         // or null
  void *unique_out;               // or null
  int unique_source;
  const void *values;
  int value_bytes;
  int64_t *unique_count;          // or null
};

template <typename K>
int runs_and_rank(const Workspace &w, const K *sk, const uint32_t *sv, uint32_t n, K sentinel,
                  int use_sentinel, const RunsOutputs &o, hipStream_t s) {
  uint32_t *head_prefix = w.scan_status;
  uint32_t *first_prefix = w.scan_status + w.tiles;
  const int fused = w.tiles <= kFusedPrefixTiles ? 1 : 0;
  head_count_kernel<K><<<w.tiles, kSortThreads, 0, s>>>(sk, n, sentinel, use_sentinel, head_prefix);
  if (!fused) scan_counts_kernel<<<1, 1024, 0, s>>>(head_prefix, w.tiles);
  runs_kernel<K><<<w.tiles, kSortThreads, 0, s>>>(
      sk, sv, n, sentinel, use_sentinel, w.run_start, w.unit_first_run, w.head_flag, w.head_run,
      w.meta, head_prefix, fused, o.run_key, o.grad_row, o.grad_sorted, o.grad_ident, o.scale,
      o.grad_row ? w.sorted_grad_row : nullptr, o.scale ? w.sorted_scale : nullptr,
      w.run_grad_row, w.run_scale, w.meta + 3);
  first_count_kernel<<<w.tiles, kSortThreads, 0, s>>>(w.head_flag, first_prefix);
  if (!fused) scan_counts_kernel<<<1, 1024, 0, s>>>(first_prefix, w.tiles);
  rank_kernel<<<w.tiles, kSortThreads, 0, s>>>(
      w.head_flag, w.head_run, n, first_prefix, fused, w.tiles, w.run_rank, o.first_indices,
      o.unique_out, o.unique_source, o.values, o.value_bytes, o.unique_count);
  FLARE_TRY_HIP(hipGetLastError());
  return FLARE_OK;
}

// After prepare: sort, runs, rank.  Sorted u32 keys/vals are left in
// w.keys[*sorted] / w.vals[*sorted].
// scale_src: per-occurrence scale gathered into sorted order (mean divisors), or null.
int dedup_rows(const Workspace &w, const RadixPlan &plan, uint32_t sentinel, int *err, hipStream_t s,
               int *sorted, int64_t *first_indices, void *unique_out, int unique_source,
               const void *values, int value_bytes, int64_t *unique_count,
               const float *scale_src, bool grad_ident = false) {
  // grad_ident: the occurrence is its own gradient row, nothing to carry or gather
  const bool carry = !grad_ident && carries_grad_rows(w, plan, 4);
  FLARE_TRY(run_sort<uint32_t>(w, plan, err, s, sorted, carry));
  const uint32_t n = static_cast<uint32_t>(w.n);
  const uint32_t *sk = static_cast<const uint32_t *>(w.keys[*sorted]);
  RunsOutputs o{w.run_key, w.grad_row, carry ? 1 : 0, grad_ident ? 1 : 0, scale_src, first_indices, unique_out,
                unique_source, values, value_bytes, unique_count};
  return runs_and_rank<uint32_t>(w, sk, w.vals[*sorted], n, sentinel, 1, o, s);
}

int optimizer_mode(const flare_optimizer *opt, int *mode) {
  if (!opt) return fail(FLARE_ERR_ARGUMENT, "optimizer configuration is required");
  if (opt->weight_decay != 0.0)
    return fail(FLARE_ERR_ARGUMENT, "sparse optimizer weight_decay must be 0, got %g", opt->weight_decay);
  switch (opt->kind) {
    case FLARE_OPT_NONE: *mode = kModeUnique; return FLARE_OK;
    case FLARE_OPT_SGD: *mode = kModeSgd; return FLARE_OK;
    case FLARE_OPT_ADAM: *mode = kModeAdam; return FLARE_OK;
    case FLARE_OPT_ROWWISE_ADAGRAD: *mode = kModeAdagrad; return FLARE_OK;
    default: return fail(FLARE_ERR_ARGUMENT, "unsupported sparse optimizer kind %d", opt->kind);
  }
}

void fill_optimizer(UpdateArgs &a, const flare_optimizer *opt) {
  a.lr = static_cast<float>(opt->learning_rate);
  a.eps = static_cast<float>(opt->eps);
  a.b1 = static_cast<float>(opt->beta1);
  a.b2 = static_cast<float>(opt->beta2);
  a.omb1 = static_cast<float>(1.0 - opt->beta1);
  a.omb2 = static_cast<float>(1.0 - opt->beta2);
  a.ln_b1 = std::log(opt->beta1);
  a.ln_b2 = std::log(opt->beta2);
}

int check_state(int mode, float *s0, float *s1, int32_t *step) {
  if (mode == kModeAdagrad && !s0) return fail(FLARE_ERR_ARGUMENT, "row-wise Adagrad requires the accumulator state");
  if (mode == kModeAdam && (!s0 || !s1 || !step))
    return fail(FLARE_ERR_ARGUMENT, "Adam requires m, v and step state");
  return FLARE_OK;
}

int check_workspace(const Workspace &need, size_t have) {
  if (have < need.total_bytes)
    return fail(FLARE_ERR_WORKSPACE, "workspace of %zu bytes is smaller than the %zu bytes required", have, need.total_bytes);
  // the layout starts at the workspace's first byte (the histograms) and its parts are
  // read and written with 16-byte vectors
  if (!aligned(need.hist, 16)) return fail(FLARE_ERR_WORKSPACE, "workspace must be 16-byte aligned");
  return FLARE_OK;
}

bool vec4_ok(const void *p) { return aligned(p, 16); }

// Shared tail of the keyed-row entry points (scatter, scatter_pooled, sparse_update).
int reduce_rows(const Workspace &w, const RadixPlan &plan, uint32_t sentinel, int *err, hipStream_t s, int mode,
                int dtype, int dim, const void *grad, int grad_mode, uint32_t grad_div,
                void *out, void *table, float *s0, float *s1, int32_t *step,
                const flare_optimizer *opt, int32_t norm_steps, int grad_dtype = FLARE_FLOAT32,
                int check_finite = 0, int32_t *nonfinite_out = nullptr, int out_bf16 = 0) {
  int sorted = 0;
  FLARE_TRY(dedup_rows(w, plan, sentinel, err, s, &sorted, nullptr, nullptr, kUniqueNone, nullptr,
                       0, nullptr, nullptr));
  UpdateArgs a{};
  a.sk = static_cast<const uint32_t *>(w.keys[sorted]);
  a.sv = w.vals[sorted];
  a.run_start = w.run_start;
  a.unit_first_run = w.unit_first_run;
  a.meta = w.meta;
  a.run_rank = w.run_rank;
  a.grad = grad;
  a.grad_bf16 = grad_dtype == FLARE_BFLOAT16;
  a.grad_mode = grad_mode;
  a.grad_div = grad_div;
  if (check_finite) {
    FLARE_TRY(launch_finite_check(grad, grad_dtype, w.n * static_cast<int64_t>(dim), w.meta + 4, nonfinite_out,
                                  err, s));
    a.reject = w.meta + 4;
  }
  a.scale_mode = kScaleNone;
  a.use_norm = norm_steps != 1;
  a.norm = static_cast<float>(norm_steps);
  a.dim = dim;
  a.partial = w.partial;
  a.sums = w.sums;
  a.run_key = w.run_key;
  a.hot_runs = w.hot_runs;
  a.out = out;
  a.out_bf16 = out_bf16;
  a.table = table;
  a.s0 = s0;
  a.s1 = s1;
  a.step = step;
  if (opt) fill_optimizer(a, opt);
  a.units = w.units;
  a.n = static_cast<uint32_t>(w.n);
  a.err = err;
  const bool v4 = vec4_ok(grad) && (out ? vec4_ok(out) : true) && (table ? aligned(table, 8) : true) &&
                  (mode == kModeAdam ? (vec4_ok(s0) && vec4_ok(s1)) : true) && vec4_ok(w.partial);
  // 16-byte lanes for bfloat16 gradients (every vector then 16-byte aligned)
  const bool v8 = v4 && a.grad_bf16 && (table ? aligned(table, 16) : true);
  Shape sh;
  FLARE_TRY(choose_shape(dim, v4, &sh, v8));
  return launch_update(mode, dtype, a, sh, s);
}

}  // namespace
}  // namespace flare

using namespace flare;

// ----------------------------------------------------------------------------
// scatter / scatter_pooled
// ----------------------------------------------------------------------------
extern "C" int flare_set_update_events(void *const *events, int32_t count) {
  if (count < 0 || count > 4 || (count > 0 && events == nullptr))
    return fail(FLARE_ERR_ARGUMENT, "update events: count must be 0..4 with that many events, got %d", count);
  for (int i = 0; i < count; ++i) t_update_events[i] = static_cast<hipEvent_t>(events[i]);
  t_update_event_count = count;
  return FLARE_OK;
}

extern "C" size_t flare_scatter_workspace_bytes(int64_t slots, int64_t emb_rows, int32_t dim) {
  (void)emb_rows;
  return layout_workspace(nullptr, slots, 4, std::max(dim, 1), false, false, true).total_bytes;
}

static int scatter_common(int64_t emb_rows, int32_t dim, const int32_t *inverse, int64_t slots,
                          int32_t pad_index, const float *grad, uint32_t grad_div, void *out,
                          int32_t out_dtype, void *workspace, size_t workspace_bytes, void *stream) {
  if (dim <= 0 || emb_rows < 0 || slots < 0) return fail(FLARE_ERR_SHAPE, "invalid scatter sizes");
  if (out_dtype != FLARE_FLOAT32 && out_dtype != FLARE_BFLOAT16)
    return fail(FLARE_ERR_DTYPE, "scatter output dtype must be float32 or bfloat16, got dtype code %d", out_dtype);
  if (slots > kMaxOccurrences) return fail(FLARE_ERR_LIMIT, "too many inverse slots (%lld)", static_cast<long long>(slots));
  if (emb_rows >= 0xffffffffll) return fail(FLARE_ERR_LIMIT, "too many embedding rows");
  hipStream_t s = as_stream(stream);
  const int out_bf16 = out_dtype == FLARE_BFLOAT16 ? 1 : 0;
  if (emb_rows > 0)  // rows no slot reaches are zero (a zero fill kernel: capturable)
    FLARE_TRY(flare_zero_bytes(out, emb_rows * static_cast<int64_t>(dim) * (out_bf16 ? 2 : 4), stream));
  if (slots == 0 || emb_rows == 0) return FLARE_OK;
  Workspace w = layout_workspace(workspace, slots, 4, dim, false, false, true);
  FLARE_TRY(check_workspace(w, workspace_bytes));
  int st = FLARE_OK;
  int *err = device_error_word(&st);
  if (!err) return st;
  const uint32_t sentinel = static_cast<uint32_t>(emb_rows);
  const RadixPlan plan = radix_plan(bits_for(sentinel), 4);
  FLARE_TRY(launch_zero(workspace, zero_bytes_for(w, plan), s));
  const int grid = static_cast<int>(std::min<int64_t>(ceil_div(slots, 256), 2048));
  prepare_rows_kernel<int32_t><<<grid, 256, 0, s>>>(inverse, slots, emb_rows, 1, pad_index,
                                                   plan.passes, plan.digit_bits,
                                                   static_cast<uint32_t *>(w.keys[0]),
                                                   w.hist, err);
  FLARE_TRY_HIP(hipGetLastError());
  return reduce_rows(w, plan, sentinel, err, s, kModeRows, FLARE_FLOAT32, dim, grad,
                     grad_div == 1 ? kGradRowOcc : kGradRowDiv, grad_div, out, nullptr, nullptr,
                     nullptr, nullptr, nullptr, 1, FLARE_FLOAT32, 0, nullptr, out_bf16);
}

extern "C" int flare_scatter(int64_t emb_rows, int32_t dim, const int32_t *inverse, int64_t slots,
                             int32_t pad_index, const float *grad, float *out, void *workspace,
                             size_t workspace_bytes, void *stream) {
  return scatter_common(emb_rows, dim, inverse, slots, pad_index, grad, 1, out, FLARE_FLOAT32, workspace,
                        workspace_bytes, stream);
}

extern "C" int flare_scatter_ex(int64_t emb_rows, int32_t dim, const int32_t *inverse, int64_t slots,
                                int32_t pad_index, const float *grad, void *out, int32_t out_dtype,
                                void *workspace, size_t workspace_bytes, void *stream) {
  return scatter_common(emb_rows, dim, inverse, slots, pad_index, grad, 1, out, out_dtype, workspace,
                        workspace_bytes, stream);
}

static int scatter_pooled_common(int64_t emb_rows, int32_t dim, const int32_t *inverse, int64_t slots,
                                 int32_t pad_index, const float *grad, int64_t batch, int32_t features,
                                 int32_t max_elements, void *out, int32_t out_dtype, void *workspace,
                                 size_t workspace_bytes, void *stream) {
  if (features <= 0 || max_elements <= 0)
    return fail(FLARE_ERR_WIDTH, "Sparse embedding pooled operations require positive target widths, got (%d, %d).", features, max_elements);
  if (slots != batch * features * static_cast<int64_t>(max_elements))
    return fail(FLARE_ERR_SHAPE, "pooled scatter inverse slots must match gradient rows times max_elements");
  return scatter_common(emb_rows, dim, inverse, slots, pad_index, grad,
                        static_cast<uint32_t>(max_elements), out, out_dtype, workspace, workspace_bytes,
                        stream);
}

extern "C" int flare_scatter_pooled(int64_t emb_rows, int32_t dim, const int32_t *inverse,
                                    int64_t slots, int32_t pad_index, const float *grad,
                                    int64_t batch, int32_t features, int32_t max_elements,
                                    float *out, void *workspace, size_t workspace_bytes,
                                    void *stream) {
  return scatter_pooled_common(emb_rows, dim, inverse, slots, pad_index, grad, batch, features, max_elements,
                               out, FLARE_FLOAT32, workspace, workspace_bytes, stream);
}

extern "C" int flare_scatter_pooled_ex(int64_t emb_rows, int32_t dim, const int32_t *inverse,
                                       int64_t slots, int32_t pad_index, const float *grad,
                                       int64_t batch, int32_t features, int32_t max_elements,
                                       void *out, int32_t out_dtype, void *workspace,
                                       size_t workspace_bytes, void *stream) {
  return scatter_pooled_common(emb_rows, dim, inverse, slots, pad_index, grad, batch, features, max_elements,
                               out, out_dtype, workspace, workspace_bytes, stream);
}

// ----------------------------------------------------------------------------
// unique_first_occurrence
// ----------------------------------------------------------------------------
extern "C" size_t flare_unique_workspace_bytes(int64_t n, int32_t key_dtype) {
  (void)key_dtype;
  return layout_workspace(nullptr, n, 8, 1, false, false, false).total_bytes + 256;
}

namespace flare {
namespace {
template <typename SrcT>
int unique_typed(const SrcT *values, int64_t n, int64_t key_bound, void *unique_out,
                 int32_t *inverse_out, int64_t *first_indices_out, int64_t *unique_count,
                 void *workspace, size_t workspace_bytes, hipStream_t s) {
  Workspace w8 = layout_workspace(workspace, n, 8, 1, false, false, false);
  FLARE_TRY(check_workspace(w8, workspace_bytes > 256 ? workspace_bytes - 256 : 0));
  int st = FLARE_OK;
  int *err = device_error_word(&st);
  if (!err) return st;
  unsigned long long *mm = reinterpret_cast<unsigned long long *>(static_cast<char *>(workspace) + w8.total_bytes);
  const int grid = static_cast<int>(std::min<int64_t>(ceil_div(n, 256), 2048));
  uint64_t range;
  const uint64_t *minimum = nullptr;
  if (key_bound > 0) {
    range = static_cast<uint64_t>(key_bound - 1);
  } else {
    init_minmax_kernel<<<1, 1, 0, s>>>(mm);
    minmax_kernel<SrcT><<<grid, 256, 0, s>>>(values, n, mm);
    FLARE_TRY_HIP(hipGetLastError());
    unsigned long long host[2];
    FLARE_TRY_HIP(hipMemcpyAsync(host, mm, sizeof(host), hipMemcpyDeviceToHost, s));
    FLARE_TRY_HIP(hipStreamSynchronize(s));
    range = host[1] - host[0];
    minimum = reinterpret_cast<const uint64_t *>(mm);
  }
  const int bits = bits_for(range);
  const int value_bytes = sizeof(SrcT);
  if (bits <= 32) {
    // same base pointer, 4-byte keys
    Workspace w = layout_workspace(workspace, n, 4, 1, false, false, false);
    const RadixPlan plan = radix_plan(bits, 4);
    FLARE_TRY(launch_zero(workspace, zero_bytes_for(w, plan), s));
    prepare_generic_kernel<SrcT, uint32_t><<<grid, 256, 0, s>>>(values, n, minimum,
                                                                static_cast<uint64_t>(key_bound), plan.passes,
                                                                plan.digit_bits,
                                                                static_cast<uint32_t *>(w.keys[0]), w.hist, err);
    FLARE_TRY_HIP(hipGetLastError());
    int sorted = 0;
    FLARE_TRY(run_sort<uint32_t>(w, plan, err, s, &sorted));
    RunsOutputs o{w.run_key, nullptr, 0, 0, nullptr, first_indices_out, unique_out, kUniqueFromValues,
                  values, value_bytes, unique_count};
    FLARE_TRY(runs_and_rank<uint32_t>(w, static_cast<const uint32_t *>(w.keys[sorted]), w.vals[sorted],
                                      static_cast<uint32_t>(n), 0u, 0, o, s));
    inverse_kernel<uint32_t><<<static_cast<int>(ceil_div(n, 256)), 256, 0, s>>>(
        static_cast<const uint32_t *>(w.keys[sorted]), w.vals[sorted], static_cast<uint32_t>(n),
        w.unit_first_run, w.run_rank, inverse_out);
    FLARE_TRY_HIP(hipGetLastError());
    return FLARE_OK;
  }
  Workspace w = w8;
  const RadixPlan plan = radix_plan(bits, 8);
  FLARE_TRY(launch_zero(workspace, zero_bytes_for(w, plan), s));
  prepare_generic_kernel<SrcT, uint64_t><<<grid, 256, 0, s>>>(values, n, minimum,
                                                              static_cast<uint64_t>(key_bound), plan.passes,
                                                              plan.digit_bits,
                                                              static_cast<uint64_t *>(w.keys[0]), w.hist, err);
  FLARE_TRY_HIP(hipGetLastError());
  int sorted = 0;
  FLARE_TRY(run_sort<uint64_t>(w, plan, err, s, &sorted));
  RunsOutputs o{nullptr, nullptr, 0, 0, nullptr, first_indices_out, unique_out, kUniqueFromValues,
                values, value_bytes, unique_count};
  FLARE_TRY(runs_and_rank<uint64_t>(w, static_cast<const uint64_t *>(w.keys[sorted]), w.vals[sorted],
                                    static_cast<uint32_t>(n), 0ull, 0, o, s));
  inverse_kernel<uint64_t><<<static_cast<int>(ceil_div(n, 256)), 256, 0, s>>>(
      static_cast<const uint64_t *>(w.keys[sorted]), w.vals[sorted], static_cast<uint32_t>(n),
      w.unit_first_run, w.run_rank, inverse_out);
  FLARE_TRY_HIP(hipGetLastError());
  return FLARE_OK;
}
}  // namespace
}  // namespace flare

extern "C" int flare_unique_first_occurrence(const void *values, int32_t key_dtype, int64_t n,
                                             int64_t key_bound, void *unique_out,
                                             int32_t *inverse_out, int64_t *first_indices_out,
                                             int64_t *unique_count, void *workspace,
                                             size_t workspace_bytes, void *stream) {
  if (n < 0) return fail(FLARE_ERR_SHAPE, "negative key count");
  if (n > kMaxOccurrences) return fail(FLARE_ERR_LIMIT, "too many keys (%lld)", static_cast<long long>(n));
  hipStream_t s = as_stream(stream);
  if (n == 0) {
    if (unique_count) FLARE_TRY(launch_zero_count(unique_count, s));
    return FLARE_OK;
  }
  switch (key_dtype) {
    case FLARE_INT32: return unique_typed(static_cast<const int32_t *>(values), n, key_bound, unique_out, inverse_out, first_indices_out, unique_count, workspace, workspace_bytes, s);
    case FLARE_UINT32: return unique_typed(static_cast<const uint32_t *>(values), n, key_bound, unique_out, inverse_out, first_indices_out, unique_count, workspace, workspace_bytes, s);
    case FLARE_INT64: return unique_typed(static_cast<const int64_t *>(values), n, key_bound, unique_out, inverse_out, first_indices_out, unique_count, workspace, workspace_bytes, s);
    case FLARE_UINT64: return unique_typed(static_cast<const uint64_t *>(values), n, key_bound, unique_out, inverse_out, first_indices_out, unique_count, workspace, workspace_bytes, s);
    default: return fail(FLARE_ERR_DTYPE, "sparse unique requires integer keys, got dtype code %d", key_dtype);
  }
}

// ----------------------------------------------------------------------------
// unique_first_occurrence without allocating: the workspace is `scratch`, a
// fixed array every GPU holds from the moment the code object loads until the
// process ends.  Host code uses the address hipGetSymbolAddress returns for
// the current device (kept per device), never the array's name: in host code
// that name is only a stand-in for the symbol, not a device address.
// ----------------------------------------------------------------------------
namespace flare {
namespace {
constexpr size_t kNoAllocScratchBytes = size_t{48} << 20;  // 2^20 keys of any dtype fit
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
std::mutex g_scratch_mutex;
void *g_scratch[64] = {};

// The current device's scratch address, looked up once per device (with it current).
int scratch_address(void **out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= 64)
    return hip_fail(e == hipSuccess ? hipErrorInvalidDevice : e, "hipGetDevice");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return hip_fail(e == hipSuccess ? hipErrorInvalidSymbol : e, "hipGetSymbolAddress(scratch)");
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return FLARE_OK;
}
}  // namespace
}  // namespace flare

extern "C" int flare_unique_first_occurrence_noalloc(const void *values, int32_t key_dtype, int64_t n,
                                                     int64_t key_bound, void *unique_out, int32_t *inverse_out,
                                                     int64_t *first_indices_out, int64_t *unique_count,
                                                     void *stream) {
  if (n < 0) return fail(FLARE_ERR_SHAPE, "negative key count");
  if (key_bound <= 0)
    return fail(FLARE_ERR_ARGUMENT, "the allocation-free unique needs key_bound > 0 (it reads nothing back to the host)");
  const size_t need = flare_unique_workspace_bytes(n, key_dtype);
  if (need > kNoAllocScratchBytes)
    return fail(FLARE_ERR_LIMIT, "%lld keys need %zu bytes of workspace; the allocation-free unique holds %zu "
                "(at most 1048576 keys)", static_cast<long long>(n), need, kNoAllocScratchBytes);
  void *workspace = nullptr;
  FLARE_TRY(scratch_address(&workspace));
  return flare_unique_first_occurrence(values, key_dtype, n, key_bound, unique_out, inverse_out, first_indices_out,
                                       unique_count, workspace, kNoAllocScratchBytes, stream);
}

// ----------------------------------------------------------------------------
// sparse_update (store accumulate_gradients + optimizer_step)
// ----------------------------------------------------------------------------
extern "C" size_t flare_sparse_update_workspace_bytes(int64_t n, int64_t rows, int32_t dim) {
  (void)rows;
  return layout_workspace(nullptr, n, 4, std::max(dim, 1), false, false, true, true).total_bytes;
}

namespace flare {
namespace {
int check_grad_dtype(int32_t grad_dtype) {
  if (grad_dtype != FLARE_FLOAT32 && grad_dtype != FLARE_BFLOAT16)
    return fail(FLARE_ERR_DTYPE, "sparse embedding gradient_transport_dtype must be one of ['bfloat16', 'float32'], "
                "got dtype code %d", grad_dtype);
  return FLARE_OK;
}
}  // namespace
}  // namespace flare

extern "C" int flare_check_finite(const void *values, int32_t dtype, int64_t count, int32_t *nonfinite_out,
                                  void *stream) {
  if (count < 0) return fail(FLARE_ERR_SHAPE, "negative element count");
  if (!nonfinite_out) return fail(FLARE_ERR_ARGUMENT, "nonfinite_out is required");
  if (count > 0 && !values) return fail(FLARE_ERR_ARGUMENT, "values are null");
  int st = FLARE_OK;
  int *err = device_error_word(&st);
  if (!err) return st;
  return launch_finite_check(values, dtype, count, nullptr, nonfinite_out, err, as_stream(stream));
}

extern "C" int flare_sparse_update(void *table, int32_t value_dtype, int64_t rows, int32_t dim,
                                   float *state0, float *state1, int32_t *step,
                                   const flare_optimizer *optimizer, const int64_t *keys, int64_t n,
                                   const float *grad, int32_t normalization_steps, void *workspace,
                                   size_t workspace_bytes, void *stream) {
  return flare_sparse_update_ex(table, value_dtype, rows, dim, state0, state1, step, optimizer, keys, n, grad,
                                FLARE_FLOAT32, 0, nullptr, normalization_steps, workspace, workspace_bytes, stream);
}

extern "C" int flare_sparse_update_ex(void *table, int32_t value_dtype, int64_t rows, int32_t dim,
                                      float *state0, float *state1, int32_t *step,
                                      const flare_optimizer *optimizer, const int64_t *keys, int64_t n,
                                      const void *grad, int32_t grad_dtype, int32_t check_finite,
                                      int32_t *nonfinite_out, int32_t normalization_steps, void *workspace,
                                      size_t workspace_bytes, void *stream) {
  FLARE_TRY(check_grad_dtype(grad_dtype));
  if (storage_bytes(value_dtype) == 0)
    return fail(FLARE_ERR_DTYPE, "sparse embedding value dtype code %d is not float16, bfloat16 or float32", value_dtype);
  if (dim <= 0 || rows < 0 || n < 0) return fail(FLARE_ERR_SHAPE, "invalid sparse update sizes");
  if (normalization_steps <= 0) return fail(FLARE_ERR_ARGUMENT, "normalization_steps must be a positive integer");
  if (n > kMaxOccurrences) return fail(FLARE_ERR_LIMIT, "too many keys (%lld)", static_cast<long long>(n));
  if (rows >= 0xffffffffll) return fail(FLARE_ERR_LIMIT, "too many table rows");
  int mode = 0;
  FLARE_TRY(optimizer_mode(optimizer, &mode));
  if (mode == kModeUnique) return fail(FLARE_ERR_ARGUMENT, "sparse update requires an optimizer (SGD, Adam or row-wise Adagrad)");
  FLARE_TRY(check_state(mode, state0, state1, step));
  if (n == 0 || rows == 0) {  // nothing to update; a requested check still reports
    if (!check_finite || !nonfinite_out) return FLARE_OK;
    int st = FLARE_OK;
    int *err = device_error_word(&st);
    if (!err) return st;
    return launch_finite_check(grad, grad_dtype, n * static_cast<int64_t>(dim), nullptr, nonfinite_out, err,
                               as_stream(stream));
  }
  Workspace w = layout_workspace(workspace, n, 4, dim, false, false, true, true);
  FLARE_TRY(check_workspace(w, workspace_bytes));
  int st = FLARE_OK;
  int *err = device_error_word(&st);
  if (!err) return st;
  hipStream_t s = as_stream(stream);
  const uint32_t sentinel = static_cast<uint32_t>(rows);
  const RadixPlan plan = radix_plan(bits_for(sentinel), 4);
  FLARE_TRY(launch_zero(workspace, zero_bytes_for(w, plan), s));
  const int grid = static_cast<int>(std::min<int64_t>(ceil_div(n, 256), 2048));
  prepare_rows_kernel<int64_t><<<grid, 256, 0, s>>>(keys, n, rows, 0, 0, plan.passes, plan.digit_bits,
                                                   static_cast<uint32_t *>(w.keys[0]),
                                                   w.hist, err);
  FLARE_TRY_HIP(hipGetLastError());
  return reduce_rows(w, plan, sentinel, err, s, mode, value_dtype, dim, grad, kGradRowOcc, 1,
                     nullptr, table, state0, state1, step, optimizer, normalization_steps, grad_dtype,
                     check_finite, nonfinite_out);
}

// ----------------------------------------------------------------------------
// pooled_backward (fused scatter_pooled + accumulate + optimizer_step)
// ----------------------------------------------------------------------------
extern "C" size_t flare_pooled_backward_workspace_bytes(int64_t n, int64_t rows, int32_t dim) {
  (void)rows;
  return layout_workspace(nullptr, n, 4, std::max(dim, 1), true, true, true, true).total_bytes;
}

namespace flare {
namespace {
int check_pooled_args(int64_t rows, int32_t dim, int32_t num_tables, int64_t batch, int64_t n,
                      int32_t pooling, const float *weights_if_needed, bool weights_required) {
  if (dim <= 0 || rows < 0 || num_tables <= 0 || batch < 0 || n < 0)
    return fail(FLARE_ERR_SHAPE, "invalid pooled backward sizes");
  if (n > kMaxOccurrences) return fail(FLARE_ERR_LIMIT, "too many occurrences (%lld)", static_cast<long long>(n));
  if (rows >= 0xffffffffll) return fail(FLARE_ERR_LIMIT, "too many table rows");
  if (pooling != FLARE_POOL_SUM && pooling != FLARE_POOL_MEAN && pooling != FLARE_POOL_WEIGHTED)
    return fail(FLARE_ERR_ARGUMENT, "unknown pooling mode %d", pooling);
  if (weights_required && pooling == FLARE_POOL_WEIGHTED && !weights_if_needed)
    return fail(FLARE_ERR_ARGUMENT, "weighted pooling requires per-sample weights");
  return FLARE_OK;
}

int check_layout(int32_t layout) {
  const int32_t base = layout & ~FLARE_LAYOUT_ONE_ID_PER_BAG;
  if (base != FLARE_LAYOUT_SAMPLE_MAJOR && base != FLARE_LAYOUT_TABLE_MAJOR)
    return fail(FLARE_ERR_ARGUMENT, "unknown pooled row layout %d", layout);
  return FLARE_OK;
}
}  // namespace
}  // namespace flare

extern "C" int flare_pooled_dedup(const void *ids, int32_t id_dtype, int64_t n,
                                  const int64_t *offsets, int32_t num_tables, int64_t batch,
                                  const int64_t *row_base, int64_t rows, int32_t dim,
                                  int32_t pooling, int32_t layout, int64_t *unique_out,
                                  int64_t *first_indices_out, int64_t *unique_count,
                                  void *workspace, size_t workspace_bytes, void *stream) {
  if (id_dtype != FLARE_INT32 && id_dtype != FLARE_INT64)
    return fail(FLARE_ERR_DTYPE, "CSR ids must be int32 or int64, got dtype code %d", id_dtype);
  FLARE_TRY(check_pooled_args(rows, dim, num_tables, batch, n, pooling, nullptr, false));
  FLARE_TRY(check_layout(layout));
  const int table_major = (layout & ~FLARE_LAYOUT_ONE_ID_PER_BAG) == FLARE_LAYOUT_TABLE_MAJOR ? 1 : 0;
  const int one_id = (layout & FLARE_LAYOUT_ONE_ID_PER_BAG) ? 1 : 0;
  hipStream_t s = as_stream(stream);
  const int64_t bags = batch * num_tables;
  if (n == 0 || bags == 0) {
    if (unique_count) FLARE_TRY(launch_zero_count(unique_count, s));
    return FLARE_OK;
  }
  Workspace w = layout_workspace(workspace, n, 4, dim, true, true, true, true);
  FLARE_TRY(check_workspace(w, workspace_bytes));
  int st = FLARE_OK;
  int *err = device_error_word(&st);
  if (!err) return st;
  const uint32_t sentinel = static_cast<uint32_t>(rows);
  const RadixPlan plan = radix_plan(bits_for(sentinel), 4);
  FLARE_TRY(launch_zero(workspace, zero_bytes_for(w, plan), s));
  const int bpb = prep_bags_per_block(bags);
  // bags of at most kPerBagLength ids on average are walked one thread per bag
  const int per_bag = n <= kPerBagLength * bags ? 1 : 0;
  const int pgrid = static_cast<int>(ceil_div(bags, bpb));
  float *aux = pooling == FLARE_POOL_MEAN ? w.aux : nullptr;
  if (one_id && table_major && n == bags) {
    const int ogrid = static_cast<int>(ceil_div(n, static_cast<int64_t>(kPrepThreads) * kPrepOneItems));
    if (id_dtype == FLARE_INT32)
      prepare_one_kernel<int32_t><<<ogrid, kPrepThreads, 0, s>>>(
          static_cast<const int32_t *>(ids), static_cast<uint32_t>(n), offsets, row_base,
          static_cast<uint32_t>(batch), rows, plan.passes, plan.digit_bits, static_cast<uint32_t *>(w.keys[0]), aux,
          w.hist, w.meta + 3, w.meta + 6, err);
    else
      prepare_one_kernel<int64_t><<<ogrid, kPrepThreads, 0, s>>>(
          static_cast<const int64_t *>(ids), static_cast<uint32_t>(n), offsets, row_base,
          static_cast<uint32_t>(batch), rows, plan.passes, plan.digit_bits, static_cast<uint32_t *>(w.keys[0]), aux,
          w.hist, w.meta + 3, w.meta + 6, err);
  } else if (id_dtype == FLARE_INT32)
    prepare_csr_kernel<int32_t><<<pgrid, kPrepThreads, 0, s>>>(
        static_cast<const int32_t *>(ids), n, offsets, bags, bpb, row_base, num_tables, batch, rows,
        plan.passes, plan.digit_bits, static_cast<uint32_t *>(w.keys[0]), w.grad_row, aux, w.hist, w.meta + 3, per_bag,
        table_major, one_id, w.meta + 6, err);
  else
    prepare_csr_kernel<int64_t><<<pgrid, kPrepThreads, 0, s>>>(
        static_cast<const int64_t *>(ids), n, offsets, bags, bpb, row_base, num_tables, batch, rows,
        plan.passes, plan.digit_bits, static_cast<uint32_t *>(w.keys[0]), w.grad_row, aux, w.hist, w.meta + 3, per_bag,
        table_major, one_id, w.meta + 6, err);
  FLARE_TRY_HIP(hipGetLastError());
  int sorted = 0;
  return dedup_rows(w, plan, sentinel, err, s, &sorted, first_indices_out, unique_out,
                    unique_out ? kUniqueFromSorted : kUniqueNone, nullptr, 0, unique_count, aux,
                    one_id && table_major);
}

extern "C" int flare_pooled_apply(void *table, int32_t value_dtype, int64_t rows, int32_t dim,
                                  float *state0, float *state1, int32_t *step,
                                  const flare_optimizer *optimizer, int64_t n,
                                  int32_t num_tables, int64_t batch, int32_t pooling,
                                  const float *weights, const float *pooled_grad,
                                  int32_t normalization_steps, float *grad_out,
                                  int32_t *inverse_out, void *workspace, size_t workspace_bytes,
                                  void *stream) {
  return flare_pooled_apply_ex(table, value_dtype, rows, dim, state0, state1, step, optimizer, n, num_tables,
                               batch, pooling, weights, pooled_grad, FLARE_FLOAT32, 0, nullptr,
                               normalization_steps, grad_out, inverse_out, workspace, workspace_bytes, stream);
}

extern "C" int flare_pooled_apply_ex(void *table, int32_t value_dtype, int64_t rows, int32_t dim,
                                     float *state0, float *state1, int32_t *step,
                                     const flare_optimizer *optimizer, int64_t n,
                                     int32_t num_tables, int64_t batch, int32_t pooling,
                                     const float *weights, const void *pooled_grad, int32_t grad_dtype,
                                     int32_t check_finite, int32_t *nonfinite_out,
                                     int32_t normalization_steps, float *grad_out,
                                     int32_t *inverse_out, void *workspace, size_t workspace_bytes,
                                     void *stream) {
  FLARE_TRY(check_grad_dtype(grad_dtype));
  if (storage_bytes(value_dtype) == 0)
    return fail(FLARE_ERR_DTYPE, "sparse embedding value dtype code %d is not float16, bfloat16 or float32", value_dtype);
  FLARE_TRY(check_pooled_args(rows, dim, num_tables, batch, n, pooling, weights, true));
  if (normalization_steps <= 0) return fail(FLARE_ERR_ARGUMENT, "normalization_steps must be a positive integer");
  int mode = 0;
  FLARE_TRY(optimizer_mode(optimizer, &mode));
  if (mode == kModeUnique && !grad_out) return fail(FLARE_ERR_ARGUMENT, "FLARE_OPT_NONE requires grad_out");
  FLARE_TRY(check_state(mode, state0, state1, step));
  if (n == 0 || batch * num_tables == 0) {  // nothing to update; a requested check still reports
    if (!check_finite || !nonfinite_out) return FLARE_OK;
    int st = FLARE_OK;
    int *err = device_error_word(&st);
    if (!err) return st;
    return launch_finite_check(pooled_grad, grad_dtype, batch * num_tables * static_cast<int64_t>(dim), nullptr,
                               nonfinite_out, err, as_stream(stream));
  }
  Workspace w = layout_workspace(workspace, n, 4, dim, true, true, true, true);
  FLARE_TRY(check_workspace(w, workspace_bytes));
  int st = FLARE_OK;
  int *err = device_error_word(&st);
  if (!err) return st;
  const int sorted = radix_plan(bits_for(static_cast<uint32_t>(rows)), 4).passes & 1;  // buffer holding the sorted pairs
  UpdateArgs a{};
  a.sk = static_cast<const uint32_t *>(w.keys[sorted]);
  a.sv = w.vals[sorted];
  a.run_start = w.run_start;
  a.unit_first_run = w.unit_first_run;
  a.meta = w.meta;
  a.run_rank = w.run_rank;
  a.inverse_out = inverse_out;
  a.grad = pooled_grad;
  a.grad_bf16 = grad_dtype == FLARE_BFLOAT16;
  a.grad_rows = static_cast<uint32_t>(batch * num_tables);
  hipStream_t s = as_stream(stream);
  if (check_finite) {
    FLARE_TRY(launch_finite_check(pooled_grad, grad_dtype, batch * num_tables * static_cast<int64_t>(dim),
                                  w.meta + 4, nonfinite_out, err, s));
    a.reject = w.meta + 4;
  }
  a.grad_mode = kGradRowArray;
  a.grad_row = w.grad_row;
  a.sorted_grad_row = w.sorted_grad_row;
  a.scale_mode = pooling == FLARE_POOL_WEIGHTED ? kScaleMul : (pooling == FLARE_POOL_MEAN ? kScaleDiv : kScaleNone);
  a.scale = pooling == FLARE_POOL_WEIGHTED ? weights : w.aux;
  a.sorted_scale = pooling == FLARE_POOL_MEAN ? w.sorted_scale : nullptr;
  a.run_grad_row = w.run_grad_row;
  a.run_scale = pooling == FLARE_POOL_MEAN ? w.run_scale : nullptr;
  a.use_norm = normalization_steps != 1;
  a.norm = static_cast<float>(normalization_steps);
  a.dim = dim;
  a.partial = w.partial;
  a.sums = w.sums;
  a.run_key = w.run_key;
  a.hot_runs = w.hot_runs;
  a.out = grad_out;
  a.table = table;
  a.s0 = state0;
  a.s1 = state1;
  a.step = step;
  fill_optimizer(a, optimizer);
  a.units = w.units;
  a.n = static_cast<uint32_t>(w.n);
  a.err = err;
  const bool v4 = vec4_ok(pooled_grad) && (grad_out ? vec4_ok(grad_out) : true) &&
                  aligned(table, 8) && (mode == kModeAdam ? (vec4_ok(state0) && vec4_ok(state1)) : true) &&
                  vec4_ok(w.partial);
  const bool v8 = v4 && a.grad_bf16 && aligned(table, 16);
  Shape sh;
  FLARE_TRY(choose_shape(dim, v4, &sh, v8));
  return launch_update(mode, value_dtype, a, sh, s);
}

extern "C" int flare_pooled_backward(void *table, int32_t value_dtype, int64_t rows, int32_t dim,
                                     float *state0, float *state1, int32_t *step,
                                     const flare_optimizer *optimizer, const void *ids,
                                     int32_t id_dtype, int64_t n, const int64_t *offsets,
                                     int32_t num_tables, int64_t batch, const int64_t *row_base,
                                     int32_t pooling, int32_t layout, const float *weights,
                                     const float *pooled_grad, int32_t normalization_steps,
                                     float *grad_out, int64_t *unique_out, int32_t *inverse_out,
                                     int64_t *first_indices_out, int64_t *unique_count,
                                     void *workspace, size_t workspace_bytes, void *stream) {
  // validate everything before enqueuing any work
  if (storage_bytes(value_dtype) == 0)
    return fail(FLARE_ERR_DTYPE, "sparse embedding value dtype code %d is not float16, bfloat16 or float32", value_dtype);
  FLARE_TRY(check_pooled_args(rows, dim, num_tables, batch, n, pooling, weights, true));
  if (normalization_steps <= 0) return fail(FLARE_ERR_ARGUMENT, "normalization_steps must be a positive integer");
  int mode = 0;
  FLARE_TRY(optimizer_mode(optimizer, &mode));
  if (mode == kModeUnique && !grad_out) return fail(FLARE_ERR_ARGUMENT, "FLARE_OPT_NONE requires grad_out");
  FLARE_TRY(check_state(mode, state0, state1, step));
  FLARE_TRY(check_layout(layout));
  FLARE_TRY(flare_pooled_dedup(ids, id_dtype, n, offsets, num_tables, batch, row_base, rows, dim,
                               pooling, layout, unique_out, first_indices_out, unique_count, workspace,
                               workspace_bytes, stream));
  return flare_pooled_apply(table, value_dtype, rows, dim, state0, state1, step, optimizer, n,
                            num_tables, batch, pooling, weights, pooled_grad, normalization_steps,
                            grad_out, inverse_out, workspace, workspace_bytes, stream);
}
