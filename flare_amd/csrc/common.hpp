// Shared device/host helpers for the gfx950 sparse-embedding kernels.
//
// Storage conversions are written from the IEEE-754 definitions
// (round-to-nearest-even); fp16 uses the hardware v_cvt_f16_f32, which rounds
// to nearest even in the default mode.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "flare_amd.h"

namespace flare {

// ----------------------------------------------------------------------------
// Host-side error state and status helpers (definitions in errors.cpp).
// ----------------------------------------------------------------------------
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_fail(hipError_t err, const char *what);
// Device word that kernels OR error bits into (one per device, lazily created).
int *device_error_word(int *status);

#define FLARE_TRY_HIP(expr)                                   \
  do {                                                        \
    hipError_t flare_e_ = (expr);                             \
    if (flare_e_ != hipSuccess) return ::flare::hip_fail(flare_e_, #expr); \
  } while (0)

#define FLARE_TRY(expr)                  \
  do {                                   \
    int flare_s_ = (expr);               \
    if (flare_s_ != FLARE_OK) return flare_s_; \
  } while (0)

// Error bits written by kernels into the device error word.
enum : int {
  kErrIndexOutOfRange = 1,  // an index outside its table was skipped / zeroed
  kErrSpinGuard = 2,        // a bounded spin-wait gave up (results invalid)
  kErrCapacity = 4,         // a key map or its table is full (keys left without a row)
  kErrNonFinite = 8,        // a checked gradient held inf / NaN (its update was skipped)
};

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline int storage_bytes(int dtype) {
  switch (dtype) {
    case FLARE_FLOAT32: return 4;
    case FLARE_FLOAT16: return 2;
    case FLARE_BFLOAT16: return 2;
    default: return 0;
  }
}

inline bool aligned(const void *p, int bytes) {
  return (reinterpret_cast<uintptr_t>(p) % static_cast<uintptr_t>(bytes)) == 0;
}

// ----------------------------------------------------------------------------
// Storage element types.  Each tag knows its element type and the exact
// conversion to / from float32.
// ----------------------------------------------------------------------------
struct TagF32 {
  using elem = float;
  static __device__ __forceinline__ float to_f32(float x) { return x; }
  static __device__ __forceinline__ float from_f32(float x) { return x; }
};

struct TagF16 {
  using elem = _Float16;
  static __device__ __forceinline__ float to_f32(_Float16 x) { return static_cast<float>(x); }
  static __device__ __forceinline__ _Float16 from_f32(float x) { return static_cast<_Float16>(x); }
};

struct TagBF16 {
  using elem = uint16_t;  // raw bfloat16 bits
  static __device__ __forceinline__ float to_f32(uint16_t x) {
    return __uint_as_float(static_cast<uint32_t>(x) << 16);
  }
  static __device__ __forceinline__ uint16_t from_f32(float x) {
    const uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);  // quiet NaN
    const uint32_t lsb = (u >> 16) & 1u;
    return static_cast<uint16_t>((u + 0x7fffu + lsb) >> 16);
  }
};

// Raw vector of N bytes used for wide loads / stores.
template <int N> struct Raw;
// 32 bytes: two 16-byte halves (eight float32 lanes of one 16-byte-lane row slice)
struct alignas(16) Bytes32 {
  uint4 lo, hi;
};
template <> struct Raw<32> { using type = Bytes32; };
template <> struct Raw<16> { using type = uint4; };
template <> struct Raw<8> { using type = uint2; };
template <> struct Raw<4> { using type = uint32_t; };
template <> struct Raw<2> { using type = uint16_t; };

// Raw (still packed) vector of VEC storage elements and its conversion to f32;
// kept packed while loads are in flight so that several rows fit in registers.
template <typename Tag, int VEC>
using RawVec = typename Raw<VEC * sizeof(typename Tag::elem)>::type;

template <typename Tag, int VEC>
__device__ __forceinline__ RawVec<Tag, VEC> load_raw(const typename Tag::elem *p) {
  return *reinterpret_cast<const RawVec<Tag, VEC> *>(p);
}

template <typename Tag, int VEC>
__device__ __forceinline__ void raw_to_f32(const RawVec<Tag, VEC> &raw, float (&out)[VEC]) {
  using E = typename Tag::elem;
  E tmp[VEC];
  __builtin_memcpy(tmp, &raw, sizeof(raw));
#pragma unroll
  for (int i = 0; i < VEC; ++i) out[i] = Tag::to_f32(tmp[i]);
}

// Load VEC consecutive storage elements (aligned to VEC*sizeof(elem)) as f32.
template <typename Tag, int VEC>
__device__ __forceinline__ void load_as_f32(const typename Tag::elem *p, float (&out)[VEC]) {
  using E = typename Tag::elem;
  using R = typename Raw<VEC * sizeof(E)>::type;
  const R raw = *reinterpret_cast<const R *>(p);
  E tmp[VEC];
  __builtin_memcpy(tmp, &raw, sizeof(raw));
#pragma unroll
  for (int i = 0; i < VEC; ++i) out[i] = Tag::to_f32(tmp[i]);
}

template <typename Tag, int VEC>
__device__ __forceinline__ void store_from_f32(typename Tag::elem *p, const float (&in)[VEC]) {
  using E = typename Tag::elem;
  using R = typename Raw<VEC * sizeof(E)>::type;
  E tmp[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) tmp[i] = Tag::from_f32(in[i]);
  R raw;
  __builtin_memcpy(&raw, tmp, sizeof(raw));
  *reinterpret_cast<R *>(p) = raw;
}

// Like store_from_f32, with a nontemporal hint for 16-byte vectors: for
// outputs that this library does not read back (the pooled rows), so they
// stream past L2 instead of evicting rows that later kernels reuse.
template <typename Tag, int VEC>
__device__ __forceinline__ void store_from_f32_stream(typename Tag::elem *p, const float (&in)[VEC]) {
  using E = typename Tag::elem;
  if constexpr (sizeof(E) * VEC == 16) {
    E tmp[VEC];
#pragma unroll
    for (int i = 0; i < VEC; ++i) tmp[i] = Tag::from_f32(in[i]);
    typedef unsigned int U4 __attribute__((ext_vector_type(4)));
    U4 raw;
    __builtin_memcpy(&raw, tmp, sizeof(raw));
    __builtin_nontemporal_store(raw, reinterpret_cast<U4 *>(p));
  } else {
    store_from_f32<Tag, VEC>(p, in);
  }
}

template <int VEC>
__device__ __forceinline__ void load_f32(const float *p, float (&out)[VEC]) {
  using R = typename Raw<VEC * 4>::type;
  const R raw = *reinterpret_cast<const R *>(p);
  __builtin_memcpy(out, &raw, sizeof(raw));
}

template <int VEC>
__device__ __forceinline__ void store_f32(float *p, const float (&in)[VEC]) {
  using R = typename Raw<VEC * 4>::type;
  R raw;
  __builtin_memcpy(&raw, in, sizeof(raw));
  *reinterpret_cast<R *>(p) = raw;
}

// ----------------------------------------------------------------------------
// Wave64 helpers.
// ----------------------------------------------------------------------------
__device__ __forceinline__ uint64_t lanemask_lt() {
  const int lane = __lane_id();
  return (lane == 0) ? 0ull : (~0ull >> (64 - lane));
}

__device__ __forceinline__ void record_error(int *err, int bits) {
  if (err) atomicOr(err, bits);
}

// Exclusive scan of one uint32 per thread over a 256-thread block.
// scratch: >= 4 uint32 of LDS.  Returns the exclusive prefix; *total gets the sum.
__device__ __forceinline__ uint32_t block_exclusive_scan_256(uint32_t v, uint32_t *scratch,
                                                             uint32_t *total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  uint32_t incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t y = __shfl_up(incl, off, 64);
    if (lane >= off) incl += y;
  }
  if (lane == 63) scratch[wave] = incl;
  __syncthreads();
  uint32_t wave_base = 0;
  uint32_t sum = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t s = scratch[w];
    if (w < wave) wave_base += s;
    sum += s;
  }
  __syncthreads();
  if (total) *total = sum;
  return wave_base + incl - v;
}

// Exclusive scan of one uint32 per thread over a block of THREADS threads.
// scratch: >= THREADS/64 uint32 of LDS.  Every thread of the block must call it.
template <int THREADS>
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t *scratch) {
  constexpr int kWaves = THREADS / 64;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  uint32_t incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t y = __shfl_up(incl, off, 64);
    if (lane >= off) incl += y;
  }
  if (lane == 63) scratch[wave] = incl;
  __syncthreads();
  uint32_t wave_base = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w)
    if (w < wave) wave_base += scratch[w];
  __syncthreads();
  return wave_base + incl - v;
}

// ----------------------------------------------------------------------------
// Decoupled look-back (single-pass chained scan across tiles).
//
// status[tile * stride + idx] holds a 2-bit flag and a 30-bit count:
//   flag 1 = this tile's own aggregate, flag 2 = inclusive prefix.
// The count travels inside the status word, so the words are written and
// read with relaxed agent-scope atomics, which bypass the per-XCD L2 and need
// no fence.  (On gfx942/gfx950 an agent-scope release or acquire writes back
// or invalidates the XCD's L2; issuing one per status word serializes the
// whole scan.)  Tiles are numbered in the order they start (atomic ticket),
// so a tile only waits for tiles that are already running and publish their
// aggregate before waiting themselves: the wait always ends.  The spin count
// is still bounded; if the guard trips, the error word gets kErrSpinGuard and
// callers clamp every write to stay inside their buffers.
// ----------------------------------------------------------------------------
constexpr uint32_t kFlagAggregate = 1u << 30;
constexpr uint32_t kFlagPrefix = 2u << 30;
constexpr uint32_t kCountMask = (1u << 30) - 1;
constexpr uint32_t kSpinLimit = 1u << 22;

__device__ __forceinline__ void publish(uint32_t *p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t peek(const uint32_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// kWindow predecessors are read per round trip: when every tile of a pass is
// resident at once (one per CU), the inclusive prefixes spread back to front
// about 2 * kWindow tiles per round trip.
template <int kWindow = 4>
__device__ __forceinline__ uint32_t lookback_exclusive(uint32_t *status, uint32_t tile,
                                                       uint32_t stride, uint32_t idx,
                                                       uint32_t value, int *err) {
  uint32_t *mine = status + static_cast<size_t>(tile) * stride + idx;
  if (tile == 0) {
    publish(mine, kFlagPrefix | value);
    return 0;
  }
  publish(mine, kFlagAggregate | value);
  // Walk back over predecessors, kWindow status words per round trip.
  uint32_t prefix = 0;
  int64_t t = static_cast<int64_t>(tile) - 1;
  uint32_t spins = 0;
  bool done = false;
  while (t >= 0 && !done) {
    uint32_t seen[kWindow];
#pragma unroll
    for (int w = 0; w < kWindow; ++w)
      seen[w] = (t - w >= 0) ? peek(status + static_cast<size_t>(t - w) * stride + idx) : kFlagPrefix;
#pragma unroll
    for (int w = 0; w < kWindow; ++w) {
      if (done) break;
      uint32_t st = seen[w];
      while ((st & ~kCountMask) == 0) {  // predecessor has not published yet
        if (++spins > kSpinLimit) {
          record_error(err, kErrSpinGuard);
          st = kFlagPrefix;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
        st = peek(status + static_cast<size_t>(t - w) * stride + idx);
      }
      prefix += st & kCountMask;
      if ((st & ~kCountMask) == kFlagPrefix) done = true;
    }
    t -= kWindow;
  }
  publish(mine, kFlagPrefix | ((prefix + value) & kCountMask));
  return prefix;
}

}  // namespace flare
