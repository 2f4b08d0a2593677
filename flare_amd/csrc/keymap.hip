// Key -> row map of the dynamic sparse store: arbitrary int64 keys mapped to
// rows of a pre-sized HBM table, new keys given rows in the order of their
// first occurrence in each call and initialised from a counter-based uniform
// hash of (seed, key, column), so a key's first values do not depend on the
// batch it arrives in.
//
// Map buffer (flare_keymap_bytes): a 256-byte header (word 0: rows handed out
// so far), then `capacity` 16-byte slots {uint64 key, uint32 row, pad}, so a
// probe reads key and row with one access.
//   key: kEmptyKey until a key claims the slot; never changes after.
//   row: kEmptyRow (no row), kPending | i (claimed in this call by its lowest
//        occurrence i), or the key's row (< kPending).
// Slots are found by linear probing from splitmix64(key) (the finaliser of
// Steele, Lea and Flood's SplitMix64) masked to the power-of-two capacity.
//
// One call of flare_keymap_lookup_or_insert:
//   probe   every occurrence finds its key's slot (or claims an empty one); a
//           key without a row is claimed by its lowest occurrence (atomicMin)
//   count   claiming occurrences per tile of 4096
//   scan    tile prefixes, the call's first row and the header's new count
//   assign  each claiming occurrence writes its key's row: first row + rank
//   values  rows out; new rows initialised in the table; values gathered
#include "common.hpp"

namespace flare {
namespace {

constexpr unsigned long long kEmptyKey = 0x8000000000000000ull;  // INT64_MIN: not a storable key
constexpr uint32_t kEmptyRow = 0xffffffffu;
constexpr uint32_t kPending = 0x80000000u;
constexpr uint32_t kFresh = 0x80000000u;  // slot_of bit: the key had no row before this call
constexpr uint32_t kNoSlot = 0xffffffffu;
constexpr size_t kHeaderBytes = 256;
constexpr int kThreads = 256;
constexpr int kItems = 16;
constexpr int kTile = kThreads * kItems;
constexpr int64_t kMinCapacity = 64;
constexpr int64_t kMaxCapacity = int64_t{1} << 30;
constexpr int64_t kMaxKeys = int64_t{1} << 30;

struct MapView {
  uint32_t *header;
  unsigned long long *slots;  // slot h: key at slots[2h], row word in the low half of slots[2h + 1]
  uint64_t mask;
  __device__ unsigned long long *key(uint64_t h) const { return slots + 2 * h; }
  __device__ uint32_t *row(uint64_t h) const { return reinterpret_cast<uint32_t *>(slots + 2 * h + 1); }
};

MapView view(void *map, int64_t capacity) {
  char *b = static_cast<char *>(map);
  return {reinterpret_cast<uint32_t *>(b), reinterpret_cast<unsigned long long *>(b + kHeaderBytes),
          static_cast<uint64_t>(capacity - 1)};
}

__host__ __device__ inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

// U(lo, hi) value of (key, column): 24 random bits scaled to [0, 1), then
// lo + (hi - lo) * u in float32 (each operation rounded).
__device__ __forceinline__ float init_uniform(uint64_t seed, uint64_t key, uint32_t col, float lo, float hi) {
  const uint64_t z = mix64(mix64(seed ^ key) + 0x9e3779b97f4a7c15ull * (static_cast<uint64_t>(col) + 1));
  const float u = static_cast<float>(static_cast<uint32_t>(z >> 40)) * 5.9604644775390625e-8f;  // 2^-24
  return lo + (hi - lo) * u;
}

__global__ __launch_bounds__(kThreads) void init_kernel(MapView m, uint64_t capacity) {
  for (uint64_t i = blockIdx.x * static_cast<uint64_t>(kThreads) + threadIdx.x; i < capacity;
       i += static_cast<uint64_t>(gridDim.x) * kThreads) {
    *m.key(i) = kEmptyKey;
    *m.row(i) = kEmptyRow;
  }
  if (blockIdx.x == 0 && threadIdx.x < kHeaderBytes / 4) m.header[threadIdx.x] = 0;
}

// code[i]: the row of keys[i] when it has one; kFresh | slot when the key had
// no row before this call (insert); kNoSlot when absent (lookup), invalid or
// the map is full.
// Probe from slot h on (linear), claiming an empty slot on insert; returns the
// code of occurrence i (see probe_kernel).
template <bool kInsert>
__device__ uint32_t probe_from(const MapView &m, unsigned long long k, uint64_t h, uint32_t i, int *err) {
  uint32_t result = kNoSlot;
  for (uint64_t probe = 0; probe <= m.mask; ++probe, h = (h + 1) & m.mask) {
    unsigned long long cur = *m.key(h);
    if (cur == kEmptyKey) {
      if (!kInsert) break;  // the key would be here: absent
      // a stale empty read is harmless: the swap then returns the slot's key
      cur = atomicCAS(m.key(h), kEmptyKey, k);
      if (cur == kEmptyKey) cur = k;
    }
    if (cur == k) {
      result = static_cast<uint32_t>(h);
      break;
    }
  }
  if (result == kNoSlot) {
    if (kInsert) record_error(err, kErrCapacity);
    return kNoSlot;
  }
  const uint32_t row = *m.row(result);
  if (row < kPending) return row;
  if (!kInsert) return kNoSlot;
  atomicMin(m.row(result), kPending | i);  // no row yet: the lowest occurrence claims it
  return result | kFresh;
}

// code[i]: the row of keys[i] when it has one; kFresh | slot when the key had
// no row before this call (insert); kNoSlot when absent (lookup), invalid or
// the map is full.  Each thread takes kProbeKeys keys and issues their first
// slot reads (key and row word in one 16-byte load) together; a key not in
// its home slot continues in probe_from.
constexpr int kProbeKeys = 4;

template <bool kInsert>
__global__ __launch_bounds__(kThreads) void probe_kernel(MapView m, const int64_t *__restrict__ keys, uint32_t n,
                                                         uint32_t *__restrict__ slot_of, int *err) {
  typedef unsigned long long U2 __attribute__((ext_vector_type(2)));
  const uint32_t stride = gridDim.x * kThreads * kProbeKeys;
  for (uint32_t base = blockIdx.x * kThreads * kProbeKeys + threadIdx.x; base < n; base += stride) {
    unsigned long long k[kProbeKeys];
    uint64_t h[kProbeKeys];
    U2 slot[kProbeKeys];
#pragma unroll
    for (int p = 0; p < kProbeKeys; ++p) {
      const uint32_t i = base + p * kThreads;
      k[p] = i < n ? static_cast<unsigned long long>(keys[i]) : kEmptyKey;
      h[p] = mix64(k[p]) & m.mask;
    }
#pragma unroll
    for (int p = 0; p < kProbeKeys; ++p) {
      slot[p] = U2{kEmptyKey, 0};
      if (k[p] != kEmptyKey) slot[p] = *reinterpret_cast<const U2 *>(m.key(h[p]));
    }
#pragma unroll
    for (int p = 0; p < kProbeKeys; ++p) {
      const uint32_t i = base + p * kThreads;
      if (i >= n) break;
      uint32_t code;
      if (k[p] == kEmptyKey) {
        record_error(err, kErrIndexOutOfRange);
        code = kNoSlot;
      } else if (slot[p].x == k[p] && static_cast<uint32_t>(slot[p].y) < kPending) {
        code = static_cast<uint32_t>(slot[p].y);  // found in its home slot with a row
      } else if (!kInsert && slot[p].x == kEmptyKey) {
        code = kNoSlot;  // absent
      } else {
        code = probe_from<kInsert>(m, k[p], h[p], i, err);
      }
      slot_of[i] = code;
    }
  }
}

// Whether occurrence i claims its key's row in this call.
__device__ __forceinline__ bool claims(const MapView &m, uint32_t s, uint32_t i) {
  return s != kNoSlot && (s & kFresh) && *m.row(s & ~kFresh) == (kPending | i);
}

__global__ __launch_bounds__(kThreads) void count_kernel(MapView m, const uint32_t *__restrict__ slot_of, uint32_t n,
                                                         uint32_t *__restrict__ counts) {
  __shared__ uint32_t s_sum[kThreads / 64];
  const uint32_t base = blockIdx.x * kTile;
  uint32_t c = 0;
#pragma unroll
  for (int k = 0; k < kItems; ++k) {
    const uint32_t i = base + k * kThreads + threadIdx.x;
    if (i < n && claims(m, slot_of[i], i)) ++c;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off, 64);
  if ((threadIdx.x & 63) == 0) s_sum[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) counts[blockIdx.x] = s_sum[0] + s_sum[1] + s_sum[2] + s_sum[3];
}

// One block: exclusive scan of the tile counts; meta[0] = the call's first
// row; the header's row count advances by the new keys (capped).
__global__ __launch_bounds__(1024) void scan_kernel(uint32_t *counts, uint32_t tiles, uint32_t *header,
                                                    uint32_t *meta, uint32_t row_capacity) {
  __shared__ uint32_t s_scan[16];
  __shared__ uint32_t s_carry;
  if (threadIdx.x == 0) s_carry = 0;
  __syncthreads();
  for (uint32_t b = 0; b < tiles; b += 1024) {
    const uint32_t t = b + threadIdx.x;
    const uint32_t v = t < tiles ? counts[t] : 0u;
    const uint32_t ex = block_exclusive_scan<1024>(v, s_scan);
    const uint32_t carry = s_carry;
    if (t < tiles) counts[t] = carry + ex;
    __syncthreads();
    if (threadIdx.x == 1023) s_carry = carry + ex + v;
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const uint32_t first = header[0];
    const uint64_t end = static_cast<uint64_t>(first) + s_carry;
    meta[0] = first;
    meta[1] = s_carry;
    header[0] = static_cast<uint32_t>(end < row_capacity ? end : row_capacity);
  }
}

__global__ __launch_bounds__(kThreads) void assign_kernel(MapView m, const uint32_t *__restrict__ slot_of, uint32_t n,
                                                          const uint32_t *__restrict__ counts,
                                                          const uint32_t *__restrict__ meta, uint32_t row_capacity,
                                                          int *err) {
  __shared__ uint32_t s_scan[4];
  const uint32_t base = blockIdx.x * kTile;
  uint32_t carry = counts[blockIdx.x];
  const uint32_t next = blockIdx.x + 1 < gridDim.x ? counts[blockIdx.x + 1] : meta[1];
  if (next == carry) return;  // no key of this tile is new (block-uniform)
  const uint32_t first = meta[0];
  for (int k = 0; k < kItems; ++k) {  // index order: rounds of 256 consecutive occurrences
    const uint32_t i = base + k * kThreads + threadIdx.x;
    const uint32_t s = i < n ? slot_of[i] : kNoSlot;
    const bool owner = i < n && claims(m, s, i);
    uint32_t round = 0;
    const uint32_t ex = block_exclusive_scan_256(owner ? 1u : 0u, s_scan, &round);
    if (owner) {
      const uint64_t row = static_cast<uint64_t>(first) + carry + ex;
      if (row < row_capacity) {
        *m.row(s & ~kFresh) = static_cast<uint32_t>(row);
      } else {
        *m.row(s & ~kFresh) = kEmptyRow;  // a later call may retry once rows are reserved
        record_error(err, kErrCapacity);
      }
    }
    carry += round;
  }
}

// rows_out[i] = row of keys[i] (-1 when absent); new rows get their initial
// values in the table; values_out[i] = the row (zeros when absent).  A group
// of G lanes per occurrence, VEC elements per lane.
template <typename Tag, int VEC, int G>
__global__ __launch_bounds__(kThreads) void values_kernel(MapView m, const int64_t *__restrict__ keys,
                                                          const uint32_t *__restrict__ slot_of, uint32_t n,
                                                          typename Tag::elem *table, int dim, float lo, float hi,
                                                          uint64_t seed, int32_t *__restrict__ rows_out,
                                                          typename Tag::elem *__restrict__ values_out) {
  using E = typename Tag::elem;
  constexpr int kGroups = kThreads / G;
  const int lane = threadIdx.x % G;
  for (uint32_t i = blockIdx.x * kGroups + threadIdx.x / G; i < n; i += gridDim.x * kGroups) {
    const uint32_t s = slot_of[i];
    int64_t row = -1;
    bool fresh = false;
    if (s != kNoSlot) {
      if (s & kFresh) {  // new in this call: its row was assigned after the probe
        const uint32_t w = *m.row(s & ~kFresh);
        if (w < kPending) {
          row = w;
          fresh = true;
        }
      } else {
        row = s;
      }
    }
    if (lane == 0 && rows_out) rows_out[i] = static_cast<int32_t>(row);
    if (!table) continue;
    const uint64_t key = static_cast<uint64_t>(keys[i]);
    for (int col = lane * VEC; col < dim; col += G * VEC) {
      float v[VEC];
      if (row < 0) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) v[e] = 0.0f;
      } else if (fresh) {
        // every occurrence of a new key writes the same initial values
#pragma unroll
        for (int e = 0; e < VEC; ++e) v[e] = init_uniform(seed, key, static_cast<uint32_t>(col + e), lo, hi);
        store_from_f32<Tag, VEC>(table + row * dim + col, v);
      } else {
        load_as_f32<Tag, VEC>(table + row * dim + col, v);
      }
      if (values_out) store_from_f32<Tag, VEC>(values_out + static_cast<int64_t>(i) * dim + col, v);
    }
  }
}

// Copies every key that has a row into a fresh (initialised) map.
__global__ __launch_bounds__(kThreads) void rehash_kernel(MapView src, uint64_t src_capacity, MapView dst, int *err) {
  if (blockIdx.x == 0 && threadIdx.x == 0) dst.header[0] = src.header[0];
  for (uint64_t j = blockIdx.x * static_cast<uint64_t>(kThreads) + threadIdx.x; j < src_capacity;
       j += static_cast<uint64_t>(gridDim.x) * kThreads) {
    const unsigned long long k = *src.key(j);
    const uint32_t r = *src.row(j);
    if (k == kEmptyKey || r >= kPending) continue;
    uint64_t h = mix64(k) & dst.mask;
    bool placed = false;
    for (uint64_t probe = 0; probe <= dst.mask; ++probe, h = (h + 1) & dst.mask) {
      const unsigned long long cur = atomicCAS(dst.key(h), kEmptyKey, k);
      if (cur == kEmptyKey || cur == k) {
        *dst.row(h) = r;
        placed = true;
        break;
      }
    }
    if (!placed) record_error(err, kErrCapacity);
  }
}

// Export: the keys that hold rows and their rows, in slot order (count per
// tile of kTile slots, scan, write).
__global__ __launch_bounds__(kThreads) void export_count_kernel(MapView m, uint64_t capacity,
                                                                uint32_t *__restrict__ counts) {
  __shared__ uint32_t s_sum[kThreads / 64];
  const uint64_t base = static_cast<uint64_t>(blockIdx.x) * kTile;
  uint32_t c = 0;
#pragma unroll
  for (int k = 0; k < kItems; ++k) {
    const uint64_t j = base + k * kThreads + threadIdx.x;
    if (j < capacity && *m.key(j) != kEmptyKey && *m.row(j) < kPending) ++c;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off, 64);
  if ((threadIdx.x & 63) == 0) s_sum[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) counts[blockIdx.x] = s_sum[0] + s_sum[1] + s_sum[2] + s_sum[3];
}

__global__ __launch_bounds__(1024) void export_scan_kernel(uint32_t *counts, uint32_t tiles, int64_t *total) {
  __shared__ uint32_t s_scan[16];
  __shared__ uint32_t s_carry;
  if (threadIdx.x == 0) s_carry = 0;
  __syncthreads();
  for (uint32_t b = 0; b < tiles; b += 1024) {
    const uint32_t t = b + threadIdx.x;
    const uint32_t v = t < tiles ? counts[t] : 0u;
    const uint32_t ex = block_exclusive_scan<1024>(v, s_scan);
    const uint32_t carry = s_carry;
    if (t < tiles) counts[t] = carry + ex;
    __syncthreads();
    if (threadIdx.x == 1023) s_carry = carry + ex + v;
    __syncthreads();
  }
  if (threadIdx.x == 0) *total = s_carry;
}

__global__ __launch_bounds__(kThreads) void export_write_kernel(MapView m, uint64_t capacity,
                                                                const uint32_t *__restrict__ counts,
                                                                int64_t *__restrict__ keys_out,
                                                                int32_t *__restrict__ rows_out) {
  __shared__ uint32_t s_scan[4];
  const uint64_t base = static_cast<uint64_t>(blockIdx.x) * kTile;
  uint32_t carry = counts[blockIdx.x];
  for (int k = 0; k < kItems; ++k) {  // slot order: rounds of 256 consecutive slots
    const uint64_t j = base + k * kThreads + threadIdx.x;
    bool has = false;
    unsigned long long key = 0;
    uint32_t row = 0;
    if (j < capacity) {
      key = *m.key(j);
      row = *m.row(j);
      has = key != kEmptyKey && row < kPending;
    }
    uint32_t round = 0;
    const uint32_t ex = block_exclusive_scan_256(has ? 1u : 0u, s_scan, &round);
    if (has) {
      keys_out[carry + ex] = static_cast<int64_t>(key);
      rows_out[carry + ex] = static_cast<int32_t>(row);
    }
    carry += round;
  }
}

int check_capacity(int64_t capacity) {
  if (capacity < kMinCapacity || capacity > kMaxCapacity || (capacity & (capacity - 1)) != 0)
    return fail(FLARE_ERR_ARGUMENT, "key map capacity must be a power of two in [%lld, %lld], got %lld",
                static_cast<long long>(kMinCapacity), static_cast<long long>(kMaxCapacity),
                static_cast<long long>(capacity));
  return FLARE_OK;
}

int grid_for(uint64_t work, int per_block, int cap = 65536) {
  const uint64_t g = (work + per_block - 1) / per_block;
  return static_cast<int>(g < 1 ? 1 : (g > static_cast<uint64_t>(cap) ? cap : g));
}

struct Workspace {
  uint32_t *slot_of;
  uint32_t *counts;
  uint32_t *meta;
  size_t bytes;
};

Workspace layout(void *base, int64_t n) {
  const size_t a = (static_cast<size_t>(n) * 4 + 255) & ~static_cast<size_t>(255);
  const size_t tiles = static_cast<size_t>(ceil_div(n > 0 ? n : 1, kTile));
  const size_t b = (tiles * 4 + 255) & ~static_cast<size_t>(255);
  char *p = static_cast<char *>(base);
  return {reinterpret_cast<uint32_t *>(p), reinterpret_cast<uint32_t *>(p + a), reinterpret_cast<uint32_t *>(p + a + b),
          a + b + 256};
}

template <typename Tag>
int launch_values(const MapView &m, const int64_t *keys, const uint32_t *slot_of, uint32_t n, void *table, int dim,
                  float lo, float hi, uint64_t seed, int32_t *rows_out, void *values_out, hipStream_t s) {
  using E = typename Tag::elem;
  E *t = static_cast<E *>(table);
  E *v = static_cast<E *>(values_out);
  constexpr int kVec = 16 / sizeof(E);  // 16-byte vectors per lane
  const bool vec = dim % kVec == 0 && aligned(table, 16) && (!values_out || aligned(values_out, 16));
  if (vec) {
    const int vectors = dim / kVec;
    if (vectors <= 8)
      values_kernel<Tag, kVec, 8><<<grid_for(n, kThreads / 8), kThreads, 0, s>>>(m, keys, slot_of, n, t, dim, lo, hi, seed, rows_out, v);
    else if (vectors <= 16)
      values_kernel<Tag, kVec, 16><<<grid_for(n, kThreads / 16), kThreads, 0, s>>>(m, keys, slot_of, n, t, dim, lo, hi, seed, rows_out, v);
    else
      values_kernel<Tag, kVec, 32><<<grid_for(n, kThreads / 32), kThreads, 0, s>>>(m, keys, slot_of, n, t, dim, lo, hi, seed, rows_out, v);
  } else {
    values_kernel<Tag, 1, 32><<<grid_for(n, kThreads / 32), kThreads, 0, s>>>(m, keys, slot_of, n, t, dim, lo, hi, seed, rows_out, v);
  }
  FLARE_TRY_HIP(hipGetLastError());
  return FLARE_OK;
}

}  // namespace
}  // namespace flare

using namespace flare;

extern "C" size_t flare_keymap_bytes(int64_t capacity) {
  if (check_capacity(capacity) != FLARE_OK) return 0;
  return kHeaderBytes + static_cast<size_t>(capacity) * 16;
}

extern "C" int flare_keymap_init(void *map, int64_t capacity, void *stream) {
  FLARE_TRY(check_capacity(capacity));
  if (!map) return fail(FLARE_ERR_ARGUMENT, "key map buffer is null");
  init_kernel<<<grid_for(static_cast<uint64_t>(capacity), kThreads, 4096), kThreads, 0, as_stream(stream)>>>(
      view(map, capacity), static_cast<uint64_t>(capacity));
  FLARE_TRY_HIP(hipGetLastError());
  return FLARE_OK;
}

extern "C" size_t flare_keymap_workspace_bytes(int64_t n) {
  if (n < 0) return 0;
  return layout(nullptr, n).bytes;
}

extern "C" int flare_keymap_lookup_or_insert(void *map, int64_t capacity, const int64_t *keys, int64_t n,
                                             int32_t insert, void *table, int32_t value_dtype,
                                             int64_t row_capacity, int32_t dim, float init_lo, float init_hi,
                                             uint64_t seed, int32_t *rows_out, void *values_out, void *workspace,
                                             size_t workspace_bytes, void *stream) {
  FLARE_TRY(check_capacity(capacity));
  if (!map) return fail(FLARE_ERR_ARGUMENT, "key map buffer is null");
  if (n < 0 || n > kMaxKeys) return fail(FLARE_ERR_LIMIT, "key count %lld outside [0, 2^30]", static_cast<long long>(n));
  if (row_capacity < 0 || row_capacity >= static_cast<int64_t>(kPending))
    return fail(FLARE_ERR_LIMIT, "row capacity %lld outside [0, 2^31)", static_cast<long long>(row_capacity));
  if (values_out && !table) return fail(FLARE_ERR_ARGUMENT, "values requested without a table");
  if (insert && !table) return fail(FLARE_ERR_ARGUMENT, "inserting keys requires the table (new rows are initialised)");
  if (table && storage_bytes(value_dtype) == 0)
    return fail(FLARE_ERR_DTYPE, "sparse embedding value dtype code %d is not float16, bfloat16 or float32", value_dtype);
  if (table && dim <= 0) return fail(FLARE_ERR_SHAPE, "invalid row width %d", dim);
  if (!(init_lo <= init_hi)) return fail(FLARE_ERR_ARGUMENT, "initializer needs min_val <= max_val");
  if (n == 0) return FLARE_OK;
  if (!keys) return fail(FLARE_ERR_ARGUMENT, "keys are null");
  const Workspace w = layout(workspace, n);
  if (!workspace || workspace_bytes < w.bytes)
    return fail(FLARE_ERR_WORKSPACE, "key map workspace of %zu bytes is smaller than the %zu required",
                workspace_bytes, w.bytes);
  int st = FLARE_OK;
  int *err = device_error_word(&st);
  if (!err) return st;
  hipStream_t s = as_stream(stream);
  const MapView m = view(map, capacity);
  const uint32_t un = static_cast<uint32_t>(n);
  const int pgrid = grid_for(un, kThreads * kProbeKeys);
  if (insert) {
    const uint32_t tiles = static_cast<uint32_t>(ceil_div(n, kTile));
    probe_kernel<true><<<pgrid, kThreads, 0, s>>>(m, keys, un, w.slot_of, err);
    count_kernel<<<tiles, kThreads, 0, s>>>(m, w.slot_of, un, w.counts);
    scan_kernel<<<1, 1024, 0, s>>>(w.counts, tiles, m.header, w.meta, static_cast<uint32_t>(row_capacity));
    assign_kernel<<<tiles, kThreads, 0, s>>>(m, w.slot_of, un, w.counts, w.meta,
                                             static_cast<uint32_t>(row_capacity), err);
  } else {
    probe_kernel<false><<<pgrid, kThreads, 0, s>>>(m, keys, un, w.slot_of, err);
  }
  FLARE_TRY_HIP(hipGetLastError());
  switch (table ? value_dtype : FLARE_FLOAT32) {
    case FLARE_FLOAT16:
      return launch_values<TagF16>(m, keys, w.slot_of, un, table, dim, init_lo, init_hi, seed, rows_out, values_out, s);
    case FLARE_BFLOAT16:
      return launch_values<TagBF16>(m, keys, w.slot_of, un, table, dim, init_lo, init_hi, seed, rows_out, values_out, s);
    default:
      return launch_values<TagF32>(m, keys, w.slot_of, un, table, table ? dim : 1, init_lo, init_hi, seed, rows_out,
                                   values_out, s);
  }
}

extern "C" int flare_keymap_rehash(const void *src, int64_t src_capacity, void *dst, int64_t dst_capacity,
                                   void *stream) {
  FLARE_TRY(check_capacity(src_capacity));
  FLARE_TRY(check_capacity(dst_capacity));
  if (!src || !dst) return fail(FLARE_ERR_ARGUMENT, "key map buffer is null");
  int st = FLARE_OK;
  int *err = device_error_word(&st);
  if (!err) return st;
  hipStream_t s = as_stream(stream);
  const MapView d = view(dst, dst_capacity);
  init_kernel<<<grid_for(static_cast<uint64_t>(dst_capacity), kThreads, 4096), kThreads, 0, s>>>(
      d, static_cast<uint64_t>(dst_capacity));
  rehash_kernel<<<grid_for(static_cast<uint64_t>(src_capacity), kThreads, 4096), kThreads, 0, s>>>(
      view(const_cast<void *>(src), src_capacity), static_cast<uint64_t>(src_capacity), d, err);
  FLARE_TRY_HIP(hipGetLastError());
  return FLARE_OK;
}

extern "C" size_t flare_keymap_export_workspace_bytes(int64_t capacity) {
  if (check_capacity(capacity) != FLARE_OK) return 0;
  return static_cast<size_t>(ceil_div(capacity, kTile)) * 4 + 256;
}

extern "C" int flare_keymap_export(const void *map, int64_t capacity, int64_t *keys_out, int32_t *rows_out,
                                   int64_t *count_out, void *workspace, size_t workspace_bytes, void *stream) {
  FLARE_TRY(check_capacity(capacity));
  if (!map || !keys_out || !rows_out || !count_out) return fail(FLARE_ERR_ARGUMENT, "key map export buffers are null");
  const size_t need = flare_keymap_export_workspace_bytes(capacity);
  if (!workspace || workspace_bytes < need)
    return fail(FLARE_ERR_WORKSPACE, "key map export workspace of %zu bytes is smaller than the %zu required",
                workspace_bytes, need);
  hipStream_t s = as_stream(stream);
  const MapView m = view(const_cast<void *>(map), capacity);
  const uint32_t tiles = static_cast<uint32_t>(ceil_div(capacity, kTile));
  uint32_t *counts = static_cast<uint32_t *>(workspace);
  export_count_kernel<<<tiles, kThreads, 0, s>>>(m, static_cast<uint64_t>(capacity), counts);
  export_scan_kernel<<<1, 1024, 0, s>>>(counts, tiles, count_out);
  export_write_kernel<<<tiles, kThreads, 0, s>>>(m, static_cast<uint64_t>(capacity), counts, keys_out, rows_out);
  FLARE_TRY_HIP(hipGetLastError());
  return FLARE_OK;
}
