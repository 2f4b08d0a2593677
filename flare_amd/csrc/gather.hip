// Forward kernels: row gather and pooled gather (padded [B,F,M] and CSR).
//
// Pooled gather layout on gfx950: a group of G lanes of one wave64 pools a
// run of consecutive bags; lane l of the group owns columns
// [l*VEC, l*VEC+VEC) (+ q*G*VEC), loaded as 16-byte vectors (VEC = 8 for
// fp16/bf16, 4 for fp32), so a D=128 bf16 row is read by 8 lanes with two
// 16-byte loads each and a wave pools 8 bags side by side.  The block's bag
// boundaries (CSR offsets) are staged in LDS with one coalesced load; each
// group reads its ids G at a time (one per lane, coalesced) and broadcasts
// them with ds_bpermute.  Accumulation is fp32, sequential in occurrence
// order (the reference's order, gpu_cupy.py:96-103).
#include "common.hpp"

namespace flare {
namespace {

constexpr int kThreads = 256;
// launch_pooled_short: shape not covered, use pooled_kernel
constexpr int FLARE_NOT_HANDLED = -1;

// ----------------------------------------------------------------------------
// gather: raw row copy in units of CH bytes (bit-exact, like K1/K3).
// ----------------------------------------------------------------------------
template <int CH>
__global__ __launch_bounds__(kThreads) void gather_rows_kernel(
    const char *__restrict__ emb, int64_t emb_rows, int64_t row_chunks,
    const int32_t *__restrict__ inverse, int64_t slots, int32_t pad_index,
    char *__restrict__ out, int *err) {
  using R = typename Raw<CH>::type;
  const int64_t total = slots * row_chunks;
  for (int64_t t = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; t < total;
       t += static_cast<int64_t>(gridDim.x) * kThreads) {
    const int64_t slot = t / row_chunks;
    const int64_t c = t - slot * row_chunks;
    const int32_t row = inverse[slot];
    R v{};
    if (row != pad_index) {
      if (row >= 0 && row < emb_rows) {
        v = reinterpret_cast<const R *>(emb)[row * row_chunks + c];
      } else {
        record_error(err, kErrIndexOutOfRange);
      }
    }
    reinterpret_cast<R *>(out)[t] = v;
  }
}

// ----------------------------------------------------------------------------
// pooled gather
// ----------------------------------------------------------------------------
struct PooledArgs {
  const void *table;
  int64_t table_rows;
  int32_t dim;
  // padded layout: ids = int32 inverse [bags * max_elements]
  // CSR layout:    ids = IdT [N], offsets int64 [bags + 1]
  const void *ids;
  int64_t num_ids;  // CSR: offsets are clamped to [0, num_ids]
  const int64_t *offsets;
  const int64_t *row_base;  // CSR: [num_tables + 1]
  int32_t num_tables;
  int64_t batch;
  int32_t max_elements;
  int32_t pad_index;
  int32_t pooling;
  int32_t table_major;  // CSR: output row o is bag o ([T, B, D]) instead of b*T + t
  int32_t one_id;       // CSR, table-major: every bag holds one id (offsets[k] == k, checked)
  const float *weights;
  void *out;
  int64_t bags;
  int *err;
};

// Blocks are dispatched round-robin over the 8 XCDs of the chip, each with its
// own L2.  With table-major rows this gives XCD x the x-th contiguous eighth of
// the bags (so of the tables): a row used by several bags of a table is
// fetched into one or two L2s instead of all eight, and every block still
// writes one contiguous range.
constexpr int kXcds = 8;
__device__ __forceinline__ int64_t xcd_block(int64_t i, int64_t blocks) {
  const int64_t per = blocks / kXcds, rem = blocks % kXcds;
  const int64_t x = i % kXcds, j = i / kXcds;
  return x < rem ? x * (per + 1) + j : rem * (per + 1) + (x - rem) * per + j;
}

// Bags per lane group: 1 when the block stages its rows in LDS (8 KiB for 32
// bf16 rows of 128; on the forward over bags of 1-8 ids, 26 tables x 65536
// bags of 128 bf16, 1 bag took 337 us, 2 bags 370 us, 4 bags 429 us), 8 when
// rows are stored directly.
constexpr int kBagsPerGroupStaged = 1;
constexpr int kBagsPerGroupDirect = 8;
// Long bags (kLong: at least kLongBagLength ids per bag on average):
// kLongDepth rows in flight, and one bag per lane group when groups are wide
// (G >= 16: at most 4 groups per wave), so that the longest bag, not the
// group's total, sets the chain of row loads.  Narrow groups (G <= 8: 8 or
// more per wave) take kLongBagsNarrow bags each, pooled as one run: a wave
// waits for its slowest group, and over 8 single bags of varied lengths that
// one is far above the mean (about 2.7x for geometric lengths), while sums of
// several bags vary less.
constexpr int64_t kLongBagLength = 8;
constexpr int kLongDepth = 8;
constexpr int kLongBagsNarrow = 4;
// Rows in flight per lane for other bags (8 was slower: 474 against 407 us on
// the workload above, from the registers it takes).
constexpr int kRunDepth = 4;

template <bool kStage, bool kLong>
constexpr int bags_per_group(int g) {
  return kLong ? (g <= 8 ? kLongBagsNarrow : 1) : (kStage ? kBagsPerGroupStaged : kBagsPerGroupDirect);
}

// Resolve one id to a table row (or -1 for a pad / out-of-range slot).
template <bool kCsr>
__device__ __forceinline__ int64_t resolve_id(const PooledArgs &a, int64_t id, int64_t row_lo, int64_t row_hi) {
  if constexpr (kCsr) {
    // inside the table's own range and inside the whole table (a row_base
    // whose entries run past table_rows must not read beyond it)
    if (id >= 0 && id < row_hi - row_lo && row_lo >= 0 && row_lo + id < a.table_rows) return row_lo + id;
    record_error(a.err, kErrIndexOutOfRange);
    return -1;
  } else {
    if (id == a.pad_index) return -1;
    if (id >= 0 && id < a.table_rows) return id;
    record_error(a.err, kErrIndexOutOfRange);
    return -1;
  }
}

template <bool kCsr, typename IdT>
__device__ __forceinline__ int64_t resolve_row(const PooledArgs &a, int64_t i, int64_t row_lo,
                                               int64_t row_hi) {
  return resolve_id<kCsr>(a, static_cast<int64_t>(static_cast<const IdT *>(a.ids)[i]), row_lo, row_hi);
}

// A block pools kBagsPerBlock consecutive OUTPUT rows (CSR: output row
// o = b*T + t is bag t*B + b), so its stores form one contiguous range.  Each
// bag's [begin, end) and table base are staged in LDS.  A group of G lanes
// pools kBagsPerGroup of those bags: it streams their ids as one virtual run
// (G ids per lane-parallel load, each lane finding its bag from the running
// lengths), gathers rows kDepth at a time regardless of bag boundaries
// (packed: kRunDepth, or kLongDepth for long bags, rows of loads in flight
// per lane), accumulates in
// occurrence order, and emits a bag's pooled row when the stream passes the
// bag's end.  Lane l holds L vectors of VEC elements at columns (q*G + l)*VEC.
// kStage: finished rows go to LDS and the block writes its whole range once,
// after all of its row loads, with coalesced nontemporal 16-byte stores (a
// wave's loads and stores share one in-order completion counter, so stores
// issued between loads would lengthen every later wait).  Otherwise each row
// is stored when finished.
// Minimum waves per SIMD asked of the compiler.  Five (at most 96 VGPRs) for
// staged blocks: on bags of 1-8 ids (26 tables x 65536 bags of 128 bf16, then
// 2 bags per lane group) that took the forward from 400 to 370 us.  Long bags
// in narrow groups keep their own allocation: four bags per group leave few
// enough waves to be resident at once (8 x 16384 bags of 64 fp16), and five
// would spill.  Unstaged blocks (8 bags per group) would spill too.
template <bool kStage, bool kLong>
constexpr int pooled_min_waves(int g) {
  return (kStage && !(kLong && g <= 8)) ? 5 : 1;
}

template <typename Tag, int VEC, int G, int L, bool kCsr, typename IdT, bool kStage, bool kLong>
__global__ __launch_bounds__(kThreads, (pooled_min_waves<kStage, kLong>(G))) void pooled_kernel(PooledArgs a) {
  constexpr int kBagsPerGroup = bags_per_group<kStage, kLong>(G);
  using E = typename Tag::elem;
  using R = RawVec<Tag, VEC>;
  constexpr int kGroups = kThreads / G;
  constexpr int kBagsPerBlock = kGroups * kBagsPerGroup;
  constexpr int kDepth = kLong ? kLongDepth : kRunDepth;
  static_assert(kDepth <= 32, "one bit of `live` per row in flight");
  __shared__ int64_t s_begin[kBagsPerBlock];
  __shared__ int64_t s_len[kBagsPerBlock];
  __shared__ int64_t s_lo[kBagsPerBlock];
  __shared__ int64_t s_rows[kBagsPerBlock];

  const int lane = threadIdx.x % G;
  const int group = threadIdx.x / G;
  const int64_t block = (kCsr && a.table_major) ? xcd_block(blockIdx.x, gridDim.x) : blockIdx.x;
  const int64_t o0 = block * kBagsPerBlock;
  const int64_t nout = (a.bags - o0) < kBagsPerBlock ? (a.bags - o0) : kBagsPerBlock;

  for (int i = threadIdx.x; i < nout; i += kThreads) {
    const int64_t o = o0 + i;
    if constexpr (kCsr) {
      int64_t t, bag;
      if (a.table_major) {
        t = o / a.batch;
        bag = o;
      } else {
        const int64_t b = o / a.num_tables;
        t = o - b * a.num_tables;
        bag = t * a.batch + b;
      }
      int64_t lo = a.offsets[bag];
      int64_t hi = a.offsets[bag + 1];
      // offsets must start at 0, end at num_ids and never decrease
      if (lo < 0 || hi > a.num_ids || hi < lo || (bag == 0 && lo != 0) || (bag + 1 == a.bags && hi != a.num_ids))
        record_error(a.err, kErrIndexOutOfRange);
      lo = lo < 0 ? 0 : (lo > a.num_ids ? a.num_ids : lo);
      hi = hi < lo ? lo : (hi > a.num_ids ? a.num_ids : hi);  // decreasing offsets pool nothing
      s_begin[i] = lo;
      s_len[i] = hi - lo;
      const int64_t base = a.row_base[t];
      s_lo[i] = base;
      s_rows[i] = a.row_base[t + 1] - base;
    } else {
      s_begin[i] = o * a.max_elements;
      s_len[i] = a.max_elements;
      s_lo[i] = 0;
      s_rows[i] = a.table_rows;
    }
  }
  __syncthreads();

  const int lb0 = group * kBagsPerGroup;  // first output row of this group, block-local
  const int nb = static_cast<int>(nout - lb0 < kBagsPerGroup ? nout - lb0 : kBagsPerGroup);
  if (!kStage && nb <= 0) return;  // a staging block still joins the final barrier
  // running start of each bag in the group's virtual id sequence
  int64_t pre[kBagsPerGroup + 1];
  pre[0] = 0;
#pragma unroll
  for (int k = 0; k < kBagsPerGroup; ++k) pre[k + 1] = pre[k] + (k < nb ? s_len[lb0 + k] : 0);
  const int64_t total = pre[kBagsPerGroup];

  const E *table = static_cast<const E *>(a.table);
  E *out = static_cast<E *>(a.out);
  extern __shared__ uint4 s_stage[];  // kStage: the block's pooled rows [nout][D]
  E *staged = reinterpret_cast<E *>(s_stage);
  const int D = a.dim;
  const bool weighted = a.pooling == FLARE_POOL_WEIGHTED;
  const bool mean = a.pooling == FLARE_POOL_MEAN;

  for (int c0 = 0; nb > 0 && c0 < D; c0 += G * VEC * L) {
    float acc[L][VEC];
#pragma unroll
    for (int q = 0; q < L; ++q)
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[q][v] = 0.0f;
    int count = 0;
    int cur = 0;  // bag being pooled, group-local

    auto flush = [&]() {
      const int64_t out_row = o0 + lb0 + cur;
      const float div = static_cast<float>(count > 0 ? count : 1);
#pragma unroll
      for (int q = 0; q < L; ++q) {
        if (mean) {
#pragma unroll
          for (int v = 0; v < VEC; ++v) acc[q][v] = acc[q][v] / div;
        }
        const int col = c0 + (q * G + lane) * VEC;
        if (col < D) {
          if constexpr (kStage) store_from_f32<Tag, VEC>(staged + static_cast<int64_t>(lb0 + cur) * D + col, acc[q]);
          else store_from_f32_stream<Tag, VEC>(out + out_row * D + col, acc[q]);
        }
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[q][v] = 0.0f;
      }
      count = 0;
      ++cur;
    };

    // The ids (and weights) of the next G virtual positions are loaded before
    // the rows of the current ones, so each step of the stream waits for one
    // memory round trip (its rows), not two (its ids, then their rows).
    // Only the block-local bag of the next id is kept: its table range is read
    // from LDS when the id is resolved (fewer registers, for occupancy).
    IdT next_id = 0;
    float next_w = 1.0f;
    int next_lb = 0;
    bool next_valid = false;
    auto fetch = [&](int64_t at) {
      const int64_t vpos = at + lane;
      next_valid = vpos < total;
      if (next_valid) {
        int k = 0;  // bag of this virtual position within the group
#pragma unroll
        for (int j = 1; j < kBagsPerGroup; ++j) k += (vpos >= pre[j]) ? 1 : 0;
        const int lb = lb0 + k;
        const int64_t i = s_begin[lb] + (vpos - pre[k]);
        next_lb = lb;
        next_id = static_cast<const IdT *>(a.ids)[i];
        if (weighted) next_w = a.weights[i];
      }
    };
    fetch(0);
    for (int64_t base = 0; base < total; base += G) {
      const int64_t lo = s_lo[next_lb];
      const int64_t my_row =
          next_valid ? resolve_id<kCsr>(a, static_cast<int64_t>(next_id), lo, lo + s_rows[next_lb]) : -1;
      const float my_w = next_w;
      if (base + G < total) fetch(base + G);
      const int n = (total - base) < G ? static_cast<int>(total - base) : G;
      for (int k = 0; k < n; k += kDepth) {
        R raw[kDepth][L];
        float w[kDepth];
        uint32_t live = 0;  // bit h: position k + h holds a valid row (the row index is not kept)
#pragma unroll
        for (int h = 0; h < kDepth; ++h) {
          const int src = (k + h < n) ? (k + h) : 0;
          int64_t row = __shfl(my_row, src, G);
          w[h] = weighted ? __shfl(my_w, src, G) : 1.0f;
          if (k + h >= n) row = -1;
          live |= (row >= 0 ? 1u : 0u) << h;
#pragma unroll
          for (int q = 0; q < L; ++q) {
            const int col = c0 + (q * G + lane) * VEC;
            if (row >= 0 && col < D) raw[h][q] = load_raw<Tag, VEC>(table + row * D + col);
            else raw[h][q] = R{};
          }
        }
#pragma unroll
        for (int h = 0; h < kDepth; ++h) {
          if (k + h < n) {  // a guard, not a break: the loop stays fully unrolled
            const int64_t p = base + k + h;
            while (cur < nb - 1 && p >= pre[cur + 1]) flush();
            if ((live >> h) & 1u) {
              ++count;
#pragma unroll
              for (int q = 0; q < L; ++q) {
                float x[VEC];
                raw_to_f32<Tag, VEC>(raw[h][q], x);
#pragma unroll
                for (int v = 0; v < VEC; ++v) {
                  if (weighted) acc[q][v] += w[h] * x[v];
                  else acc[q][v] += x[v];
                }
              }
            }
          }
        }
      }
    }
    while (cur < nb) flush();  // the last bag and any empty bags after it
  }
  if constexpr (kStage) {
    // one contiguous, fully coalesced write of the block's rows (rows are a
    // multiple of 16 bytes and the output is 16-byte aligned when staging)
    __syncthreads();
    typedef unsigned int U4 __attribute__((ext_vector_type(4)));
    const int64_t n16 = nout * D * static_cast<int64_t>(sizeof(E)) / 16;
    U4 *dst = reinterpret_cast<U4 *>(out + o0 * D);
    const U4 *src = reinterpret_cast<const U4 *>(s_stage);
    for (int64_t i = threadIdx.x; i < n16; i += kThreads) __builtin_nontemporal_store(src[i], dst + i);
  }
}

// Short CSR bags (at most kShortBagLength ids per bag on average, e.g. one id
// per bag): one lane group of G lanes per kShortRows consecutive output rows.
// Lane k of the group reads bag k's offsets and table range and resolves its
// first id, so the group's kShortRows rows are gathered with all their loads
// in flight; the remaining ids of a longer bag follow one at a time.  The
// first id is loaded together with the offsets, from occurrence `bag` (where
// it is when every bag before this one holds one id), and used when the
// offsets confirm it: one dependent load fewer before the row.  Each
// pooled row is written as soon as it is done with 16-byte nontemporal
// stores, kShortRows consecutive rows forming one contiguous range per group.
// Accumulation as in pooled_kernel: fp32 from zero in occurrence order, the
// mean divides by the number of valid ids (at least 1).
constexpr int64_t kShortBagLength = 2;
constexpr int kShortRows = 4;

template <typename Tag, int VEC, int G, int L, typename IdT>
__global__ __launch_bounds__(kThreads) void pooled_short_kernel(PooledArgs a) {
  static_assert(G >= kShortRows, "one lane per bag of the group");
  using E = typename Tag::elem;
  using R = RawVec<Tag, VEC>;
  constexpr int kGroups = kThreads / G;
  const int lane = threadIdx.x % G;
  const int64_t o0 = (static_cast<int64_t>(blockIdx.x) * kGroups + threadIdx.x / G) * kShortRows;
  if (o0 >= a.bags) return;  // whole groups: the kernel has no barrier
  const E *table = static_cast<const E *>(a.table);
  E *out = static_cast<E *>(a.out);
  const int D = a.dim;
  const bool weighted = a.pooling == FLARE_POOL_WEIGHTED;
  const bool mean = a.pooling == FLARE_POOL_MEAN;

  // lane k < kShortRows: bag of output row o0 + k, its ids [lo, lo + len), its table range
  int64_t lo = 0, len = 0, base = 0, rows = 0, first = -1;
  float first_w = 1.0f;
  if (lane < kShortRows && o0 + lane < a.bags) {
    const int64_t o = o0 + lane;
    int64_t t, bag;
    if (a.table_major) {
      t = o / a.batch;
      bag = o;
    } else {
      const int64_t b = o / a.num_tables;
      t = o - b * a.num_tables;
      bag = t * a.batch + b;
    }
    // speculative first id and weight of the bag, read with its offsets
    const int64_t guess = bag < a.num_ids ? bag : 0;
    const bool can_guess = bag < a.num_ids;
    const int64_t guess_id = can_guess ? static_cast<int64_t>(static_cast<const IdT *>(a.ids)[guess]) : 0;
    const float guess_w = (can_guess && weighted) ? a.weights[guess] : 1.0f;
    int64_t hi;
    lo = a.offsets[bag];
    hi = a.offsets[bag + 1];
    // offsets must start at 0, end at num_ids and never decrease
    if (lo < 0 || hi > a.num_ids || hi < lo || (bag == 0 && lo != 0) || (bag + 1 == a.bags && hi != a.num_ids))
      record_error(a.err, kErrIndexOutOfRange);
    lo = lo < 0 ? 0 : (lo > a.num_ids ? a.num_ids : lo);
    hi = hi < lo ? lo : (hi > a.num_ids ? a.num_ids : hi);  // decreasing offsets pool nothing
    len = hi - lo;
    base = a.row_base[t];
    rows = a.row_base[t + 1] - base;
    if (len > 0) {
      if (can_guess && lo == bag) {
        first = resolve_id<true>(a, guess_id, base, base + rows);
        first_w = guess_w;
      } else {
        first = resolve_row<true, IdT>(a, lo, base, base + rows);
        if (weighted) first_w = a.weights[lo];
      }
    }
  }
  for (int c0 = 0; c0 < D; c0 += G * VEC * L) {
    R raw[kShortRows][L];
    int64_t row_k[kShortRows];
#pragma unroll
    for (int k = 0; k < kShortRows; ++k) {
      row_k[k] = __shfl(first, k, G);
#pragma unroll
      for (int q = 0; q < L; ++q) {
        const int col = c0 + (q * G + lane) * VEC;
        raw[k][q] = (row_k[k] >= 0 && col < D) ? load_raw<Tag, VEC>(table + row_k[k] * D + col) : R{};
      }
    }
#pragma unroll
    for (int k = 0; k < kShortRows; ++k) {
      const int64_t o = o0 + k;
      if (o >= a.bags) break;
      const int64_t blen = __shfl(len, k, G);
      const int64_t blo = __shfl(lo, k, G);
      const int64_t bbase = __shfl(base, k, G);
      const int64_t brows = __shfl(rows, k, G);
      const float bw = __shfl(first_w, k, G);
      float acc[L][VEC];
      int count = 0;
#pragma unroll
      for (int q = 0; q < L; ++q)
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[q][v] = 0.0f;
      if (row_k[k] >= 0) {
        ++count;
#pragma unroll
        for (int q = 0; q < L; ++q) {
          float x[VEC];
          raw_to_f32<Tag, VEC>(raw[k][q], x);
#pragma unroll
          for (int v = 0; v < VEC; ++v) {
            if (weighted) acc[q][v] += bw * x[v];
            else acc[q][v] += x[v];
          }
        }
      }
      for (int64_t i = blo + 1; i < blo + blen; ++i) {  // ids after the first (longer bags)
        const int64_t row = resolve_row<true, IdT>(a, i, bbase, bbase + brows);
        if (row < 0) continue;
        const float w = weighted ? a.weights[i] : 1.0f;
        ++count;
#pragma unroll
        for (int q = 0; q < L; ++q) {
          const int col = c0 + (q * G + lane) * VEC;
          float x[VEC];
          if (col < D) {
            load_as_f32<Tag, VEC>(table + row * D + col, x);
          } else {
#pragma unroll
            for (int v = 0; v < VEC; ++v) x[v] = 0.0f;
          }
#pragma unroll
          for (int v = 0; v < VEC; ++v) {
            if (weighted) acc[q][v] += w * x[v];
            else acc[q][v] += x[v];
          }
        }
      }
      const float div = static_cast<float>(count > 0 ? count : 1);
#pragma unroll
      for (int q = 0; q < L; ++q) {
        if (mean) {
#pragma unroll
          for (int v = 0; v < VEC; ++v) acc[q][v] = acc[q][v] / div;
        }
        const int col = c0 + (q * G + lane) * VEC;
        if (col < D) store_from_f32_stream<Tag, VEC>(out + o * D + col, acc[q]);
      }
    }
  }
}

// One id per bag in table-major order (FLARE_LAYOUT_ONE_ID_PER_BAG, checked):
// output row o is bag o and occurrence o.  One lane group of G lanes per
// kShortRows consecutive rows; lane k < kShortRows reads the id, weight and
// both offsets of row o0 + k and its table's range, none of these loads
// waiting on another, and the group then loads its rows together.  A bag
// whose offsets are not (o, o + 1) sets error bit 1 and gets a zero row.  The
// pooled row of one id is 0 + x (sum), (0 + x) / 1 (mean) or 0 + w * x
// (weighted) in fp32, rounded to nearest even: the same bits pooled_short_kernel
// writes for such a bag.
template <typename Tag, int VEC, int G, int L, typename IdT>
__global__ __launch_bounds__(kThreads) void pooled_one_kernel(PooledArgs a) {
  static_assert(G >= kShortRows, "one lane per bag of the group");
  using E = typename Tag::elem;
  using R = RawVec<Tag, VEC>;
  constexpr int kGroups = kThreads / G;
  const int lane = threadIdx.x % G;
  const int64_t o0 = (static_cast<int64_t>(blockIdx.x) * kGroups + threadIdx.x / G) * kShortRows;
  if (o0 >= a.bags) return;  // whole groups: the kernel has no barrier
  const E *table = static_cast<const E *>(a.table);
  E *out = static_cast<E *>(a.out);
  const int D = a.dim;
  const bool weighted = a.pooling == FLARE_POOL_WEIGHTED;
  const bool mean = a.pooling == FLARE_POOL_MEAN;
  int64_t row = -1;
  float w = 1.0f;
  if (lane < kShortRows && o0 + lane < a.bags) {
    const int64_t o = o0 + lane;  // < bags == num_ids (checked by the host)
    const int64_t t = o / a.batch;
    const int64_t id = static_cast<int64_t>(static_cast<const IdT *>(a.ids)[o]);
    const float wo = weighted ? a.weights[o] : 1.0f;
    const int64_t lo = a.offsets[o], hi = a.offsets[o + 1];
    const int64_t base = a.row_base[t];
    const int64_t rows = a.row_base[t + 1] - base;
    if (lo == o && hi == o + 1) {
      row = resolve_id<true>(a, id, base, base + rows);
      w = wo;
    } else {
      record_error(a.err, kErrIndexOutOfRange);
    }
  }
  for (int c0 = 0; c0 < D; c0 += G * VEC * L) {
    R raw[kShortRows][L];
    int64_t row_k[kShortRows];
#pragma unroll
    for (int k = 0; k < kShortRows; ++k) {
      row_k[k] = __shfl(row, k, G);
#pragma unroll
      for (int q = 0; q < L; ++q) {
        const int col = c0 + (q * G + lane) * VEC;
        raw[k][q] = (row_k[k] >= 0 && col < D) ? load_raw<Tag, VEC>(table + row_k[k] * D + col) : R{};
      }
    }
#pragma unroll
    for (int k = 0; k < kShortRows; ++k) {
      const int64_t o = o0 + k;
      if (o >= a.bags) break;
      const float bw = __shfl(w, k, G);
#pragma unroll
      for (int q = 0; q < L; ++q) {
        float x[VEC], acc[VEC];
        raw_to_f32<Tag, VEC>(raw[k][q], x);
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          acc[v] = 0.0f;
          if (row_k[k] >= 0) acc[v] += weighted ? bw * x[v] : x[v];
          if (mean) acc[v] = acc[v] / 1.0f;
        }
        const int col = c0 + (q * G + lane) * VEC;
        if (col < D) store_from_f32_stream<Tag, VEC>(out + o * D + col, acc);
      }
    }
  }
}

// ----------------------------------------------------------------------------
// host dispatch
// ----------------------------------------------------------------------------
int grid_for(int64_t work, int64_t per_block) {
  const int64_t g = ceil_div(work, per_block);
  return static_cast<int>(g < 1 ? 1 : (g > 0x7fffffff ? 0x7fffffff : g));
}

// Pooled rows of a block are staged in LDS and written in one coalesced pass
// when they fit this budget (16-byte vectors only).
constexpr int64_t kStageBytes = 32768;

template <typename Tag, int VEC, int L, bool kCsr, typename IdT, bool kStage, bool kLong>
int launch_pooled_gs(const PooledArgs &a, int G, hipStream_t s) {
  const int64_t per_block = (kThreads / G) * bags_per_group<kStage, kLong>(G);
  const int grid = grid_for(a.bags, per_block);
  const size_t lds = kStage ? static_cast<size_t>(per_block) * a.dim * sizeof(typename Tag::elem) : 0;
  switch (G) {
    case 4: pooled_kernel<Tag, VEC, 4, L, kCsr, IdT, kStage, kLong><<<grid, kThreads, lds, s>>>(a); break;
    case 8: pooled_kernel<Tag, VEC, 8, L, kCsr, IdT, kStage, kLong><<<grid, kThreads, lds, s>>>(a); break;
    case 16: pooled_kernel<Tag, VEC, 16, L, kCsr, IdT, kStage, kLong><<<grid, kThreads, lds, s>>>(a); break;
    case 32: pooled_kernel<Tag, VEC, 32, L, kCsr, IdT, kStage, kLong><<<grid, kThreads, lds, s>>>(a); break;
    default: pooled_kernel<Tag, VEC, 64, L, kCsr, IdT, kStage, kLong><<<grid, kThreads, lds, s>>>(a); break;
  }
  FLARE_TRY_HIP(hipGetLastError());
  return FLARE_OK;
}

template <typename Tag, int VEC, int L, bool kCsr, typename IdT, bool kLong>
int launch_pooled_g(const PooledArgs &a, int G, hipStream_t s) {
  const int64_t stage = static_cast<int64_t>(kThreads / G) * bags_per_group<true, kLong>(G) * a.dim *
                        sizeof(typename Tag::elem);
  if (VEC * sizeof(typename Tag::elem) == 16 && stage <= kStageBytes)
    return launch_pooled_gs<Tag, VEC, L, kCsr, IdT, true, kLong>(a, G, s);
  return launch_pooled_gs<Tag, VEC, L, kCsr, IdT, false, kLong>(a, G, s);
}

int group_size(int vectors, int min_g) {
  int g = min_g;
  while (g < vectors && g < 64) g <<= 1;
  return g;
}

template <typename Tag, int VEC, typename IdT>
int launch_pooled_short(const PooledArgs &a, int vectors, hipStream_t s) {
  // one 16-byte vector per lane and chunk: G lanes (at least kShortRows), L chunks per row
  int G = kShortRows;
  while (G < vectors && G < 64) G <<= 1;
  const int L = static_cast<int>(ceil_div(vectors, G));
  const int grid = grid_for(a.bags, static_cast<int64_t>(kThreads / G) * kShortRows);
#define FLARE_SHORT(G_, L_) pooled_short_kernel<Tag, VEC, G_, L_, IdT><<<grid, kThreads, 0, s>>>(a)
  if (L == 1) {
    switch (G) {
      case 4: FLARE_SHORT(4, 1); break;
      case 8: FLARE_SHORT(8, 1); break;
      case 16: FLARE_SHORT(16, 1); break;
      case 32: FLARE_SHORT(32, 1); break;
      default: FLARE_SHORT(64, 1); break;
    }
  } else if (L == 2) {
    FLARE_SHORT(64, 2);
  } else {
    return FLARE_NOT_HANDLED;
  }
#undef FLARE_SHORT
  FLARE_TRY_HIP(hipGetLastError());
  return FLARE_OK;
}

template <typename Tag, int VEC, typename IdT>
int launch_pooled_one(const PooledArgs &a, int vectors, hipStream_t s) {
  int G = kShortRows;
  while (G < vectors && G < 64) G <<= 1;
  const int L = static_cast<int>(ceil_div(vectors, G));
  const int grid = grid_for(a.bags, static_cast<int64_t>(kThreads / G) * kShortRows);
#define FLARE_ONE(G_, L_) pooled_one_kernel<Tag, VEC, G_, L_, IdT><<<grid, kThreads, 0, s>>>(a)
  if (L == 1) {
    switch (G) {
      case 4: FLARE_ONE(4, 1); break;
      case 8: FLARE_ONE(8, 1); break;
      case 16: FLARE_ONE(16, 1); break;
      case 32: FLARE_ONE(32, 1); break;
      default: FLARE_ONE(64, 1); break;
    }
  } else if (L == 2) {
    FLARE_ONE(64, 2);
  } else {
    return FLARE_NOT_HANDLED;
  }
#undef FLARE_ONE
  FLARE_TRY_HIP(hipGetLastError());
  return FLARE_OK;
}

template <typename Tag, bool kCsr, typename IdT>
int launch_pooled_tag(PooledArgs a, hipStream_t s) {
  constexpr int kWide = 16 / sizeof(typename Tag::elem);
  const bool wide = (a.dim % kWide == 0) && aligned(a.table, 16) && aligned(a.out, 16);
  const int64_t ids = kCsr ? a.num_ids : a.bags * a.max_elements;
  if (wide) {
    const int vectors = a.dim / kWide;  // 16-byte vectors per row
    if constexpr (kCsr) {
      if (a.one_id) {
        const int st = launch_pooled_one<Tag, kWide, IdT>(a, vectors, s);
        if (st != FLARE_NOT_HANDLED) return st;
      }
      if (ids <= kShortBagLength * a.bags) {
        const int st = launch_pooled_short<Tag, kWide, IdT>(a, vectors, s);
        if (st != FLARE_NOT_HANDLED) return st;
      }
    }
    if (vectors <= 64 && ids >= kLongBagLength * a.bags)
      return launch_pooled_g<Tag, kWide, 1, kCsr, IdT, true>(a, group_size(vectors, 4), s);
    if (vectors >= 8) return launch_pooled_g<Tag, kWide, 2, kCsr, IdT, false>(a, group_size(vectors / 2, 4), s);
    return launch_pooled_g<Tag, kWide, 1, kCsr, IdT, false>(a, group_size(vectors, 4), s);
  }
  return launch_pooled_g<Tag, 1, 1, kCsr, IdT, false>(a, group_size(a.dim, 8), s);
}

template <bool kCsr, typename IdT>
int launch_pooled(int dtype, const PooledArgs &a, hipStream_t s) {
  switch (dtype) {
    case FLARE_FLOAT32: return launch_pooled_tag<TagF32, kCsr, IdT>(a, s);
    case FLARE_FLOAT16: return launch_pooled_tag<TagF16, kCsr, IdT>(a, s);
    case FLARE_BFLOAT16: return launch_pooled_tag<TagBF16, kCsr, IdT>(a, s);
    default: return fail(FLARE_ERR_DTYPE, "sparse pooled gather requires float16, bfloat16 or float32 embeddings, got dtype code %d", dtype);
  }
}

int check_pooling(int pooling, const float *weights) {
  if (pooling != FLARE_POOL_SUM && pooling != FLARE_POOL_MEAN && pooling != FLARE_POOL_WEIGHTED)
    return fail(FLARE_ERR_ARGUMENT, "unknown pooling mode %d", pooling);
  if (pooling == FLARE_POOL_WEIGHTED && !weights)
    return fail(FLARE_ERR_ARGUMENT, "weighted pooling requires per-sample weights");
  return FLARE_OK;
}

}  // namespace
}  // namespace flare

using namespace flare;

extern "C" int flare_gather(const void *emb, int32_t value_dtype, int64_t emb_rows, int32_t dim,
                            const int32_t *inverse, int64_t slots, int32_t pad_index, void *out,
                            void *stream) {
  const int esz = storage_bytes(value_dtype);
  if (esz == 0)
    return fail(FLARE_ERR_DTYPE, "sparse gather requires float16, bfloat16 or float32 embeddings, got dtype code %d", value_dtype);
  if (dim <= 0 || slots < 0 || emb_rows < 0) return fail(FLARE_ERR_SHAPE, "invalid gather sizes");
  if (slots == 0) return FLARE_OK;
  int st = FLARE_OK;
  int *err = device_error_word(&st);
  if (!err) return st;
  hipStream_t s = as_stream(stream);
  const int64_t row_bytes = static_cast<int64_t>(dim) * esz;
  int ch = 2;
  for (int c : {16, 8, 4}) {
    if (row_bytes % c == 0 && aligned(emb, c) && aligned(out, c)) { ch = c; break; }
  }
  if (ch == 2 && (row_bytes % 2 != 0)) return fail(FLARE_ERR_SHAPE, "row size not a multiple of 2 bytes");
  const int64_t chunks = row_bytes / ch;
  const int64_t total = slots * chunks;
  const int grid = static_cast<int>(std::min<int64_t>(ceil_div(total, kThreads), 1 << 20));
  const char *e = static_cast<const char *>(emb);
  char *o = static_cast<char *>(out);
  switch (ch) {
    case 16: gather_rows_kernel<16><<<grid, kThreads, 0, s>>>(e, emb_rows, chunks, inverse, slots, pad_index, o, err); break;
    case 8: gather_rows_kernel<8><<<grid, kThreads, 0, s>>>(e, emb_rows, chunks, inverse, slots, pad_index, o, err); break;
    case 4: gather_rows_kernel<4><<<grid, kThreads, 0, s>>>(e, emb_rows, chunks, inverse, slots, pad_index, o, err); break;
    default: gather_rows_kernel<2><<<grid, kThreads, 0, s>>>(e, emb_rows, chunks, inverse, slots, pad_index, o, err); break;
  }
  FLARE_TRY_HIP(hipGetLastError());
  return FLARE_OK;
}

extern "C" int flare_gather_pooled(const void *emb, int32_t value_dtype, int64_t emb_rows,
                                   int32_t dim, const int32_t *inverse, int64_t batch,
                                   int32_t features, int32_t max_elements, int32_t pad_index,
                                   int32_t pooling, const float *weights, void *out,
                                   void *stream) {
  if (storage_bytes(value_dtype) == 0)
    return fail(FLARE_ERR_DTYPE, "sparse pooled gather requires float16, bfloat16 or float32 embeddings, got dtype code %d", value_dtype);
  if (features <= 0 || max_elements <= 0)
    return fail(FLARE_ERR_WIDTH, "Sparse embedding pooled operations require positive target widths, got (%d, %d).", features, max_elements);
  if (dim <= 0 || batch < 0 || emb_rows < 0) return fail(FLARE_ERR_SHAPE, "invalid pooled gather sizes");
  FLARE_TRY(check_pooling(pooling, weights));
  const int64_t bags = batch * features;
  if (bags == 0) return FLARE_OK;
  int st = FLARE_OK;
  int *err = device_error_word(&st);
  if (!err) return st;
  PooledArgs a{};
  a.table = emb;
  a.table_rows = emb_rows;
  a.dim = dim;
  a.ids = inverse;
  a.max_elements = max_elements;
  a.pad_index = pad_index;
  a.pooling = pooling;
  a.weights = weights;
  a.out = out;
  a.bags = bags;
  a.err = err;
  return launch_pooled<false, int32_t>(value_dtype, a, as_stream(stream));
}

extern "C" int flare_gather_pooled_csr(const void *table, int32_t value_dtype, int64_t table_rows,
                                       int32_t dim, const void *ids, int32_t id_dtype, int64_t n,
                                       const int64_t *offsets, int32_t num_tables, int64_t batch,
                                       const int64_t *row_base, int32_t pooling,
                                       int32_t layout, const float *weights, void *out,
                                       void *stream) {
  if (storage_bytes(value_dtype) == 0)
    return fail(FLARE_ERR_DTYPE, "sparse pooled gather requires float16, bfloat16 or float32 embeddings, got dtype code %d", value_dtype);
  if (id_dtype != FLARE_INT32 && id_dtype != FLARE_INT64)
    return fail(FLARE_ERR_DTYPE, "CSR ids must be int32 or int64, got dtype code %d", id_dtype);
  if (num_tables <= 0 || batch < 0 || dim <= 0 || table_rows < 0 || n < 0)
    return fail(FLARE_ERR_SHAPE, "invalid CSR pooled gather sizes");
  FLARE_TRY(check_pooling(pooling, weights));
  const bool one_id = (layout & FLARE_LAYOUT_ONE_ID_PER_BAG) != 0;
  layout &= ~FLARE_LAYOUT_ONE_ID_PER_BAG;
  if (layout != FLARE_LAYOUT_SAMPLE_MAJOR && layout != FLARE_LAYOUT_TABLE_MAJOR)
    return fail(FLARE_ERR_ARGUMENT, "unknown pooled row layout %d", layout);
  const int64_t bags = batch * num_tables;
  if (one_id && layout == FLARE_LAYOUT_TABLE_MAJOR && n != bags)
    return fail(FLARE_ERR_SHAPE, "one id per bag needs as many ids as bags (%lld ids, %lld bags)",
                static_cast<long long>(n), static_cast<long long>(bags));
  if (bags == 0) return FLARE_OK;
  int st = FLARE_OK;
  int *err = device_error_word(&st);
  if (!err) return st;
  PooledArgs a{};
  a.table_major = layout == FLARE_LAYOUT_TABLE_MAJOR ? 1 : 0;
  a.one_id = (one_id && a.table_major) ? 1 : 0;  // ignored with sample-major rows, as in the dedup
  a.table = table;
  a.table_rows = table_rows;
  a.dim = dim;
  a.ids = ids;
  a.num_ids = n;
  a.offsets = offsets;
  a.row_base = row_base;
  a.num_tables = num_tables;
  a.batch = batch;
  a.pooling = pooling;
  a.weights = weights;
  a.out = out;
  a.bags = bags;
  a.err = err;
  hipStream_t s = as_stream(stream);
  if (id_dtype == FLARE_INT32) return launch_pooled<true, int32_t>(value_dtype, a, s);
  return launch_pooled<true, int64_t>(value_dtype, a, s);
}
