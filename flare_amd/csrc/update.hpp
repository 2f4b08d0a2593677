// Deterministic segment reduction and the fused sparse optimizer row update:
// the kernels (sums, fold_chunks, fold, apply), their arguments and the
// launch sequence.  Instantiated per value dtype in update_rows.hip,
// update_f32.hip, update_f16.hip and update_bf16.hip (compiled in parallel);
// backward.hip dispatches to them through launch_update.
#pragma once

#include "backward.hpp"

#include <algorithm>
#include <cmath>

namespace flare {

// ----------------------------------------------------------------------------
// update: deterministic segment reduction + optimizer
// ----------------------------------------------------------------------------
// Workspace word (UpdateArgs::meta) set by the CSR dedup when each occurrence
// is its own gradient row (one id per bag, table-major rows): no gradient row
// is stored or sorted, the sorted position's occurrence is the row.
constexpr int kMetaGradIdent = 6;
enum ApplyMode : int { kModeRows = 0, kModeUnique = 1, kModeSgd = 2, kModeAdam = 3, kModeAdagrad = 4 };
enum GradRowMode : int { kGradRowOcc = 0, kGradRowDiv = 1, kGradRowArray = 2 };
enum ScaleMode : int { kScaleNone = 0, kScaleMul = 1, kScaleDiv = 2 };

struct UpdateArgs {
  const uint32_t *sk;
  const uint32_t *sv;
  const uint32_t *run_start;
  const uint32_t *unit_first_run;
  const uint32_t *meta;
  const uint32_t *run_rank;
  int32_t *inverse_out;
  const void *grad;
  int grad_bf16;       // grad holds bfloat16 (the reference's gradient transport dtype), else float32
  const uint32_t *reject;  // when non-null and set: a non-finite gradient, the update does nothing
  uint32_t grad_rows;  // rows of grad when > 0: gradient rows read from the workspace are checked
  int grad_mode;
  uint32_t grad_div;
  const uint32_t *grad_row;
  int scale_mode;
  const float *scale;  // weights (kScaleMul) or divisors (kScaleDiv), per occurrence
  const uint32_t *sorted_grad_row;  // gradient row per sorted position, or null
  const float *sorted_scale;        // scale per sorted position, or null
  const uint32_t *run_grad_row;     // gradient row of each key's first position (with sorted_grad_row)
  const float *run_scale;           // scale of each key's first position (with sorted_scale)
  int use_norm;
  float norm;
  int dim;
  float *partial;
  float *sums;  // [runs][dim] per-key gradient sums (optimizer modes)
  const uint32_t *run_key;
  uint32_t *hot_runs;  // keys spanning more than kInlineSpan + 1 units (meta[2] of them)
  void *out;           // kModeRows / kModeUnique results: float32, or bfloat16 when out_bf16
  int out_bf16;
  void *table;
  float *s0;
  float *s1;
  int32_t *step;
  float lr, eps, b1, b2, omb1, omb2;
  double ln_b1, ln_b2;  // natural logs of the Adam betas (bias corrections 1 - beta^step)
  uint32_t units;
  uint32_t n;
  int *err;
};

template <int G>
__device__ __forceinline__ double group_sum(double v) {
#pragma unroll
  for (int m = G / 2; m > 0; m >>= 1) v += __shfl_xor(v, m, G);
  return v;
}

// Row state loaded ahead of the gradient sum (SGD / Adagrad rows, the
// destination rank of a reduced gradient).
template <int NC, int VEC>
struct RowAhead {
  float w[NC][VEC];
  float s0;
  int64_t dest;
};

template <typename Tag, int VEC, int G, int NC, int MODE>
__device__ __forceinline__ void load_ahead(const UpdateArgs &a, uint32_t r, uint32_t key,
                                           RowAhead<NC, VEC> &ahead, int lane) {
  if constexpr (MODE == kModeUnique) {
    ahead.dest = a.run_rank[r];
  } else if constexpr (MODE == kModeSgd || MODE == kModeAdagrad) {
    using E = typename Tag::elem;
    const E *table = static_cast<const E *>(a.table);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int col = (c * G + lane) * VEC;
      if (col < a.dim) {
        load_as_f32<Tag, VEC>(table + static_cast<int64_t>(key) * a.dim + col, ahead.w[c]);
      } else {
#pragma unroll
        for (int v = 0; v < VEC; ++v) ahead.w[c][v] = 0.0f;
      }
    }
    if constexpr (MODE == kModeAdagrad) ahead.s0 = a.s0[key];
  }
}

// A finished keyed sum written to the output: float32, or rounded to nearest
// even bfloat16 (the gradient transport dtype, train_worker.py:518-522) in the
// same store that would have written the float32 row.
template <int VEC>
__device__ __forceinline__ void store_out(const UpdateArgs &a, int64_t at, const float (&x)[VEC]) {
  if (a.out_bf16) store_from_f32<TagBF16, VEC>(static_cast<uint16_t *>(a.out) + at, x);
  else store_f32<VEC>(static_cast<float *>(a.out) + at, x);
}

template <typename Tag, int VEC, int G, int NC, int MODE>
__device__ __forceinline__ void apply_update(const UpdateArgs &a, uint32_t key, float (&g)[NC][VEC],
                                             const RowAhead<NC, VEC> &ahead, int lane) {
  const int D = a.dim;
  if (a.use_norm) {
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int v = 0; v < VEC; ++v) g[c][v] = g[c][v] / a.norm;
  }
  if constexpr (MODE == kModeRows || MODE == kModeUnique) {
    const int64_t row = (MODE == kModeRows) ? static_cast<int64_t>(key) : ahead.dest;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int col = (c * G + lane) * VEC;
      if (col < D) store_out<VEC>(a, row * D + col, g[c]);
    }
  } else {
    using E = typename Tag::elem;
    E *table = static_cast<E *>(a.table);
    const int64_t row = key;
    if constexpr (MODE == kModeAdagrad) {
      double ss = 0.0;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int col = (c * G + lane) * VEC;
        if (col < D)
#pragma unroll
          for (int v = 0; v < VEC; ++v) ss += static_cast<double>(g[c][v]) * static_cast<double>(g[c][v]);
      }
      ss = group_sum<G>(ss);
      const float accn = static_cast<float>(static_cast<double>(ahead.s0) + ss / static_cast<double>(D));
      const float den = sqrtf(accn) + a.eps;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int col = (c * G + lane) * VEC;
        if (col >= D) continue;
        float w[VEC];
#pragma unroll
        for (int v = 0; v < VEC; ++v) w[v] = ahead.w[c][v] - (a.lr * g[c][v]) / den;
        store_from_f32<Tag, VEC>(table + row * D + col, w);
      }
      if (lane == 0) a.s0[row] = accn;
    } else if constexpr (MODE == kModeSgd) {
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int col = (c * G + lane) * VEC;
        if (col >= D) continue;
        float w[VEC];
#pragma unroll
        for (int v = 0; v < VEC; ++v) w[v] = ahead.w[c][v] - a.lr * g[c][v];
        store_from_f32<Tag, VEC>(table + row * D + col, w);
      }
    } else {  // Adam: m, v and the row are loaded here (too many registers to load ahead)
      const int32_t st = a.step[row] + 1;
      // beta^step as exp(step * ln beta) in double, ln beta from the host: a few
      // double ulps from pow, so the same bias corrections once rounded to float,
      // at a quarter of pow's cost (on 1.1M rows of 128: 643 against 849 us)
      const float bc1 = static_cast<float>(1.0 - exp(static_cast<double>(st) * a.ln_b1));
      const float bc2 = static_cast<float>(1.0 - exp(static_cast<double>(st) * a.ln_b2));
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int col = (c * G + lane) * VEC;
        if (col >= D) continue;
        float w[VEC], m[VEC], v2[VEC];
        load_as_f32<Tag, VEC>(table + row * D + col, w);
        load_f32<VEC>(a.s0 + row * D + col, m);
        load_f32<VEC>(a.s1 + row * D + col, v2);
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          const float gv = g[c][v];
          m[v] = a.b1 * m[v] + a.omb1 * gv;
          v2[v] = a.b2 * v2[v] + a.omb2 * (gv * gv);
          const float mh = m[v] / bc1;
          const float vh = v2[v] / bc2;
          w[v] = w[v] - (a.lr * mh) / (sqrtf(vh) + a.eps);
        }
        store_f32<VEC>(a.s0 + row * D + col, m);
        store_f32<VEC>(a.s1 + row * D + col, v2);
        store_from_f32<Tag, VEC>(table + row * D + col, w);
      }
      if (lane == 0) a.step[row] = st;
    }
  }
}

// A key is "short" when all its sorted positions lie in one unit and there
// are at most kShortRun of them: apply_kernel sums its gradient rows itself
// (all loads in flight at once), so no per-key sum is written for it.  Every
// other key goes through sums_kernel.
constexpr uint32_t kShortRun = 4;
// A key whose positions span more than kInlineSpan + 1 units is "hot": its
// unit partials are folded by a whole block (fold_kernel) instead of one
// lane group of apply_kernel.
constexpr uint32_t kInlineSpan = 8;
// Lane groups launched for apply_kernel at most: fewer, busier blocks beat
// one block per 8 keys once there are more keys than the GPU holds at once.
constexpr int64_t kApplyGroups = 131072;
// A hot key spanning more than kFoldChunk units is folded in two levels: each
// run of kFoldChunk consecutive unit partials left to right (in parallel over
// the runs, fold_chunks_kernel), then the run results left to right
// (fold_kernel).  Keys of up to kFoldChunk units are folded left to right.
constexpr uint32_t kFoldChunk = 64;
// Partial rows per lane group and fold round (at most; fewer for wide rows).
constexpr int kFoldDepth = 16;
// Rows of a lane group in flight in the folds: kFoldDepth for lanes of up to
// 4 floats, half as many for 8-float lanes (same registers).
__host__ __device__ constexpr int fold_rows(int nc, int vec) { return kFoldDepth / nc / (vec > 4 ? vec / 4 : 1); }

// VEC consecutive gradient elements as float32 (a bfloat16 transport gradient
// widens exactly, so this equals casting first and reducing after).
// kGrad: bit 1 bfloat16 gradient, bit 2 streamed.  When each gradient row is
// read about once (no more occurrences than rows: one id per bag), the 16- and
// 8-byte loads are nontemporal and stream past L2 instead of evicting lines
// that others reuse (sums_kernel 173 -> 153 us on 1.26M rows of 512 bytes).
// With longer bags several occurrences read one bag's row, and L2 hits pay.
constexpr int kGradBf16 = 1;
constexpr int kGradStream = 2;

template <int VEC, int kGrad>
__device__ __forceinline__ void load_grad(const UpdateArgs &a, int64_t offset, float (&out)[VEC]) {
  constexpr bool kBf16 = (kGrad & kGradBf16) != 0;
  constexpr bool kStream = (kGrad & kGradStream) != 0;
  if constexpr (kBf16 && kStream && VEC == 8) {
    typedef unsigned int U4 __attribute__((ext_vector_type(4)));
    const U4 raw = __builtin_nontemporal_load(
        reinterpret_cast<const U4 *>(static_cast<const uint16_t *>(a.grad) + offset));
    uint16_t tmp[8];
    __builtin_memcpy(tmp, &raw, sizeof(raw));
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = TagBF16::to_f32(tmp[i]);
  } else if constexpr (kBf16 && kStream && VEC == 4) {
    typedef unsigned int U2 __attribute__((ext_vector_type(2)));
    const U2 raw = __builtin_nontemporal_load(
        reinterpret_cast<const U2 *>(static_cast<const uint16_t *>(a.grad) + offset));
    uint16_t tmp[4];
    __builtin_memcpy(tmp, &raw, sizeof(raw));
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = TagBF16::to_f32(tmp[i]);
  } else if constexpr (kBf16) {
    load_as_f32<TagBF16, VEC>(static_cast<const uint16_t *>(a.grad) + offset, out);
  } else if constexpr (kStream && VEC == 4) {
    typedef float F4 __attribute__((ext_vector_type(4)));
    const F4 raw = __builtin_nontemporal_load(reinterpret_cast<const F4 *>(static_cast<const float *>(a.grad) + offset));
    out[0] = raw.x;
    out[1] = raw.y;
    out[2] = raw.z;
    out[3] = raw.w;
  } else {
    load_f32<VEC>(static_cast<const float *>(a.grad) + offset, out);
  }
}

// Gradient rows recorded in the workspace are in range whenever the batch's
// offsets were valid; after invalid offsets (reported by the dedup) a row is
// checked before it is read.
__device__ __forceinline__ uint32_t checked_grad_row(const UpdateArgs &a, uint32_t gr) {
  if (a.grad_rows == 0 || gr < a.grad_rows) return gr;
  record_error(a.err, kErrIndexOutOfRange);
  return 0;
}

__device__ __forceinline__ uint32_t grad_row_of(const UpdateArgs &a, uint32_t o) {
  if (a.grad_mode == kGradRowDiv) return o / a.grad_div;
  if (a.grad_mode == kGradRowArray) return a.grad_row[o];
  return o;
}

__device__ __forceinline__ float scaled(const UpdateArgs &a, float x, float sc) {
  if (a.scale_mode == kScaleMul) return x * sc;
  if (a.scale_mode == kScaleDiv) return x / sc;
  return x;
}

// Segment sums of the long keys.  One group of G lanes per unit of
// kReduceUnit sorted positions lists the unit's positions that belong to long
// keys and streams their gradient rows eight at a time, in order; at each key
// head the running fp32 sum of the finished piece is stored and restarted.  A
// piece holding a whole key goes to its destination (the per-key sums for an
// optimizer, or straight to the output for scatter / reduced gradients); a
// piece of a key that spans units goes to this unit's partial slot (1 = the
// key's first piece, 0 = a later one) for apply_kernel to fold.  The group
// also writes the inverse (rank of the key) of every position of the unit.
template <typename Tag, int VEC, int G, int NC, int MODE, int kGrad>
__global__ __launch_bounds__(256) void sums_kernel(UpdateArgs a) {
  if (a.reject && *a.reject) return;
  const bool ident = a.meta[kMetaGradIdent] != 0;
  constexpr int kGroups = 256 / G;
  constexpr int kPPL = kReduceUnit / G;  // sorted positions per lane in the prefetch
  constexpr bool kDirect = MODE == kModeRows || MODE == kModeUnique;
  __shared__ uint32_t s_grow[kGroups][kReduceUnit];
  __shared__ float s_scale[kGroups][kReduceUnit];
  __shared__ uint32_t s_dest[kGroups][kReduceUnit];
  __shared__ uint8_t s_list[kGroups][kReduceUnit];

  const int lane = threadIdx.x % G;
  const int group = threadIdx.x / G;
  const int group_lane0 = (threadIdx.x & 63) - lane;  // first lane of this group in the wave
  const uint64_t group_mask = (G == 64) ? ~0ull : ((1ull << G) - 1);
  const uint32_t u = blockIdx.x * kGroups + group;
  const uint32_t nvalid = a.meta[0];
  const uint32_t j0 = u * kReduceUnit;
  const bool active = (u < a.units) && (j0 < nvalid);
  const uint32_t j1 = active ? min(j0 + kReduceUnit, nvalid) : j0;
  const int cnt = static_cast<int>(j1 - j0);
  const int D = a.dim;
  const uint32_t r0 = active ? a.unit_first_run[u] : 0;

  // occurrence and key head of every position
  uint32_t occ[kPPL];
  uint32_t keyv[kPPL];
  uint64_t heads = 0;
  const bool tail_head = !active || j1 >= nvalid || (a.sk[j1] != a.sk[j1 - 1]);
#pragma unroll
  for (int q = 0; q < kPPL; ++q) {
    const int p = q * G + lane;
    bool head = false;
    occ[q] = 0;
    keyv[q] = 0;
    if (p < cnt) {
      const uint32_t j = j0 + p;
      uint32_t o = a.sv[j];
      if (o >= a.n) {  // only if the sort was corrupted (tripped spin guard)
        record_error(a.err, kErrSpinGuard);
        o = 0;
      }
      occ[q] = o;
      keyv[q] = a.sk[j];
      head = (j == 0) || (keyv[q] != a.sk[j - 1]);
    }
    const uint64_t bal = __ballot(head);
    heads |= ((bal >> group_lane0) & group_mask) << (q * G);
  }
  // long positions: their gradient row, scale and (scatter) destination key
  uint64_t longmask = 0;
#pragma unroll
  for (int q = 0; q < kPPL; ++q) {
    const int p = q * G + lane;
    bool lng = false;
    if (p < cnt) {
      const uint64_t le = (p == 63) ? ~0ull : ((2ull << p) - 1);
      const uint64_t below = heads & le;
      const uint64_t above = heads & ~le;
      const int ps = below ? 63 - __builtin_clzll(below) : -1;
      const int pe = above ? __builtin_ctzll(above) : cnt;
      const bool cross_right = (pe == cnt) && !tail_head;
      lng = ps < 0 || cross_right || static_cast<uint32_t>(pe - ps) > kShortRun;
      if (lng) {
        const uint32_t j = j0 + p;
        s_grow[group][p] = checked_grad_row(a, ident ? occ[q] : (a.sorted_grad_row ? a.sorted_grad_row[j]
                                                                                   : grad_row_of(a, occ[q])));
        s_scale[group][p] = (a.scale_mode == kScaleNone) ? 1.0f
                            : (a.sorted_scale ? a.sorted_scale[j] : a.scale[occ[q]]);
        if constexpr (MODE == kModeRows) s_dest[group][p] = keyv[q];
      }
    }
    const uint64_t bal = __ballot(lng);
    longmask |= ((bal >> group_lane0) & group_mask) << (q * G);
  }
#pragma unroll
  for (int q = 0; q < kPPL; ++q) {
    const int p = q * G + lane;
    if (p < cnt && ((longmask >> p) & 1ull))
      s_list[group][__popcll(longmask & ((1ull << p) - 1))] = static_cast<uint8_t>(p);
  }
  if constexpr (MODE == kModeUnique) {
    // rank of each key of the unit: runs r0 .. r0 + (heads after position 0)
    const int nruns = 1 + __popcll(heads & ~1ull);
    for (int k = lane; k < nruns && active && longmask; k += G) s_dest[group][k] = a.run_rank[r0 + k];
  }
  __syncthreads();
  if (!active) return;

  const int nlong = __popcll(longmask);
  float acc[NC][VEC];
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[c][v] = 0.0f;
  int piece_first = -1;
  int prev = 0;

  auto flush = [&](int pf, int pl) {
    const bool starts = (heads >> pf) & 1ull;
    const bool ends_here = (pl + 1 < cnt) || tail_head;
    const bool whole = starts && ends_here;
    const uint64_t le = (pf == 63) ? ~0ull : ((2ull << pf) - 1);
    const int k = __popcll(heads & ~1ull & le);  // key index within the unit
    float *dst = nullptr;
    int64_t out_at = -1;  // kDirect whole keys: element offset of the key's output row
    if (whole) {
      if constexpr (MODE == kModeRows) {
        out_at = static_cast<int64_t>(s_dest[group][pf]) * D;
      } else if constexpr (MODE == kModeUnique) {
        out_at = static_cast<int64_t>(s_dest[group][k]) * D;
      } else {
        dst = a.sums + static_cast<int64_t>(r0 + k) * D;
      }
    } else {
      dst = a.partial + (static_cast<size_t>(u) * 2 + (starts ? 1 : 0)) * D;
      if (starts && lane == 0) {
        // head piece of a key that continues past this unit: hot when the key
        // still holds the position kInlineSpan + 1 units further on
        const uint32_t probe = (u + kInlineSpan + 1) * kReduceUnit;
        if (probe < nvalid && a.sk[probe] == a.sk[j0 + pf])
          a.hot_runs[atomicAdd(const_cast<uint32_t *>(a.meta) + 2, 1u)] = r0 + k;
      }
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int col = (c * G + lane) * VEC;
      if (kDirect && whole && a.use_norm) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[c][v] = acc[c][v] / a.norm;
      }
      if (col < D) {
        if (out_at >= 0) store_out<VEC>(a, out_at + col, acc[c]);
        else store_f32<VEC>(dst + col, acc[c]);
      }
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[c][v] = 0.0f;
    }
  };

  for (int i0 = 0; i0 < nlong; i0 += 8) {
    float x[8][NC][VEC];
    float sc[8];
    int pos[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const bool ok = i0 + t < nlong;
      pos[t] = ok ? s_list[group][i0 + t] : 0;
      const int64_t gr = ok ? static_cast<int64_t>(s_grow[group][pos[t]]) : 0;
      sc[t] = ok ? s_scale[group][pos[t]] : 0.0f;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int col = (c * G + lane) * VEC;
        if (ok && col < D) {
          load_grad<VEC, kGrad>(a, gr * D + col, x[t][c]);
        } else {
#pragma unroll
          for (int v = 0; v < VEC; ++v) x[t][c][v] = 0.0f;
        }
      }
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      if (i0 + t >= nlong) break;
      const int p = pos[t];
      if (piece_first >= 0 && ((heads >> p) & 1ull)) {
        flush(piece_first, prev);
        piece_first = -1;
      }
      if (piece_first < 0) piece_first = p;
      prev = p;
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[c][v] += scaled(a, x[t][c][v], sc[t]);
    }
  }
  if (piece_first >= 0) flush(piece_first, prev);

  if (a.inverse_out) {
#pragma unroll
    for (int q = 0; q < kPPL; ++q) {
      const int pos = q * G + lane;
      if (pos < cnt) {
        const uint64_t upto = (pos == 63) ? ~0ull : ((2ull << pos) - 1);
        const uint32_t rr = r0 + __popcll(heads & upto & ~1ull);
        a.inverse_out[occ[q]] = static_cast<int32_t>(a.run_rank[rr]);
      }
    }
  }
}

// Row-parallel apply over keys (runs), after sums_kernel.  A short key's
// gradient rows are summed here in occurrence order; a long key whose
// positions lie in one unit takes its sum from sums_kernel; a key spanning
// several units is folded from the unit partials left to right: the first
// unit's slot 1, then slot 0 of each following unit.  The table row (and
// Adagrad accumulator) is loaded before the gradient.
template <typename Tag, int VEC, int G, int NC, int MODE, int kGrad>
__global__ __launch_bounds__(256) void apply_kernel(UpdateArgs a) {
  if (a.reject && *a.reject) return;
  constexpr int kGroups = 256 / G;
  constexpr bool kDirect = MODE == kModeRows || MODE == kModeUnique;
  static_assert(G >= static_cast<int>(kShortRun), "one lane per position of a short key");
  const int lane = threadIdx.x % G;
  const int D = a.dim;
  const uint32_t runs = a.meta[1];
  const uint32_t stride = gridDim.x * kGroups;
  // fold_kernel (launched before) has read the hot-key count: clear it for
  // the next update that reuses this dedup
  if (blockIdx.x == 0 && threadIdx.x == 0) const_cast<uint32_t *>(a.meta)[2] = 0;
  for (uint32_t r = blockIdx.x * kGroups + threadIdx.x / G; r < runs; r += stride) {
    const uint32_t seg_start = a.run_start[r];
    const uint32_t seg_end = a.run_start[r + 1];
    const uint32_t key = a.run_key[r];
    if (seg_end <= seg_start || seg_end > a.n) continue;  // only after a tripped spin guard
    const uint32_t h = seg_start / kReduceUnit;
    const uint32_t last = (seg_end - 1) / kReduceUnit;
    const uint32_t len = seg_end - seg_start;
    const bool is_short = (h == last) && len <= kShortRun;
    if (kDirect && h == last && !is_short) continue;  // written by sums_kernel
    if (last - h > kInlineSpan) continue;             // hot key: fold_kernel
    RowAhead<NC, VEC> ahead;
    load_ahead<Tag, VEC, G, NC, MODE>(a, r, key, ahead, lane);
    float g[NC][VEC];
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int v = 0; v < VEC; ++v) g[c][v] = 0.0f;
    if (is_short) {
      uint32_t my_gr = 0;
      float my_sc = 1.0f;
      if (len == 1 && a.sorted_grad_row && (a.scale_mode == kScaleNone || a.sorted_scale)) {
        // one occurrence: its gradient row was recorded with the key
        my_gr = checked_grad_row(a, a.run_grad_row[r]);
        if (a.scale_mode != kScaleNone) my_sc = a.run_scale[r];
      } else if (static_cast<uint32_t>(lane) < len) {
        const uint32_t j = seg_start + lane;
        const bool ident = a.meta[kMetaGradIdent] != 0;
        const bool need_occ = ident || !a.sorted_grad_row || (a.scale_mode != kScaleNone && !a.sorted_scale);
        uint32_t o = 0;
        if (need_occ) {
          o = a.sv[j];
          if (o >= a.n) {
            record_error(a.err, kErrSpinGuard);
            o = 0;
          }
        }
        my_gr = checked_grad_row(a, ident ? o : (a.sorted_grad_row ? a.sorted_grad_row[j] : grad_row_of(a, o)));
        if (a.scale_mode != kScaleNone) my_sc = a.sorted_scale ? a.sorted_scale[j] : a.scale[o];
      }
      for (uint32_t k = 0; k < len; k += 4) {
        float x[4][NC][VEC];
        float sc[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const bool ok = k + t < len;
          const int src = ok ? static_cast<int>(k + t) : 0;
          const int64_t gr = static_cast<int64_t>(__shfl(my_gr, src, G));
          sc[t] = __shfl(my_sc, src, G);
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const int col = (c * G + lane) * VEC;
            if (ok && col < D) {
              load_grad<VEC, kGrad>(a, gr * D + col, x[t][c]);
            } else {
#pragma unroll
              for (int v = 0; v < VEC; ++v) x[t][c][v] = 0.0f;
            }
          }
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          if (k + t >= len) break;
#pragma unroll
          for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int v = 0; v < VEC; ++v) g[c][v] += scaled(a, x[t][c][v], sc[t]);
        }
      }
    } else {
      const float *first = (h == last) ? a.sums + static_cast<int64_t>(r) * D
                                       : a.partial + (static_cast<size_t>(h) * 2 + 1) * D;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int col = (c * G + lane) * VEC;
        if (col < D) load_f32<VEC>(first + col, g[c]);
      }
      uint32_t x = h + 1;
      for (; x + 4 <= last + 1; x += 4) {  // four partial loads in flight
        float y[4][NC][VEC];
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const int col = (c * G + lane) * VEC;
            if (col < D) load_f32<VEC>(a.partial + (static_cast<size_t>(x + t) * 2) * D + col, y[t][c]);
          }
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int v = 0; v < VEC; ++v) g[c][v] += y[t][c][v];
      }
      for (; x <= last; ++x) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const int col = (c * G + lane) * VEC;
          if (col < D) {
            float y[VEC];
            load_f32<VEC>(a.partial + (static_cast<size_t>(x) * 2) * D + col, y);
#pragma unroll
            for (int v = 0; v < VEC; ++v) g[c][v] += y[v];
          }
        }
      }
    }
    apply_update<Tag, VEC, G, NC, MODE>(a, key, g, ahead, lane);
  }
}

// ----------------------------------------------------------------------------
// Optimizer updates in one pass over the sorted positions
// ----------------------------------------------------------------------------
// Gradient rows kept packed (storage bits) while their loads are in flight.
template <int VEC, int kGrad>
using GradRaw = typename Raw<VEC * ((kGrad & kGradBf16) ? 2 : 4)>::type;

template <int VEC, int kGrad>
__device__ __forceinline__ GradRaw<VEC, kGrad> load_grad_raw(const UpdateArgs &a, int64_t offset) {
  using R = GradRaw<VEC, kGrad>;
  constexpr bool kBf16 = (kGrad & kGradBf16) != 0;
  constexpr bool kStream = (kGrad & kGradStream) != 0;
  const void *p = kBf16 ? static_cast<const void *>(static_cast<const uint16_t *>(a.grad) + offset)
                        : static_cast<const void *>(static_cast<const float *>(a.grad) + offset);
  R r;
  if constexpr (kStream && sizeof(R) == 16) {
    typedef unsigned int U4 __attribute__((ext_vector_type(4)));
    const U4 v = __builtin_nontemporal_load(static_cast<const U4 *>(p));
    __builtin_memcpy(&r, &v, sizeof(r));
  } else if constexpr (kStream && sizeof(R) == 32) {
    typedef unsigned int U4 __attribute__((ext_vector_type(4)));
    const U4 v0 = __builtin_nontemporal_load(static_cast<const U4 *>(p));
    const U4 v1 = __builtin_nontemporal_load(static_cast<const U4 *>(p) + 1);
    __builtin_memcpy(&r, &v0, 16);
    __builtin_memcpy(reinterpret_cast<char *>(&r) + 16, &v1, 16);
  } else if constexpr (kStream && sizeof(R) == 8) {
    typedef unsigned int U2 __attribute__((ext_vector_type(2)));
    const U2 v = __builtin_nontemporal_load(static_cast<const U2 *>(p));
    __builtin_memcpy(&r, &v, sizeof(r));
  } else {
    r = *static_cast<const R *>(p);
  }
  return r;
}

template <int VEC, int kGrad>
__device__ __forceinline__ void grad_raw_to_f32(const GradRaw<VEC, kGrad> &raw, float (&out)[VEC]) {
  if constexpr ((kGrad & kGradBf16) != 0) {
    uint16_t tmp[VEC];
    __builtin_memcpy(tmp, &raw, sizeof(raw));
#pragma unroll
    for (int i = 0; i < VEC; ++i) out[i] = TagBF16::to_f32(tmp[i]);
  } else {
    __builtin_memcpy(out, &raw, sizeof(raw));
  }
}

// arr[p / G] of lane p % G of the calling lane group (p the same on all of
// the group's lanes).
template <int N, int G>
__device__ __forceinline__ uint32_t group_pick(const uint32_t (&arr)[N], int p) {
  const int q = p / G;
  uint32_t v = arr[0];
#pragma unroll
  for (int i = 1; i < N; ++i) v = (q == i) ? arr[i] : v;
  return static_cast<uint32_t>(__shfl(static_cast<int>(v), p % G, G));
}

template <int N, int G>
__device__ __forceinline__ float group_pick(const float (&arr)[N], int p) {
  const int q = p / G;
  float v = arr[0];
#pragma unroll
  for (int i = 1; i < N; ++i) v = (q == i) ? arr[i] : v;
  return __shfl(v, p % G, G);
}

// Mask of positions 0 .. p (p < 64).
__device__ __forceinline__ uint64_t upto_mask(int p) { return p >= 63 ? ~0ull : ((2ull << p) - 1); }

// Gradient rows in flight per lane group in piece_sums_kernel.
template <int NC>
constexpr int piece_batch() { return NC == 1 ? 2 : 1; }

// Segment sums for the optimizer updates.  One lane group of G lanes per unit
// of kReduceUnit sorted positions streams the gradient rows of the unit's
// positions in order, piece_batch() rows in flight, skipping keys with a
// single occurrence (key_apply_kernel reads their one row itself).  Each
// piece (the positions of one key inside the unit) is summed from zero in
// position order, which is occurrence order since the sort is stable; at the
// piece's last position the sum goes to the key's row of a.sums when the key
// lies in the unit, else to the unit's partial slot (1: the key's first
// piece, 0: a later one) for the folds.  The group also writes the inverse
// (rank of the key) of every position of the unit.  No lane of the kernel
// branches on another group's keys except around the stores, so a wave's
// four groups stream their units together.
template <typename Tag, int VEC, int G, int NC, int MODE, int kGrad>
__global__ __launch_bounds__(256) void piece_sums_kernel(UpdateArgs a) {
  if (a.reject && *a.reject) return;
  constexpr int kGroups = 256 / G;
  constexpr int kPPL = kReduceUnit / G;  // sorted positions per lane
  constexpr int kBatch = piece_batch<NC>();
  const int lane = threadIdx.x % G;
  const int group = threadIdx.x / G;
  const int group_lane0 = (threadIdx.x & 63) - lane;
  const uint64_t group_mask = (G == 64) ? ~0ull : ((1ull << G) - 1);
  const uint32_t u = blockIdx.x * kGroups + group;
  const uint32_t nvalid = a.meta[0];
  const uint32_t j0 = u * kReduceUnit;
  const bool active = (u < a.units) && (j0 < nvalid);
  const uint32_t j1 = active ? min(j0 + kReduceUnit, nvalid) : j0;
  const int cnt = static_cast<int>(j1 - j0);
  const int D = a.dim;
  const bool ident = a.meta[kMetaGradIdent] != 0;

  uint32_t grow[kPPL];
  float scl[kPPL];
  uint64_t heads = 0;
#pragma unroll
  for (int q = 0; q < kPPL; ++q) {
    const int p = q * G + lane;
    bool head = false;
    grow[q] = 0;
    scl[q] = 1.0f;
    if (p < cnt) {
      const uint32_t j = j0 + p;
      head = (j == 0) || (a.sk[j] != a.sk[j - 1]);
      const bool need_occ = ident || !a.sorted_grad_row || (a.scale_mode != kScaleNone && !a.sorted_scale);
      uint32_t o = 0;
      if (need_occ) {
        o = a.sv[j];
        if (o >= a.n) {  // only if the sort was corrupted (tripped spin guard)
          record_error(a.err, kErrSpinGuard);
          o = 0;
        }
      }
      grow[q] = checked_grad_row(a, ident ? o : (a.sorted_grad_row ? a.sorted_grad_row[j] : grad_row_of(a, o)));
      if (a.scale_mode != kScaleNone) scl[q] = a.sorted_scale ? a.sorted_scale[j] : a.scale[o];
    }
    const uint64_t bal = __ballot(head);
    heads |= ((bal >> group_lane0) & group_mask) << (q * G);
  }
  if (!active) return;  // whole groups: no lane of an active group leaves
  const bool tail_head = j1 >= nvalid || (a.sk[j1] != a.sk[j1 - 1]);
  const uint32_t r0 = a.unit_first_run[u];
  const uint64_t valid = cnt >= 64 ? ~0ull : ((1ull << cnt) - 1);
  const uint64_t last_bit = 1ull << (cnt - 1);
  // bit p: the key of position p has no position after p in the unit
  const uint64_t ends = ((heads >> 1) | last_bit) & valid;
  // keys with one occurrence: a head whose key ends there and does not go on
  const uint64_t single = heads & ((heads >> 1) | (tail_head ? last_bit : 0ull)) & valid;
  uint64_t todo = valid & ~single;

  float acc[NC][VEC];
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[c][v] = 0.0f;
  while (todo) {
    int pos[kBatch];
    GradRaw<VEC, kGrad> x[kBatch][NC];
#pragma unroll
    for (int t = 0; t < kBatch; ++t) {
      pos[t] = todo ? __builtin_ctzll(todo) : -1;
      todo &= todo - 1;
      const bool ok = pos[t] >= 0;
      const int64_t gr = ok ? static_cast<int64_t>(group_pick<kPPL, G>(grow, pos[t])) : 0;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int col = (c * G + lane) * VEC;
        x[t][c] = (ok && col < D) ? load_grad_raw<VEC, kGrad>(a, gr * D + col) : GradRaw<VEC, kGrad>{};
      }
    }
#pragma unroll
    for (int t = 0; t < kBatch; ++t) {
      const int p = pos[t];
      if (p < 0) break;
      const bool head = (heads >> p) & 1ull;
      const float sc = group_pick<kPPL, G>(scl, p);
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        float xv[VEC];
        grad_raw_to_f32<VEC, kGrad>(x[t][c], xv);
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[c][v] = (head ? 0.0f : acc[c][v]) + scaled(a, xv[v], sc);
      }
      if ((ends >> p) & 1ull) {
        // the piece ends at p; it starts at the unit's first position or at a head
        const uint64_t before = heads & upto_mask(p);
        const int ps = before ? 63 - __builtin_clzll(before) : 0;
        const bool starts = (heads >> ps) & 1ull;
        const bool whole = starts && ((p + 1 < cnt) || tail_head);
        const uint32_t r = r0 + __popcll(heads & ~1ull & upto_mask(p));
        float *dst;
        if (whole) {
          dst = a.sums + static_cast<int64_t>(r) * D;
        } else {
          dst = a.partial + (static_cast<size_t>(u) * 2 + (starts ? 1 : 0)) * D;
          if (starts && lane == 0) {
            // head piece of a key that continues past this unit: hot when the
            // key still holds the position kInlineSpan + 1 units further on
            const uint32_t probe = (u + kInlineSpan + 1) * kReduceUnit;
            if (probe < nvalid && a.sk[probe] == a.sk[j0 + ps])
              a.hot_runs[atomicAdd(const_cast<uint32_t *>(a.meta) + 2, 1u)] = r;
          }
        }
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const int col = (c * G + lane) * VEC;
          if (col < D) store_f32<VEC>(dst + col, acc[c]);
        }
      }
    }
  }

  if (a.inverse_out) {
#pragma unroll
    for (int q = 0; q < kPPL; ++q) {
      const int pos = q * G + lane;
      if (pos < cnt) {
        const uint32_t o = a.sv[j0 + pos];
        if (o < a.n) {
          const uint32_t rr = r0 + __popcll(heads & upto_mask(pos) & ~1ull);
          a.inverse_out[o] = static_cast<int32_t>(a.run_rank[rr]);
        }
      }
    }
  }
}

// Run bounds, key and (single occurrence) gradient row and scale of run r.
struct KeyMeta {
  uint32_t start, end, key, grad_row;
  float scale;
};

__device__ __forceinline__ KeyMeta key_meta(const UpdateArgs &a, uint32_t r) {
  KeyMeta m;
  m.start = a.run_start[r];
  m.end = a.run_start[r + 1];
  m.key = a.run_key[r];
  m.grad_row = a.run_grad_row ? a.run_grad_row[r] : 0;
  m.scale = (a.scale_mode != kScaleNone && a.run_scale) ? a.run_scale[r] : 1.0f;
  return m;
}

// The optimizer update of every key but the hot ones (fold_kernel), after
// piece_sums_kernel: one key per lane group, looping, the next key's run
// bounds loaded while the current key is updated.  The gradient is the key's
// one row (a key with a single occurrence), its row of a.sums (a key inside
// one unit), or its unit partials folded left to right (the first unit's slot
// 1, then slot 0 of each following unit).  The table row (and Adagrad
// accumulator) is loaded together with the gradient.  Also clears the
// hot-key count that the folds read.
// Rows of one pass (NC == 1) ask for five waves per SIMD (at most 96 VGPRs;
// Adam's instantiation for 128-wide bf16 rows needs 97 otherwise: 640 against
// 645 us on 1.08M keys, a small gain), wider rows keep their own allocation
// (five would spill).
template <typename Tag, int VEC, int G, int NC, int MODE, int kGrad>
__global__ __launch_bounds__(256, NC == 1 ? 5 : 1) void key_apply_kernel(UpdateArgs a) {
  if (a.reject && *a.reject) return;
  constexpr int kGroups = 256 / G;
  const int lane = threadIdx.x % G;
  const int D = a.dim;
  const uint32_t runs = a.meta[1];
  const uint32_t stride = gridDim.x * kGroups;
  if (blockIdx.x == 0 && threadIdx.x == 0) const_cast<uint32_t *>(a.meta)[2] = 0;
  uint32_t r = blockIdx.x * kGroups + threadIdx.x / G;
  KeyMeta next{};
  if (r < runs) next = key_meta(a, r);
  for (; r < runs; r += stride) {
    const KeyMeta m = next;
    if (r + stride < runs) next = key_meta(a, r + stride);
    if (m.end <= m.start || m.end > a.n) continue;  // only after a tripped spin guard
    const uint32_t h = m.start / kReduceUnit;
    const uint32_t last = (m.end - 1) / kReduceUnit;
    if (last - h > kInlineSpan) continue;  // hot key: fold_kernel
    RowAhead<NC, VEC> ahead;
    load_ahead<Tag, VEC, G, NC, MODE>(a, r, m.key, ahead, lane);
    float g[NC][VEC];
    if (m.end - m.start == 1) {
      uint32_t o = 0;
      const bool need_occ = !a.run_grad_row || (a.scale_mode != kScaleNone && !a.run_scale && !a.sorted_scale);
      if (need_occ) {
        o = a.sv[m.start];
        if (o >= a.n) {
          record_error(a.err, kErrSpinGuard);
          o = 0;
        }
      }
      const int64_t gr = checked_grad_row(a, a.run_grad_row ? m.grad_row : grad_row_of(a, o));
      float sc = m.scale;
      if (a.scale_mode != kScaleNone && !a.run_scale) sc = a.sorted_scale ? a.sorted_scale[m.start] : a.scale[o];
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int col = (c * G + lane) * VEC;
        float xv[VEC];
        if (col < D) {
          grad_raw_to_f32<VEC, kGrad>(load_grad_raw<VEC, kGrad>(a, gr * D + col), xv);
        } else {
#pragma unroll
          for (int v = 0; v < VEC; ++v) xv[v] = 0.0f;
        }
        // the sum of one row, from zero as every key's
#pragma unroll
        for (int v = 0; v < VEC; ++v) g[c][v] = 0.0f + scaled(a, xv[v], sc);
      }
    } else {
      const float *first = (h == last) ? a.sums + static_cast<int64_t>(r) * D
                                       : a.partial + (static_cast<size_t>(h) * 2 + 1) * D;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int col = (c * G + lane) * VEC;
        if (col < D) {
          load_f32<VEC>(first + col, g[c]);
        } else {
#pragma unroll
          for (int v = 0; v < VEC; ++v) g[c][v] = 0.0f;
        }
      }
      // slot 0 of units h + 1 .. last (at most kInlineSpan), 16 floats a lane in flight
      constexpr int kIn = VEC * NC >= 8 ? 2 : 4;
      for (uint32_t x = h + 1; x <= last; x += kIn) {
        float y[kIn][NC][VEC];
#pragma unroll
        for (int t = 0; t < kIn; ++t)
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const int col = (c * G + lane) * VEC;
            if (x + t <= last && col < D) load_f32<VEC>(a.partial + (static_cast<size_t>(x + t) * 2) * D + col, y[t][c]);
          }
#pragma unroll
        for (int t = 0; t < kIn; ++t)
          if (x + t <= last) {
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
              for (int v = 0; v < VEC; ++v) g[c][v] += y[t][c][v];
          }
      }
    }
    apply_update<Tag, VEC, G, NC, MODE>(a, m.key, g, ahead, lane);
  }
}

// Unit partials of key r: piece 0 is the first unit's slot 1, piece p > 0 the
// slot 0 of unit h + p.
__device__ __forceinline__ float *piece_row(const UpdateArgs &a, uint32_t h, uint32_t p) {
  return a.partial + (static_cast<size_t>(h + p) * 2 + (p == 0 ? 1 : 0)) * a.dim;
}

// First level of the fold of keys with more than kFoldChunk pieces: one lane
// group per run of kFoldChunk pieces sums them left to right and writes the
// result over the run's first piece.  Work items: every unit (the run that
// starts there, for runs after a key's first) and every hot key (its first
// run).
template <int VEC, int G, int NC>
__global__ __launch_bounds__(256) void fold_chunks_kernel(UpdateArgs a) {
  if (a.reject && *a.reject) return;
  constexpr int kGroups = 256 / G;
  constexpr int kAhead = fold_rows(NC, VEC);
  const int lane = threadIdx.x % G;
  const int D = a.dim;
  const uint32_t nvalid = a.meta[0];
  const uint32_t hot = a.meta[2];
  const uint32_t items = a.units + hot;
  for (uint32_t w = blockIdx.x * kGroups + threadIdx.x / G; w < items; w += gridDim.x * kGroups) {
    uint32_t r, first;
    if (w < a.units) {
      if (w * kReduceUnit >= nvalid) continue;
      r = a.unit_first_run[w];
      if (a.run_start[r] >= w * kReduceUnit) continue;  // the unit's first key starts in it
      first = w - a.run_start[r] / kReduceUnit;
      if (first % kFoldChunk != 0) continue;
    } else {
      r = a.hot_runs[w - a.units];
      first = 0;
    }
    const uint32_t seg_start = a.run_start[r];
    const uint32_t seg_end = a.run_start[r + 1];
    if (seg_end <= seg_start || seg_end > a.n) continue;
    const uint32_t h = seg_start / kReduceUnit;
    const uint32_t count = (seg_end - 1) / kReduceUnit - h + 1;
    if (count <= kFoldChunk) continue;  // one level: fold_kernel
    const uint32_t m = min(kFoldChunk, count - first);
    float g[NC][VEC];
    const float *seed = piece_row(a, h, first);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int col = (c * G + lane) * VEC;
      if (col < D) load_f32<VEC>(seed + col, g[c]);
    }
    for (uint32_t k = 1; k < m; k += kAhead) {  // kAhead rows in flight, added in order
      float y[kAhead][NC][VEC];
#pragma unroll
      for (int t = 0; t < kAhead; ++t) {
        const bool ok = k + t < m;
        const float *src = piece_row(a, h, first + (ok ? k + t : 0));
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const int col = (c * G + lane) * VEC;
          if (ok && col < D) {
            load_f32<VEC>(src + col, y[t][c]);
          } else {
#pragma unroll
            for (int v = 0; v < VEC; ++v) y[t][c][v] = 0.0f;
          }
        }
      }
#pragma unroll
      for (int t = 0; t < kAhead; ++t) {
        if (k + t < m) {  // predicated, so the rows stay in registers
#pragma unroll
          for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int v = 0; v < VEC; ++v) g[c][v] += y[t][c][v];
        }
      }
    }
    float *dst = piece_row(a, h, first);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int col = (c * G + lane) * VEC;
      if (col < D) store_f32<VEC>(dst + col, g[c]);
    }
  }
}

// Hot keys: one block per key folds the key's unit partials in order.  Each
// round the block's lane groups load up to kFoldDepth partial rows each into LDS
// (all loads in flight together), then group 0 adds them left to right: the
// first unit's slot 1, then slot 0 of every following unit.  Group 0 then
// applies the update.
template <typename Tag, int VEC, int G, int NC, int MODE>
__global__ __launch_bounds__(256) void fold_kernel(UpdateArgs a, int depth) {
  if (a.reject && *a.reject) return;
  constexpr int kGroups = 256 / G;
  extern __shared__ float s_rows[];  // [kGroups * depth][dim]
  const int lane = threadIdx.x % G;
  const int group = threadIdx.x / G;
  const int D = a.dim;
  const uint32_t chunk = static_cast<uint32_t>(kGroups * depth);
  const uint32_t hot = a.meta[2];
  for (uint32_t i = blockIdx.x; i < hot; i += gridDim.x) {
    const uint32_t r = a.hot_runs[i];
    const uint32_t seg_start = a.run_start[r];
    const uint32_t seg_end = a.run_start[r + 1];
    const uint32_t key = a.run_key[r];
    if (seg_end <= seg_start || seg_end > a.n) continue;  // block-uniform
    const uint32_t h = seg_start / kReduceUnit;
    const uint32_t last = (seg_end - 1) / kReduceUnit;
    const uint32_t pieces = last - h + 1;
    // rows to fold, in order: the pieces, or the results of fold_chunks_kernel
    // (one per run of kFoldChunk pieces, over the run's first piece)
    const bool chunked = pieces > kFoldChunk;
    const uint32_t count = chunked ? (pieces + kFoldChunk - 1) / kFoldChunk : pieces;
    const uint32_t stride = chunked ? kFoldChunk : 1;
    RowAhead<NC, VEC> ahead;
    float g[NC][VEC];
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int v = 0; v < VEC; ++v) g[c][v] = 0.0f;
    if (group == 0) load_ahead<Tag, VEC, G, NC, MODE>(a, r, key, ahead, lane);
    for (uint32_t base = 0; base < count; base += chunk) {
      // all of this group's rows of the round in flight before any LDS store
      constexpr int kDepthMax = fold_rows(NC, VEC);  // the host's depth never exceeds it
      float y[kDepthMax][NC][VEC];
#pragma unroll
      for (int t = 0; t < kDepthMax; ++t) {
        const uint32_t k = base + group * depth + t;
        const bool ok = t < depth && k < count;
        const float *src = piece_row(a, h, ok ? k * stride : 0);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const int col = (c * G + lane) * VEC;
          if (ok && col < D) load_f32<VEC>(src + col, y[t][c]);
        }
      }
#pragma unroll
      for (int t = 0; t < kDepthMax; ++t) {
        const uint32_t k = base + group * depth + t;
        const bool ok = t < depth && k < count;
        float *dst = s_rows + static_cast<size_t>(group * depth + (ok ? t : 0)) * D;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const int col = (c * G + lane) * VEC;
          if (ok && col < D) store_f32<VEC>(dst + col, y[t][c]);
        }
      }
      __syncthreads();
      if (group == 0) {
        const uint32_t m = min(chunk, count - base);
        uint32_t k = 0;
        if (base == 0) {  // the first row seeds the sum
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const int col = (c * G + lane) * VEC;
            if (col < D) load_f32<VEC>(s_rows + col, g[c]);
          }
          k = 1;
        }
        for (; k + 8 <= m; k += 8) {  // eight LDS rows read ahead of the in-order adds
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const int col = (c * G + lane) * VEC;
            if (col < D) {
              float y[8][VEC];
#pragma unroll
              for (int t = 0; t < 8; ++t) load_f32<VEC>(s_rows + static_cast<size_t>(k + t) * D + col, y[t]);
#pragma unroll
              for (int t = 0; t < 8; ++t)
#pragma unroll
                for (int v = 0; v < VEC; ++v) g[c][v] += y[t][v];
            }
          }
        }
        for (; k < m; ++k) {
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const int col = (c * G + lane) * VEC;
            if (col < D) {
              float y[VEC];
              load_f32<VEC>(s_rows + static_cast<size_t>(k) * D + col, y);
#pragma unroll
              for (int v = 0; v < VEC; ++v) g[c][v] += y[v];
            }
          }
        }
      }
      __syncthreads();
    }
    if (group == 0) apply_update<Tag, VEC, G, NC, MODE>(a, key, g, ahead, lane);
  }
}

// ----------------------------------------------------------------------------
// host orchestration
// ----------------------------------------------------------------------------
struct Shape {
  int vec;
  int g;
  int nc;
};

// vec8_ok: 16-byte lanes of 8 elements (bfloat16 gradients): a row slice
// of 16 bytes per lane keeps twice the gradient rows in flight per lane
// group as 8-byte lanes, and random 256-byte rows read as 16 lanes x 16 bytes
// run at about 1.4 times the rate of 32 lanes x 8 bytes.
inline int choose_shape(int dim, bool vec4_ok, Shape *out, bool vec8_ok = false) {
  const int vec = (vec8_ok && dim % 8 == 0) ? 8 : (vec4_ok && dim % 4 == 0) ? 4 : 1;
  const int cols = dim / vec;
  if (cols <= 64) {
    int g = 8;
    while (g < cols) g <<= 1;
    *out = {vec, g, 1};
    return FLARE_OK;
  }
  int nc = 2;
  while (nc * 64 < cols) nc <<= 1;
  if (nc > 8) return fail(FLARE_ERR_LIMIT, "embedding dim %d exceeds the supported maximum (%d)", dim, vec * 512);
  *out = {vec, 64, nc};
  return FLARE_OK;
}



// Optional timing markers of the calling thread (flare_set_update_events):
// recorded on the update's stream before sums_kernel, after it, after the
// folds and after apply_kernel (null entries record nothing).
extern thread_local hipEvent_t t_update_events[4];
extern thread_local int t_update_event_count;

inline void mark_update(int i, hipStream_t s) {
  if (i < t_update_event_count && t_update_events[i]) (void)hipEventRecord(t_update_events[i], s);
}

template <typename Tag, int VEC, int MODE>
int launch_update_vec(const UpdateArgs &a, const Shape &sh, hipStream_t s) {
  auto grid = [&](int g) { return static_cast<int>(std::max<int64_t>(1, ceil_div(a.units, 256 / g))); };
  // apply: the key count is only known on the device, so the grid covers n
  // keys, one per lane group, up to kApplyGroups groups (more keys loop; idle
  // groups exit at once)
  auto apply_grid = [&](int g) {
    return static_cast<int>(std::max<int64_t>(1, ceil_div(std::min<int64_t>(a.n, kApplyGroups), 256 / g)));
  };
  // fold: partial rows staged per round, at most 64 KiB of LDS (128 rows of
  // 128 floats: most hot keys fold in one or two rounds)
  auto fold_depth = [&](int g, int vec, int nc) {
    const int groups = 256 / g;
    int depth = fold_rows(nc, vec);
    while (depth > 1 && static_cast<int64_t>(groups) * depth * a.dim * 4 > 65536) depth >>= 1;
    return depth;
  };
  auto fold_lds = [&](int g, int vec, int nc) {
    return static_cast<size_t>(256 / g) * fold_depth(g, vec, nc) * a.dim * 4;
  };
  const int fold_grid = static_cast<int>(std::min<int64_t>(1024, std::max<int64_t>(1, ceil_div(a.units, kInlineSpan + 1))));
  // fold_chunks: one work item per unit plus one per hot key (at most one per
  // kInlineSpan + 1 units); the grid strides over them
  auto chunk_grid = [&](int g) {
    const int64_t items = static_cast<int64_t>(a.units) + a.units / (kInlineSpan + 1) + 1;
    return static_cast<int>(std::min<int64_t>(16384, std::max<int64_t>(1, ceil_div(items, 256 / g))));
  };
  // gradient rows streamed when each is read about once (see load_grad); only
  // 4-wide vectors have streamed loads, so narrower shapes keep two variants
  const int gm = (a.grad_bf16 ? kGradBf16 : 0) | (a.grad_rows > 0 && a.n <= a.grad_rows ? kGradStream : 0);
#define FLARE_GRAD_LAUNCH_X(KERNEL, G_, NC_, GRID, ARGS)                                         \
  if constexpr (VEC == 8) {                                                                     \
    if (gm & kGradStream) KERNEL<Tag, VEC, G_, NC_, MODE, kGradBf16 | kGradStream><<<GRID, 256, 0, s>>> ARGS; \
    else KERNEL<Tag, VEC, G_, NC_, MODE, kGradBf16><<<GRID, 256, 0, s>>> ARGS;                  \
  } else if constexpr (VEC == 4) {                                                              \
    switch (gm) {                                                                               \
      case 0: KERNEL<Tag, VEC, G_, NC_, MODE, 0><<<GRID, 256, 0, s>>> ARGS; break;              \
      case kGradBf16: KERNEL<Tag, VEC, G_, NC_, MODE, kGradBf16><<<GRID, 256, 0, s>>> ARGS; break; \
      case kGradStream: KERNEL<Tag, VEC, G_, NC_, MODE, kGradStream><<<GRID, 256, 0, s>>> ARGS; break; \
      default: KERNEL<Tag, VEC, G_, NC_, MODE, kGradBf16 | kGradStream><<<GRID, 256, 0, s>>> ARGS; break; \
    }                                                                                           \
  } else if (gm & kGradBf16) {                                                                  \
    KERNEL<Tag, VEC, G_, NC_, MODE, kGradBf16><<<GRID, 256, 0, s>>> ARGS;                       \
  } else {                                                                                      \
    KERNEL<Tag, VEC, G_, NC_, MODE, 0><<<GRID, 256, 0, s>>> ARGS;                               \
  }
#define FLARE_GRAD_LAUNCH(KERNEL, G_, NC_, GRID) FLARE_GRAD_LAUNCH_X(KERNEL, G_, NC_, GRID, (a))
// The folds of hot keys read and add float32 partial rows only: with 8-float
// lanes of one chunk they run on twice the lanes of 4 floats each (LDS reads
// of 16 bytes per lane and twice the lanes adding; 33 -> 22 us on 13K hot
// units of 128 floats).
#define FLARE_FOLDS(G_, NC_)                                                                 \
  {                                                                                          \
    constexpr bool kNarrow = VEC == 8 && NC_ == 1 && G_ <= 32;                               \
    constexpr int kFV = kNarrow ? 4 : VEC;                                                   \
    constexpr int kFG = kNarrow ? 2 * G_ : G_;                                               \
    fold_chunks_kernel<kFV, kFG, NC_><<<chunk_grid(kFG), 256, 0, s>>>(a);                    \
    fold_kernel<Tag, kFV, kFG, NC_, MODE><<<fold_grid, 256, fold_lds(kFG, kFV, NC_), s>>>(a, fold_depth(kFG, kFV, NC_)); \
  }
// keyed sums (scatter, reduced gradients): sums_kernel for long keys, apply_kernel for the rest
#define FLARE_UPDATE_PAIR(G_, NC_)                                                          \
  mark_update(0, s);                                                                        \
  FLARE_GRAD_LAUNCH(sums_kernel, G_, NC_, grid(G_))                                         \
  mark_update(1, s);                                                                        \
  FLARE_FOLDS(G_, NC_)                                                                      \
  mark_update(2, s);                                                                        \
  FLARE_GRAD_LAUNCH(apply_kernel, G_, NC_, apply_grid(G_))                                  \
  mark_update(3, s);
// optimizer updates: per-piece sums, the folds of hot keys, then one key per lane group
#define FLARE_UPDATE_UNITS(G_, NC_)                                                         \
  mark_update(0, s);                                                                        \
  FLARE_GRAD_LAUNCH(piece_sums_kernel, G_, NC_, grid(G_))                                   \
  mark_update(1, s);                                                                        \
  FLARE_FOLDS(G_, NC_)                                                                      \
  mark_update(2, s);                                                                        \
  FLARE_GRAD_LAUNCH(key_apply_kernel, G_, NC_, apply_grid(G_))                              \
  mark_update(3, s);
#define FLARE_SHAPES(SEQ)                                                                   \
  if (sh.nc == 1) {                                                                         \
    switch (sh.g) {                                                                         \
      case 8: SEQ(8, 1) break;                                                              \
      case 16: SEQ(16, 1) break;                                                            \
      case 32: SEQ(32, 1) break;                                                            \
      default: SEQ(64, 1) break;                                                            \
    }                                                                                       \
  } else {                                                                                  \
    switch (sh.nc) {                                                                        \
      case 2: SEQ(64, 2) break;                                                             \
      case 4: SEQ(64, 4) break;                                                             \
      default: SEQ(64, 8) break;                                                            \
    }                                                                                       \
  }
  if constexpr (MODE == kModeRows || MODE == kModeUnique) {
    FLARE_SHAPES(FLARE_UPDATE_PAIR)
  } else {
    FLARE_SHAPES(FLARE_UPDATE_UNITS)
  }
#undef FLARE_SHAPES
#undef FLARE_FOLDS
#undef FLARE_UPDATE_UNITS
#undef FLARE_UPDATE_PAIR
#undef FLARE_GRAD_LAUNCH
#undef FLARE_GRAD_LAUNCH_X
  FLARE_TRY_HIP(hipGetLastError());
  return FLARE_OK;
}

template <typename Tag, int MODE>
int launch_update_tag(const UpdateArgs &a, const Shape &sh, hipStream_t s) {
  if (sh.vec == 8) return launch_update_vec<Tag, 8, MODE>(a, sh, s);
  if (sh.vec == 4) return launch_update_vec<Tag, 4, MODE>(a, sh, s);
  return launch_update_vec<Tag, 1, MODE>(a, sh, s);
}

// One per translation unit: mode kModeRows / kModeUnique (float32 outputs),
// or an optimizer mode over a table of the unit's value dtype.
int launch_update_rows(int mode, const UpdateArgs &a, const Shape &sh, hipStream_t s);
int launch_update_f32(int mode, const UpdateArgs &a, const Shape &sh, hipStream_t s);
int launch_update_f16(int mode, const UpdateArgs &a, const Shape &sh, hipStream_t s);
int launch_update_bf16(int mode, const UpdateArgs &a, const Shape &sh, hipStream_t s);

}  // namespace flare
