// Internal interface of the sort-based dedup / segment-reduce engine.
#pragma once

#include "common.hpp"

namespace flare {

// Scan-type passes over sorted keys and occurrences (head counts, runs, first
// counts, ranks): 4096-position tiles of 1024 threads x 4 positions, so that
// a call of a few thousand tiles keeps 16 waves of each CU busy.
constexpr int kSortThreads = 1024;
constexpr int kSortItems = 4;
constexpr int kSortTile = kSortThreads * kSortItems;  // 4096 occurrences per tile
// Radix passes use larger tiles: 1024 threads x 8 keys (one tile per CU).
constexpr int kOneThreads = 1024;
constexpr int kOneItems = 8;
constexpr int kOneTile = kOneThreads * kOneItems;
// Digits of 8, 9 or 10 bits (chosen per call from the key width, so that
// 25-27-bit rows sort in 3 passes instead of 4); 64-bit keys use 8.
constexpr int kMaxDigitBits = 10;
constexpr int kMaxRadix = 1 << kMaxDigitBits;
// LDS histogram bins of the prepare kernels: passes x 2^digit bits.
constexpr int kMaxHistBins = 3 * kMaxRadix;
// Sorted positions are reduced in units of kReduceUnit consecutive positions;
// a key's occurrences inside one unit are summed sequentially and the unit
// partials of a key that spans several units are folded left to right.
constexpr int kReduceUnit = 64;
constexpr int64_t kMaxOccurrences = (int64_t{1} << 30) - 1;
// Blocks add their digit histograms into one of kHistCopies copies (by block
// index) to spread same-address atomics; a radix pass sums the copies.
constexpr int kHistCopies = 16;
constexpr int kMaxPasses = 8;
constexpr uint32_t kNoRun = 0xffffffffu;

// Where every array of one call lives inside the caller's workspace.
struct Workspace {
  // zero-initialized region (first)
  uint32_t *hist;         // [kHistCopies][kMaxPasses][kMaxRadix] digit histograms
  uint32_t *tickets;      // [16] tile tickets (8 sort passes, runs, rank)
  uint32_t *meta;         // [8]: nvalid, unique count, hot-key count, rejected batch, non-finite gradient,
                          //      (unused), occurrences are their own gradient rows
  uint32_t *sort_status;  // [passes][sort_tiles][2^digit bits] (last in the zeroed region)
  uint32_t *scan_status;  // [2][tiles]
  uint8_t *head_flag;     // [tiles * kSortTile] 1 at o: occurrence o is its key's first (else 0)
  size_t zero_bytes;      // whole zeroed region (sort status sized for the widest plan)
  size_t sort_status_offset;
  // not initialized
  void *keys[2];
  uint32_t *vals[2];
  uint32_t *grad_row;     // [n] (CSR gradient row of each occurrence)
  float *aux;             // [n] (mean-pooling divisor of each occurrence)
  uint32_t *sorted_grad_row;  // [n] grad_row of the occurrence at each sorted position
  float *sorted_scale;        // [n] aux of the occurrence at each sorted position
  uint32_t *run_grad_row;     // [n] sorted_grad_row at each key's first position
  float *run_scale;           // [n] sorted_scale at each key's first position
  uint2 *head_run;        // [n] {run, low 32 key bits} of each first occurrence (where head_flag is set)
  uint32_t *run_start;    // [n + 1]
  uint32_t *run_rank;     // [n]
  uint32_t *run_key;      // [n] key of each run (32-bit sorts)
  uint32_t *unit_first_run;  // [units]
  uint32_t *hot_runs;     // [units] keys whose partials apply_kernel does not fold
  float *partial;         // [units][2][dim]
  float *sums;            // [n][dim] per-key gradient sums (optimizer modes)
  size_t total_bytes;
  int64_t n;
  uint32_t tiles;       // kSortTile tiles (scans)
  uint32_t sort_tiles;  // kOneTile tiles (radix passes)
  uint32_t units;
  int key_bytes;
};

// Radix sort shape for keys of `bits` significant bits.
struct RadixPlan {
  int digit_bits;
  int passes;
};
RadixPlan radix_plan(int bits, int key_bytes);

// Bytes to clear before a call whose sort follows `plan`.
size_t zero_bytes_for(const Workspace &w, const RadixPlan &plan);

// Computes the layout; with base == nullptr only sizes are filled in.
Workspace layout_workspace(void *base, int64_t n, int key_bytes, int dim, bool need_grad_row,
                           bool need_aux, bool need_partials, bool need_sums = false);

int bits_for(uint64_t max_value);

}  // namespace flare
