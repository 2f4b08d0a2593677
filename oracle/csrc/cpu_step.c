/*
 * CPU restatement of the reference's sparse-embedding CPU path, timed as the
 * baseline beside the GPU.  TEST INFRASTRUCTURE ONLY: nothing in the product
 * links this file; bench.py's cpu_baseline leg and tests load it.
 *
 * Decomposition follows the reference's Numba kernels:
 *   pooled gather   bag-parallel, fp32 accumulation in occurrence order
 *                   (src/flare/ops/sparse_gather.py:39-63,100-123)
 *   dedup           serial first-occurrence open addressing, Fibonacci
 *                   multiplier 11400714819323198485, capacity = smallest
 *                   power of two with 2*cap >= 3*n, linear probing
 *                   (src/flare/ops/sparse_unique.py:16-48); independent
 *                   tables run concurrently, as InputSPMD runs sparse groups
 *                   (src/flare/runtime/fluxway/workers/sparse_input.py:280-282)
 *   keyed scatter   per table, slot order, into a private [U, D] fp32
 *                   accumulator (src/flare/ops/sparse_scatter.py:59-96)
 *   optimizer       row-parallel row-wise Adagrad / Adam
 *                   (tools/validation/audit_sparse_training.py:460-471)
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

enum { ST_F32 = 0, ST_F16 = 1, ST_BF16 = 2 };
enum { POOL_SUM = 0, POOL_MEAN = 1, POOL_WEIGHTED = 2 };
enum { OPT_NONE = 0, OPT_SGD = 1, OPT_ADAM = 2, OPT_ADAGRAD = 3 };

/* ---- storage conversions (IEEE-754 definitions, round to nearest even) ---- */
static inline float bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static inline uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
static inline float f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1fu, man = h & 0x3ffu, u;
  if (exp == 0) {
    if (man == 0) {
      u = sign;
    } else { /* subnormal: normalize */
      int e = -1;
      do { man <<= 1; ++e; } while (!(man & 0x400u));
      u = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
    }
  } else if (exp == 31) {
    u = sign | 0x7f800000u | (man << 13);
  } else {
    u = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static inline uint16_t f32_to_f16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520 -> inf */
  if (a < 0x38800000u) { /* subnormal or zero in fp16 */
    if (a < 0x33000000u) return (uint16_t)sign;             /* < 2^-25 rounds to 0 */
    uint32_t man = (a & 0x7fffffu) | 0x800000u;
    int shift = 126 - (int)(a >> 23); /* 14..24 */
    uint32_t half = 1u << (shift - 1), rem = man & ((1u << shift) - 1), q = man >> shift;
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
  }
  uint32_t r = a + 0xfffu + ((a >> 13) & 1u) - 0x38000000u;
  return (uint16_t)(sign | (r >> 13));
}

static inline float load_st(const void *t, int st, int64_t i) {
  if (st == ST_F32) return ((const float *)t)[i];
  if (st == ST_F16) return f16_to_f32(((const uint16_t *)t)[i]);
  return bf16_to_f32(((const uint16_t *)t)[i]);
}
static inline void store_st(void *t, int st, int64_t i, float v) {
  if (st == ST_F32) ((float *)t)[i] = v;
  else if (st == ST_F16) ((uint16_t *)t)[i] = f32_to_f16(v);
  else ((uint16_t *)t)[i] = f32_to_bf16(v);
}

int cpu_threads(void) { return omp_get_max_threads(); }
void cpu_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }

/* Deterministic U(lo, hi) init (splitmix64 per element), parallel. */
void cpu_init_table(void *table, int st, int64_t count, float lo, float hi, uint64_t seed) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < count; ++i) {
    uint64_t z = seed + 0x9e3779b97f4a7c15ull * (uint64_t)(i + 1);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    z ^= z >> 31;
    float u = (float)((z >> 40) * (1.0 / 16777216.0));
    store_st(table, st, i, lo + (hi - lo) * u);
  }
}

/* Pooled gather over CSR bags, table-major (bag k = t*B + b), out [B, T, D]. */
void cpu_pooled_forward(const void *table, int st, int32_t dim, const int64_t *ids,
                        const int64_t *offsets, int32_t num_tables, int64_t batch,
                        const int64_t *row_base, int32_t pooling, const float *weights, void *out) {
  const int64_t bags = (int64_t)num_tables * batch;
#pragma omp parallel
  {
    float *acc = (float *)malloc(sizeof(float) * (size_t)dim);
#pragma omp for schedule(dynamic, 256)
    for (int64_t k = 0; k < bags; ++k) {
      const int64_t t = k / batch, b = k - t * batch;
      for (int d = 0; d < dim; ++d) acc[d] = 0.0f;
      int64_t count = 0;
      for (int64_t i = offsets[k]; i < offsets[k + 1]; ++i) {
        const int64_t row = row_base[t] + ids[i];
        const float w = pooling == POOL_WEIGHTED ? weights[i] : 1.0f;
        for (int d = 0; d < dim; ++d) {
          const float x = load_st(table, st, row * dim + d);
          acc[d] += pooling == POOL_WEIGHTED ? w * x : x;
        }
        ++count;
      }
      const int64_t o = (b * num_tables + t) * dim;
      const float div = (float)(count > 0 ? count : 1);
      for (int d = 0; d < dim; ++d) store_st(out, st, o + d, pooling == POOL_MEAN ? acc[d] / div : acc[d]);
    }
    free(acc);
  }
}

/* Serial first-occurrence dedup of keys[0..n) (sparse_unique.py:24-48). */
static int64_t dedup_first_occurrence(const int64_t *keys, int64_t n, int64_t *unique_out,
                                      int32_t *inverse_out, int64_t *first_out) {
  if (n == 0) return 0;
  uint64_t cap = 1;
  while (cap * 2 < (uint64_t)n * 3) cap <<= 1;
  const uint64_t mask = cap - 1;
  int64_t *slot_key = (int64_t *)malloc(sizeof(int64_t) * cap);
  int32_t *slot_id = (int32_t *)malloc(sizeof(int32_t) * cap);
  uint8_t *occupied = (uint8_t *)calloc(cap, 1);
  int64_t u = 0;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t key = keys[i];
    uint64_t s = ((uint64_t)key * 11400714819323198485ull) & mask;
    while (occupied[s] && slot_key[s] != key) s = (s + 1) & mask;
    if (!occupied[s]) {
      occupied[s] = 1;
      slot_key[s] = key;
      slot_id[s] = (int32_t)u;
      unique_out[u] = key;
      first_out[u] = i;
      inverse_out[i] = (int32_t)u;
      ++u;
    } else {
      inverse_out[i] = slot_id[s];
    }
  }
  free(slot_key);
  free(slot_id);
  free(occupied);
  return u;
}

/*
 * Backward + update of one batch: per table (concurrently) dedup of the
 * table's occurrences, keyed gradient sums in slot order, then the optimizer
 * on every unique row.  opt: OPT_ADAGAD (state0 = acc [rows]), OPT_ADAM
 * (state0 = m, state1 = v [rows, D], step [rows]), OPT_SGD, or OPT_NONE
 * (reduced gradients written to grad_out in first-occurrence order per table,
 * tables concatenated).  Returns the total unique count.
 */
int64_t cpu_pooled_backward(void *table, int st, int32_t dim, float *state0, float *state1,
                            int32_t *step, int32_t opt, double lr, double beta1, double beta2,
                            double eps, const int64_t *ids, const int64_t *offsets,
                            int32_t num_tables, int64_t batch, const int64_t *row_base,
                            int32_t pooling, const float *weights, const float *pooled_grad,
                            float *grad_out, int64_t *unique_out, int32_t *inverse_out) {
  int64_t *table_unique = (int64_t *)calloc((size_t)num_tables + 1, sizeof(int64_t));
  const int64_t n_total = offsets[(int64_t)num_tables * batch];
  int64_t *first = (int64_t *)malloc(sizeof(int64_t) * (size_t)(n_total > 0 ? n_total : 1));
#pragma omp parallel for schedule(dynamic, 1)
  for (int32_t t = 0; t < num_tables; ++t) {
    const int64_t lo = offsets[(int64_t)t * batch], hi = offsets[(int64_t)(t + 1) * batch];
    const int64_t n = hi - lo;
    int64_t *keys = (int64_t *)malloc(sizeof(int64_t) * (size_t)(n > 0 ? n : 1));
    for (int64_t i = 0; i < n; ++i) keys[i] = ids[lo + i];
    const int64_t u = dedup_first_occurrence(keys, n, unique_out + lo, inverse_out + lo, first + lo);
    table_unique[t] = u;
    float *acc = (float *)calloc((size_t)(u > 0 ? u : 1) * (size_t)dim, sizeof(float));
    int64_t k = (int64_t)t * batch; /* bag of occurrence lo + i */
    for (int64_t i = 0; i < n; ++i) {
      while (offsets[k + 1] <= lo + i) ++k;
      const int64_t b = k - (int64_t)t * batch;
      const float *g = pooled_grad + (b * num_tables + t) * dim;
      float *a = acc + (int64_t)inverse_out[lo + i] * dim;
      if (pooling == POOL_WEIGHTED) {
        const float w = weights[lo + i];
        for (int d = 0; d < dim; ++d) a[d] += g[d] * w;
      } else if (pooling == POOL_MEAN) {
        const float len = (float)(offsets[k + 1] - offsets[k]);
        for (int d = 0; d < dim; ++d) a[d] += g[d] / len;
      } else {
        for (int d = 0; d < dim; ++d) a[d] += g[d];
      }
    }
    for (int64_t j = 0; j < u; ++j) {
      const int64_t row = row_base[t] + unique_out[lo + j];
      float *g = acc + j * dim;
      if (opt == OPT_NONE) {
        memcpy(grad_out + (lo + j) * dim, g, sizeof(float) * (size_t)dim);
      } else if (opt == OPT_SGD) {
        for (int d = 0; d < dim; ++d)
          store_st(table, st, row * dim + d, load_st(table, st, row * dim + d) - (float)lr * g[d]);
      } else if (opt == OPT_ADAGRAD) {
        double ss = 0.0;
        for (int d = 0; d < dim; ++d) ss += (double)g[d] * (double)g[d];
        const float a = (float)((double)state0[row] + ss / (double)dim);
        state0[row] = a;
        const float den = sqrtf(a) + (float)eps;
        for (int d = 0; d < dim; ++d)
          store_st(table, st, row * dim + d, load_st(table, st, row * dim + d) - ((float)lr * g[d]) / den);
      } else {
        const int32_t s = step[row] + 1;
        step[row] = s;
        const float bc1 = (float)(1.0 - pow(beta1, (double)s)), bc2 = (float)(1.0 - pow(beta2, (double)s));
        for (int d = 0; d < dim; ++d) {
          float *m = state0 + row * dim + d, *v = state1 + row * dim + d;
          *m = (float)beta1 * *m + (float)(1.0 - beta1) * g[d];
          *v = (float)beta2 * *v + (float)(1.0 - beta2) * (g[d] * g[d]);
          const float w = load_st(table, st, row * dim + d) - ((float)lr * (*m / bc1)) / (sqrtf(*v / bc2) + (float)eps);
          store_st(table, st, row * dim + d, w);
        }
      }
    }
    free(acc);
    free(keys);
  }
  int64_t total = 0;
  for (int32_t t = 0; t < num_tables; ++t) total += table_unique[t];
  free(table_unique);
  free(first);
  return total;
}

double cpu_now(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}
