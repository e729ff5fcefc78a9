/*
 * CPU oracle for exact top-k inner-product search.  TEST INFRASTRUCTURE ONLY:
 * it is the checker that the HIP path is compared against (tests/, the smoke
 * test in __graft_entry__.py and the cpu_baseline leg of bench.py).  Nothing in
 * the shipped package links, loads or calls it.
 *
 * What it restates:
 *   - cuda_vector_search/reference.py:18-34 (exact_topk_fp32): the ground truth
 *     is the top-k of the fp32 scores q . x over the *stored* fp16 values.  Here
 *     every score is the exactly-accumulated (double) dot product of the fp16
 *     values, rounded once to fp32.  Any fp32 summation order (BLAS, MFMA)
 *     differs from it by at most its own rounding error.
 *   - the output order of kernels.cu:277-279 (ranks_before) and the merge at
 *     kernels.cu:373-445: score descending, ties broken by the smaller id.
 *   - kernels.cu:472-497 (scores): the full [nq, n] fp32 score matrix.
 *
 * fp16 decoding is done bit-exactly in integer arithmetic (IEEE 754 binary16
 * -> binary32 is exact), so the oracle needs no compiler _Float16 support.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* IEEE 754 binary16 -> binary32, exact for every one of the 65536 inputs. */
float cvs_oracle_half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign; /* +-0 */
    } else {       /* subnormal: normalise into a binary32 normal */
      int e = -1;
      do {
        man <<= 1;
        ++e;
      } while ((man & 0x400u) == 0);
      man &= 0x3ffu;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13); /* inf / nan (payload kept) */
  } else {
    bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, sizeof f);
  return f;
}

/* 65536-entry decode table, filled once (idempotent, so a benign race). */
static float g_lut[65536];
static volatile int g_lut_ready = 0;

static void lut_init(void) {
  if (g_lut_ready) return;
  for (uint32_t h = 0; h < 65536u; ++h) g_lut[h] = cvs_oracle_half_to_float((uint16_t)h);
  __sync_synchronize();
  g_lut_ready = 1;
}

/* True when (va, ia) ranks strictly before (vb, ib): score desc, then id asc. */
static int ranks_before(float va, int64_t ia, float vb, int64_t ib) {
  return va > vb || (va == vb && ia < ib);
}

/* Bounded min-heap of the k best seen so far; heap[0] is the worst kept. */
typedef struct {
  float* v;
  int64_t* id;
  int64_t size, cap;
} heap_t;

static void heap_swap(heap_t* h, int64_t a, int64_t b) {
  float tv = h->v[a];
  int64_t ti = h->id[a];
  h->v[a] = h->v[b];
  h->id[a] = h->id[b];
  h->v[b] = tv;
  h->id[b] = ti;
}

static void heap_sift_down(heap_t* h, int64_t i) {
  for (;;) {
    int64_t l = 2 * i + 1, r = l + 1, w = i;
    if (l < h->size && ranks_before(h->v[w], h->id[w], h->v[l], h->id[l])) w = l;
    if (r < h->size && ranks_before(h->v[w], h->id[w], h->v[r], h->id[r])) w = r;
    if (w == i) return;
    heap_swap(h, i, w);
    i = w;
  }
}

static void heap_sift_up(heap_t* h, int64_t i) {
  while (i > 0) {
    int64_t p = (i - 1) / 2;
    if (!ranks_before(h->v[p], h->id[p], h->v[i], h->id[i])) return;
    heap_swap(h, i, p);
    i = p;
  }
}

static void heap_offer(heap_t* h, float v, int64_t id) {
  if (h->size < h->cap) {
    h->v[h->size] = v;
    h->id[h->size] = id;
    heap_sift_up(h, h->size++);
  } else if (ranks_before(v, id, h->v[0], h->id[0])) {
    h->v[0] = v;
    h->id[0] = id;
    heap_sift_down(h, 0);
  }
}

/* Exact dot product of two fp16 rows, accumulated in double, rounded once. */
static float dot_exact(const uint16_t* a, const uint16_t* b, int64_t d) {
  double s = 0.0;
  for (int64_t j = 0; j < d; ++j) s += (double)g_lut[a[j]] * (double)g_lut[b[j]];
  return (float)s;
}

typedef struct {
  float v;
  int64_t id;
} entry_t;

static int entry_cmp(const void* pa, const void* pb) {
  const entry_t* a = (const entry_t*)pa;
  const entry_t* b = (const entry_t*)pb;
  if (ranks_before(a->v, a->id, b->v, b->id)) return -1;
  if (ranks_before(b->v, b->id, a->v, a->id)) return 1;
  return 0;
}

/*
 * Exact top-k.  q: [nq, d] fp16 bits, x: [n, d] fp16 bits (row-major).
 * out_v: [nq, k] fp32, out_i: [nq, k] int64, sorted by (score desc, id asc).
 * Rows are split into ranges; each range keeps its own top-k heap and the
 * per-range winners are merged by a full sort (the union of the per-range
 * top-k always contains the global top-k).  Requires 1 <= k <= n.
 * Returns 0 on success, -1 on bad arguments / memory.
 */
int cvs_oracle_topk(const uint16_t* q, const uint16_t* x, int64_t nq, int64_t n, int64_t d,
                    int64_t k, float* out_v, int64_t* out_i, int nthreads) {
  if (nq < 0 || n < 1 || d < 1 || k < 1 || k > n) return -1;
  if (nq == 0) return 0;
  lut_init();
  int nt = nthreads > 0 ? nthreads : 1;
  int64_t ranges = (4 * (int64_t)nt + nq - 1) / nq;
  if (ranges > n / (k > 64 ? k : 64)) ranges = n / (k > 64 ? k : 64);
  if (ranges < 1) ranges = 1;
  const int64_t tasks = nq * ranges;
  entry_t* part = (entry_t*)malloc(sizeof(entry_t) * (size_t)(tasks * k));
  int64_t* pcount = (int64_t*)calloc((size_t)tasks, sizeof(int64_t));
  if (!part || !pcount) {
    free(part);
    free(pcount);
    return -1;
  }
  int err = 0;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
  for (int64_t t = 0; t < tasks; ++t) {
    const int64_t i = t / ranges, r = t % ranges;
    const int64_t lo = n * r / ranges, hi = n * (r + 1) / ranges;
    heap_t h;
    h.v = (float*)malloc(sizeof(float) * (size_t)k);
    h.id = (int64_t*)malloc(sizeof(int64_t) * (size_t)k);
    h.size = 0;
    h.cap = k;
    if (!h.v || !h.id) {
      free(h.v);
      free(h.id);
#pragma omp atomic write
      err = 1;
      continue;
    }
    const uint16_t* qi = q + i * d;
    for (int64_t row = lo; row < hi; ++row) heap_offer(&h, dot_exact(qi, x + row * d, d), row);
    for (int64_t j = 0; j < h.size; ++j) {
      part[t * k + j].v = h.v[j];
      part[t * k + j].id = h.id[j];
    }
    pcount[t] = h.size;
    free(h.v);
    free(h.id);
  }
  if (!err) {
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
    for (int64_t i = 0; i < nq; ++i) {
      /* compact this query's per-range winners to the front, then sort */
      entry_t* base = part + i * ranges * k;
      int64_t m = 0;
      for (int64_t r = 0; r < ranges; ++r)
        for (int64_t j = 0; j < pcount[i * ranges + r]; ++j) base[m++] = base[r * k + j];
      qsort(base, (size_t)m, sizeof(entry_t), entry_cmp);
      for (int64_t j = 0; j < k; ++j) {
        out_v[i * k + j] = base[j].v;
        out_i[i * k + j] = base[j].id;
      }
    }
  }
  free(part);
  free(pcount);
  return err ? -1 : 0;
}

/* Full score matrix out[i, r] = fp32(exact q_i . x_r).  Same contract as kernels.cu:472-497. */
int cvs_oracle_scores(const uint16_t* q, const uint16_t* x, int64_t nq, int64_t n, int64_t d,
                      float* out, int nthreads) {
  if (nq < 0 || n < 0 || d < 1) return -1;
  lut_init();
  const int64_t blk = 4096;
  const int64_t nblk = (n + blk - 1) / blk;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads > 0 ? nthreads : 1)
  for (int64_t t = 0; t < nq * nblk; ++t) {
    const int64_t i = t / nblk, lo = (t % nblk) * blk;
    const int64_t hi = lo + blk < n ? lo + blk : n;
    for (int64_t r = lo; r < hi; ++r) out[i * n + r] = dot_exact(q + i * d, x + r * d, d);
  }
  return 0;
}
