// Exact top-k selection over candidate lists, one 256-thread workgroup per query.
//
// Replaces the merge of csrc/kernels.cu:373-445.  The reference merges exactly
// k candidates per chunk with one warp and k serial arg-max rounds; here each
// query's candidates (any number per list) are streamed into an LDS buffer in
// batches, filtered against the running k-th best key, and the buffer is cut
// down to its k best keys with a radix select (8-bit digits of the 64-bit key,
// most significant first, per-wave LDS histograms, early exit once the k-th
// key's digit bin is exhausted) followed by one compaction pass.  Only the
// final k survivors are sorted.  Keys order by (score desc, id asc) and are
// unique, so the k largest keys are exactly the top-k and the output is sorted
// like the reference's.
//
// Threshold mode returns only the score of the k-th best key (used to turn the
// sampling pre-pass's unit maxima into per-query thresholds).  With one list
// per query holding a whole score row it is also the row top-k of a score
// matrix (k up to 1024: the large-k path).
//
// Rescore mode finishes the int8 pre-filter: list entries are (score upper
// bound, row id) pairs whose bound reached the threshold, and exact scores are
// recomputed here from the fp16 rows (fp32 accumulation, v_dot2_f32_f16), first
// for the k candidates of largest bound and then only for the others whose
// bound reaches the k-th best exact score found so far.  A list that
// overflowed in the scan (count > cap) is replaced by every row of its corpus
// range, so the result stays exact whatever the data.
#include "cvs_common.h"
#include "cvs_kernels.h"
#include "cvs_q8_row.h"

namespace cvs {

namespace {

constexpr int kBuf = 4096;    // LDS key buffer
constexpr int kBatch = 2048;  // candidates gathered per round
constexpr int kWaves = kBlock / kWave;
constexpr int kGather = kBatch / kBlock;  // entries per thread per round

template <int MAXL>
struct SelSharedT {
  uint64_t keys[kBuf];
  int pre[MAXL + 1];
  int part[kBlock];
  int hist[kWaves][256];
  int nbuf;
  int ncut;
  int digit;
  int above;
  int stop;
  uint64_t thr_key;
};
typedef SelSharedT<kSelectMaxLists> SelShared;
typedef SelSharedT<1> RowShared;  // no list offsets: ~38 KB, several workgroups per CU

// Cuts keys[0..nb) down to its k largest keys (nb > k), in place and in any
// order, and returns the k-th largest key.  Whole block.
template <class SH>
__device__ __forceinline__ uint64_t block_keep_top(SH& S, int nb, int k) {
  const int tid = threadIdx.x;
  const int w = tid / kWave;
  const int lane = tid % kWave;
  uint64_t prefix = 0, pmask = 0;
  int need = k;  // rank of the wanted key among keys matching `prefix`
  for (int shift = 56; shift >= 0; shift -= 8) {
    for (int i = tid; i < kWaves * 256; i += kBlock) (&S.hist[0][0])[i] = 0;
    __syncthreads();
    for (int i = tid; i < nb; i += kBlock) {
      const uint64_t key = S.keys[i];
      if ((key & pmask) == prefix) atomicAdd(&S.hist[w][(int)((key >> shift) & 255)], 1);
    }
    __syncthreads();
    // digit d such that (#keys with digit > d) < need <= (#keys with digit >= d)
    if (w == 0) {
      int c[4];
      int s = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {  // lane owns bins 255-4*lane-j (descending)
        const int b = 255 - (4 * lane + j);
        c[j] = S.hist[0][b] + S.hist[1][b] + S.hist[2][b] + S.hist[3][b];
        s += c[j];
      }
      // exclusive prefix over lanes of s (descending bin order)
      int incl = wave_incl_sum_i32(s);
      int run = incl - s;  // keys in bins strictly above this lane's first bin
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (run < need && need <= run + c[j]) {
          S.digit = 255 - (4 * lane + j);
          S.above = run;
          S.stop = (run + c[j] == need) ? 1 : 0;
        }
        run += c[j];
      }
    }
    __syncthreads();
    const uint64_t dg = (uint64_t)S.digit;
    need -= S.above;
    prefix |= dg << shift;
    pmask |= 255ull << shift;
    if (S.stop) break;  // every key with this prefix is in the top k
    __syncthreads();
  }
  // keep keys >= prefix (with the undecided low bits at zero): exactly k keys
  if (tid == 0) S.ncut = 0;
  __syncthreads();
  uint64_t keep[kBuf / kBlock];
  int nk = 0;
  for (int i = tid; i < nb; i += kBlock) {
    const uint64_t key = S.keys[i];
    if (key >= prefix) keep[nk++] = key;
  }
  __syncthreads();
  int pos = nk ? atomicAdd(&S.ncut, nk) : 0;
  for (int j = 0; j < nk; ++j) S.keys[pos + j] = keep[j];
  __syncthreads();
  return prefix;
}

// Descending bitonic sort of keys[0..N) (N a power of two), whole block.
__device__ __forceinline__ void block_sort_desc(uint64_t* keys, int N) {
  const int tid = threadIdx.x;
  for (int size = 2; size <= N; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = tid; i < (N >> 1); i += kBlock) {
        const int lo = ((i & ~(stride - 1)) << 1) | (i & (stride - 1));
        const int hi = lo + stride;
        const bool desc = ((lo & size) == 0);
        const uint64_t x = keys[lo], y = keys[hi];
        if (desc ? (x < y) : (x > y)) {
          keys[lo] = y;
          keys[hi] = x;
        }
      }
      __syncthreads();
    }
  }
}

// Descending sort of keys[0..nb) in place for nb <= kBlock: each key's rank is
// the number of keys above it (keys are unique, so the ranks are a permutation
// of 0..nb-1), and the key moves to that slot.  G = min(8, kBlock / P) threads
// (P = nb rounded up to a power of two) count for each key, thread t over the
// t / P-th of G slices of the keys, so a short buffer still keeps every wave
// busy; thread t < nb sums its key's G counts.  Two barriers instead of the
// bitonic network's log2(N)(log2(N)+1)/2; every lane of a wave reads the same
// key at a time (an LDS broadcast).  Whole block.
__device__ __forceinline__ void block_rank_sort(uint64_t* keys, int nb) {
  __shared__ int part[kBlock];
  const int tid = threadIdx.x;
  int P = 1;
  while (P < nb) P <<= 1;
  const int G = min(8, kBlock / P);
  const int i = tid & (P - 1), g = tid / P;
  const int per = (nb + G - 1) / G;
  const int j0 = min(nb, g * per), j1 = min(nb, j0 + per);
  uint64_t mine = 0;
  int rank = 0;
  if (i < nb && g < G) {
    mine = keys[i];
#pragma unroll 8
    for (int j = j0; j < j1; ++j) rank += keys[j] > mine ? 1 : 0;  // (reads in flight together)
  }
  part[tid] = rank;
  __syncthreads();
  if (tid < nb) {  // (g == 0: mine is keys[tid])
    for (int gg = 1; gg < G; ++gg) rank += part[gg * P + tid];
    keys[rank] = mine;
  }
  __syncthreads();
}

// Descending sort of keys[0..nb) (nb <= kBuf / 2 when nb > kBlock).  Whole block.
__device__ __forceinline__ void block_sort_keys(uint64_t* keys, int nb) {
  if (nb <= kBlock) {
    block_rank_sort(keys, nb);
    return;
  }
  int N = 2;
  while (N < nb) N <<= 1;
  for (int i = nb + threadIdx.x; i < N; i += kBlock) keys[i] = 0ull;
  __syncthreads();
  block_sort_desc(keys, N);
}

constexpr int kSelFinal = 0, kSelTau = 1, kSelRescore = 2, kSelRescoreWide = 3, kSelRescoreMid = 4;
constexpr int kSelTauRescore = 5;  // launch mode: threshold from an int8 sampling pass
constexpr int kMaxD = 1536;

// Entries of list L of query q: its count, or in rescore mode the size of its
// row range when it overflowed.
__device__ __forceinline__ int list_len(const SelectArgs& a, int q, int L, bool rescore) {
  if (!a.lcount) return a.cap;
  const int c = a.lcount[(int64_t)q * a.nlists + L];
  if (rescore && c > a.cap) return (int)(a.tpc * a.wave_rows);
  return c;
}

// Corpus rows of the companion rows ids[0..N): out[j] = perm[ids[j]] (ids[j]
// when perm is null), -1 for ids outside [0, n).  The lookups are
// unconditional (index 0 stands in for the invalid ids) so that all N issue
// back to back: behind a per-lane branch each one waits for the one before.
template <int N>
__device__ __forceinline__ void map_rows(const int (&ids)[N], int (&out)[N], const int* perm, int n) {
  bool ok[N];
#pragma unroll
  for (int j = 0; j < N; ++j) ok[j] = ids[j] >= 0 && ids[j] < n;
  if (perm != nullptr && n > 0) {
    int r[N];
#pragma unroll
    for (int j = 0; j < N; ++j) r[j] = perm[ok[j] ? ids[j] : 0];
#pragma unroll
    for (int j = 0; j < N; ++j) out[j] = ok[j] ? r[j] : -1;
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) out[j] = ok[j] ? ids[j] : -1;
  }
}

// sids[0..m) <- perm[sids[0..m)] (nothing when perm is null), 8 independent
// lookups per thread at a time.  Whole block; ends with a barrier.
__device__ __forceinline__ void map_sids(int* sids, int m, const int* perm) {
  if (perm != nullptr) {
    for (int b0 = 0; b0 < m; b0 += 8 * kBlock) {
      int r[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int i = b0 + j * kBlock + threadIdx.x;
        r[j] = perm[i < m ? sids[i] : 0];
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int i = b0 + j * kBlock + threadIdx.x;
        if (i < m) sids[i] = r[j];
      }
    }
  }
  __syncthreads();
}

// Exclusive prefix sums of query q's list lengths into S.pre[0..NL], and an
// empty key buffer.  Each thread reads the counts of its (at most 32)
// consecutive lists once.  In rescore mode a list whose count exceeds cap
// overflowed in the scan and stands for its whole row range; its bit is set in
// `ovf` (zeroed by the caller) and *any_ovf becomes 1.  Whole block; returns
// the total (S.pre[NL]).
template <class SH>
__device__ __forceinline__ int list_prefix(SH& S, const SelectArgs& a, int q, bool rescore, unsigned* ovf = nullptr,
                           int* any_ovf = nullptr) {
  constexpr int kPer = kSelectMaxLists / kBlock;
  const int tid = threadIdx.x;
  const int NL = a.nlists;
  const int per = (NL + kBlock - 1) / kBlock;
  const int l0 = tid * per;
  int len[kPer];
  int sum = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    if (j >= per) break;  // (uniform)
    const int L = l0 + j;
    int c = 0;
    if (L < NL) {
      c = a.lcount ? a.lcount[(int64_t)q * NL + L] : a.cap;
      if (rescore && c > a.cap) {
        c = (int)(a.tpc * a.wave_rows);
        if (ovf) {
          atomicOr(&ovf[L >> 5], 1u << (L & 31));
          *any_ovf = 1;
        }
      }
    }
    len[j] = c;
    sum += c;
  }
  S.part[tid] = sum;
  if (tid == 0) {
    S.nbuf = 0;
    S.thr_key = 0ull;
  }
  __syncthreads();
  if (tid < kWave) {  // scan of the 256 partial sums by wave 0
    int v[4], s = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = S.part[4 * tid + j];
      s += v[j];
    }
    int incl = wave_incl_sum_i32(s);
    int run = incl - s;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      S.part[4 * tid + j] = run;
      run += v[j];
    }
    if (tid == kWave - 1) S.pre[NL] = incl;
  }
  __syncthreads();
  int run = S.part[tid];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    if (j >= per) break;
    const int L = l0 + j;
    if (L < NL) {
      S.pre[L] = run;
      run += len[j];
    }
  }
  __syncthreads();
  return S.pre[NL];
}

// The list holding flat entry gi: the largest L with S.pre[L] <= gi.
template <class SH>
__device__ __forceinline__ int list_of(const SH& S, int NL, int gi) {
  int lo = 0, hi = NL;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (S.pre[mid] <= gi) lo = mid; else hi = mid;
  }
  return lo;
}

// Smallest of keys[0..nb) (~0 when nb == 0).  Whole block; `red` is kWaves
// words of LDS.
__device__ __forceinline__ uint64_t block_min_key(const uint64_t* keys, int nb, uint64_t* red) {
  const int tid = threadIdx.x;
  uint64_t m = ~0ull;
  for (int i = tid; i < nb; i += kBlock) m = min(m, keys[i]);
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) m = min(m, __shfl_xor(m, off));
  if (tid % kWave == 0) red[tid / kWave] = m;
  __syncthreads();
  uint64_t r = red[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) r = min(r, red[w]);
  __syncthreads();
  return r;
}

// Wave 0 of a block, over per-wave 256-bin histograms: the highest bin b such
// that the bins >= b hold >= k counts in all, into *bstar, and that count into
// *above (bin 0 and the whole count when it is below k).  The caller barriers
// before (histograms complete) and after (results visible).
__device__ __forceinline__ void hist_cut_bin(const int (*hist)[256], int k, int* bstar, int* above) {
  const int lane = threadIdx.x % kWave;
  int c[4];
  int sum = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {  // lane owns bins 255-4*lane-j (descending)
    const int b = 255 - (4 * lane + j);
    c[j] = hist[0][b] + hist[1][b] + hist[2][b] + hist[3][b];
    sum += c[j];
  }
  int incl = wave_incl_sum_i32(sum);
  int run = incl - sum;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (run < k && k <= run + c[j]) {
      *bstar = 255 - (4 * lane + j);
      *above = run + c[j];
    }
    run += c[j];
  }
  if (lane == kWave - 1 && incl < k) {
    *bstar = 0;
    *above = incl;
  }
}

// Loose cut of the buffer's keys by score: a 256-bin histogram over the
// scores' [min, max] picks the fewest top bins holding at least k keys, and
// every key in them (m >= k keys, exactly those >= the returned key) is kept,
// compacted to keys[0..m).  Seven barriers (five without want_min), where the
// exact radix cut needs three or four per 8-bit digit.  Returns the smallest
// kept key (0 without want_min), or 0 leaving the buffer alone when m would
// exceed `limit` (many keys sharing a score).  Whole block; nb > k.
template <class SH>
__device__ __forceinline__ uint64_t block_cut_hist(SH& S, int nb, int k, int limit, uint64_t* red, int* m_out,
                                                   bool want_min = true) {
  constexpr int PER = kBuf / kBlock;
  __shared__ float mm[2][kWaves];
  const int tid = threadIdx.x;
  const int w = tid / kWave;
  const int lane = tid % kWave;
  uint64_t r[PER];
  float lo = __builtin_inff(), hi = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int i = j * kBlock + tid;
    r[j] = i < nb ? S.keys[i] : 0ull;
    if (i < nb) {
      const float v = key_score(r[j]);
      lo = fminf(lo, v);
      hi = fmaxf(hi, v);
    }
  }
  lo = wave_min_f32(lo);
  hi = wave_max_f32(hi);
  if (lane == 0) {
    mm[0][w] = lo;
    mm[1][w] = hi;
  }
  for (int i = tid; i < kWaves * 256; i += kBlock) (&S.hist[0][0])[i] = 0;
  __syncthreads();
  lo = mm[0][0];
  hi = mm[1][0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) {
    lo = fminf(lo, mm[0][i]);
    hi = fmaxf(hi, mm[1][i]);
  }
  // bin(score): non-decreasing in the score, the same arithmetic everywhere, and
  // in [0, 255] whatever the scores (infinite or NaN ones land in bin 0 or 255,
  // and no out-of-range float reaches the integer conversion)
  const bool span = hi > lo && __builtin_isfinite(lo) && __builtin_isfinite(hi);
  const float scale = span ? 256.0f / (hi - lo) : 0.0f;
  auto bin = [&](uint64_t key) {
    const float t = (key_score(key) - lo) * scale;
    return (int)(t >= 0.0f ? fminf(t, 255.0f) : 0.0f);
  };
#pragma unroll
  for (int j = 0; j < PER; ++j)
    if (j * kBlock + tid < nb) atomicAdd(&S.hist[w][bin(r[j])], 1);
  __syncthreads();
  if (w == 0) {  // the highest bin b with #(keys in bins >= b) >= k
    hist_cut_bin(S.hist, k, &S.digit, &S.above);
    if (lane == 0) S.ncut = 0;
  }
  __syncthreads();
  const int bstar = S.digit;
  const int m = S.above;
  *m_out = m;
  if (m > limit) return 0ull;
#pragma unroll
  for (int j = 0; j < PER; ++j)
    if (j * kBlock + tid < nb && bin(r[j]) >= bstar) S.keys[atomicAdd(&S.ncut, 1)] = r[j];
  __syncthreads();
  return want_min ? block_min_key(S.keys, m, red) : 0ull;
}

// End of a batch of appends.  When the next batch might not fit, the buffer is
// cut to the keys of its top histogram bins (at least k, raising the threshold
// key), or to exactly its k best when those bins hold too many.  After the last
// batch the buffer is cut to at most kBlock keys that hold its k best the same
// way and sorted by rank, leaving the k best first.  Whole block.  Every thread
// reads the count before any thread can append again, so all take the same
// branch.  Returns true when keys[0..min(nbuf, k)) are sorted (descending).
template <bool HIST = true, class SH>
__device__ __forceinline__ bool end_batch(SH& S, int k, bool last) {
  __shared__ uint64_t red[kWaves];
  __syncthreads();
  int nb = S.nbuf;
  bool sorted = false;
  if (!HIST) {  // exact cuts only (the row top-k: large k, registers needed elsewhere)
    if (last && nb <= kBlock) {
      block_rank_sort(S.keys, nb);
      sorted = true;
      if (threadIdx.x == 0 && nb > k) {
        S.nbuf = k;
        S.thr_key = S.keys[k - 1];
      }
    } else if (nb > kBuf - kBatch || (last && nb > k)) {
      const uint64_t kth = block_keep_top(S, nb, k);
      if (threadIdx.x == 0) {
        S.nbuf = k;
        S.thr_key = kth;
      }
    }
  } else if (!last && nb > kBuf - kBatch) {  // make room: a loose cut, else the exact one
    int m = 0;
    const uint64_t cut = block_cut_hist(S, nb, k, kBuf - kBatch, red, &m);
    if (m <= kBuf - kBatch) {
      if (threadIdx.x == 0) {
        S.nbuf = m;
        S.thr_key = cut - 1;  // keys >= cut (a real key, > 0) may still enter
      }
    } else {
      const uint64_t kth = block_keep_top(S, nb, k);
      if (threadIdx.x == 0) {
        S.nbuf = k;
        S.thr_key = kth;
      }
    }
  } else if (last && nb > k) {
    uint64_t kth = 0ull;
    if (nb > kBlock) {  // down to at most kBlock keys holding the k best
      int m = 0;
      block_cut_hist(S, nb, k, kBlock, red, &m, false);
      if (m > kBlock) {
        kth = block_keep_top(S, nb, k);
        m = k;
      }
      nb = m;
    }
    if (nb <= kBlock) {
      block_rank_sort(S.keys, nb);  // sorted: the k best first
      sorted = true;
      if (threadIdx.x == 0) {
        S.nbuf = k;
        S.thr_key = S.keys[k - 1];
      }
    } else if (threadIdx.x == 0) {  // k > kBlock: the exact cut's k keys, unsorted
      S.nbuf = k;
      S.thr_key = kth;
    }
  }
  __syncthreads();
  return sorted;
}


// Writes row q of the outputs from the descending keys[0..nb) (nb <= k),
// padded with (-inf, -1).  Whole block.
__device__ __forceinline__ void write_keys(const uint64_t* keys, const SelectArgs& a, int q, int nb) {
  const int k = a.k;
  for (int r = threadIdx.x; r < k; r += kBlock) {
    const bool ok = r < nb;
    a.out_v[(int64_t)q * k + r] = ok ? key_score(keys[r]) : -__builtin_inff();
    const int id = ok ? key_id(keys[r]) : -1;
    if (a.ids64)
      ((int64_t*)a.out_i)[(int64_t)q * k + r] = id;
    else
      ((int*)a.out_i)[(int64_t)q * k + r] = id;
  }
}

// Sorts the nb (<= k) surviving keys and writes row q of the outputs.  Whole block.
__device__ __forceinline__ void write_topk(SelShared& S, const SelectArgs& a, int q, int nb) {
  block_sort_keys(S.keys, nb);
  write_keys(S.keys, a, q, nb);
}

// Final and threshold modes: query blockIdx.x's candidate keys are streamed
// through the LDS buffer in kBatch steps, each filtered against the running
// k-th best key.
template <int MODE>
__global__ __launch_bounds__(kBlock) void select_kernel(SelectArgs a) {
  __shared__ SelShared S;
  const int tid = threadIdx.x;
  const int q = blockIdx.x;
  const int NL = a.nlists;
  const int k = a.k;
  // int8 pre-filter: wave 1 loads this query's row now and quantises it after
  // the selection (the load latency hides behind the selection's work)
  float qrow[kQ8RowPer];  // (dead outside the threshold mode)
  const bool quant = MODE == kSelTau && a.qq_out != nullptr && tid >= kWave && tid < 2 * kWave;
  if (MODE == kSelTau && quant) q8_load_row(a.q + (int64_t)q * a.d, a.d, tid - kWave, qrow);

  const int total = list_prefix(S, a, q, false);
  bool sorted = false;
  for (int base = 0; base < total; base += kBatch) {
    const uint64_t t = S.thr_key;
    // all of this thread's list lookups and loads first, then the appends: an
    // append (an LDS store) would otherwise order every later lookup after it
    // and expose one memory latency per entry
    float val[kGather];
    int idv[kGather];
#pragma unroll
    for (int j = 0; j < kGather; ++j) {
      const int gi = base + j * kBlock + tid;
      val[j] = 0.f;
      idv[j] = 0;
      if (gi < total) {
        const int L = list_of(S, NL, gi);
        const int idx = gi - S.pre[L];
        const int64_t off = ((int64_t)q * NL + L) * a.cap + idx;
        idv[j] = a.li ? a.li[off] : (int)((int64_t)L * a.cap + idx);
        val[j] = a.lv[off];
      }
    }
#pragma unroll
    for (int j = 0; j < kGather; ++j) {
      const uint64_t key = make_key(val[j], idv[j]);
      if (base + j * kBlock + tid < total && key > t) S.keys[atomicAdd(&S.nbuf, 1)] = key;
    }
    sorted = end_batch(S, k, base + kBatch >= total);
  }

  const int nb = min(S.nbuf, k);
  if (MODE == kSelTau) {
    if (quant)
      q8_quantize_row(qrow, a.d, a.dq, a.qq_out + (int64_t)q * a.dq, a.qmeta_out + q, tid - kWave, a.qf_out, q);
    // the k-th best key is the smallest survivor
    if (tid < kWave) {
      uint64_t m = ~0ull;
      for (int i = tid; i < nb; i += kWave) m = min(m, S.keys[i]);
#pragma unroll
      for (int off = kWave / 2; off > 0; off >>= 1) m = min(m, __shfl_xor(m, off));
      if (tid == 0) a.tau[q] = (nb >= k) ? key_score(m) : -__builtin_inff();
    }
  } else if (sorted) {
    write_keys(S.keys, a, q, nb);
  } else {
    write_topk(S, a, q, nb);
  }
}

// The threshold kernels stop their bit search above the kTauLowBits low bits
// of the 32-bit order key: the result, the largest key t with #(keys >= t) >= k
// among keys whose low bits are zero, is at most the exact k-th largest key
// (so still a valid filter: a lower bound on the k-th best score) and below
// it by less than 2^kTauLowBits order steps, about 2^-11 of the score.
constexpr int kTauLowBits = 12;

// Threshold mode with few units (<= 64 U per query, the sampling pre-pass's
// maxima in one list of `cap` floats): one wave per query.  The k-th largest
// score is found as the largest 32-bit order key t with #(keys >= t) >= k, bit
// by bit from the most significant down to kTauLowBits, each count a ballot per
// register and a scalar popcount (no cross-lane shuffles).  The int8
// pre-filter's query quantisation rides along.
template <int U>
__global__ __launch_bounds__(kWave) void tau_kernel(SelectArgs a) {
  const int q = blockIdx.x;
  const int lane = threadIdx.x;
  const int m = a.cap;
  const float* src = a.lv + (int64_t)q * m;
  float qrow[kQ8RowPer];
  const bool quant = a.qq_out != nullptr;
  if (quant) q8_load_row(a.q + (int64_t)q * a.d, a.d, lane, qrow);
  // Slots past m hold key 0, below every candidate t | (1 << bit) >= 1, so they
  // are never counted.  (A NaN score whose bits are all ones also maps to 0.)
  uint32_t key[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int i = u * kWave + lane;
    key[u] = i < m ? float_order(src[i]) : 0u;
  }
  uint32_t t = 0;
  if (m >= a.k) {
#pragma unroll 1
    for (int bit = 31; bit >= kTauLowBits; --bit) {
      const uint32_t cand = t | (1u << bit);
      int c = 0;
#pragma unroll
      for (int u = 0; u < U; ++u) c += __popcll(__ballot(key[u] >= cand));
      if (c >= a.k) t = cand;
    }
  }
  if (lane == 0) a.tau[q] = (m >= a.k) ? order_threshold(t) : -__builtin_inff();
  if (quant) q8_quantize_row(qrow, a.d, a.dq, a.qq_out + (int64_t)q * a.dq, a.qmeta_out + q, lane, a.qf_out, q);
}

// Threshold mode with up to U * 256 units per query (one list, as tau_kernel
// takes): the same bit-by-bit search over one 256-thread workgroup, each
// thread holding U keys; a bit's count is the four waves' ballot counts summed
// in LDS.  The count buffers alternate by bit, so one barrier per bit suffices:
// a wave writes buffer b & 1 again only after the barrier of bit b - 1, which
// every wave reaches after reading bit b's counts.  Wave 0 quantises the query
// for the int8 pre-filter as tau_kernel does.
template <int U>
__global__ __launch_bounds__(kBlock) void tau_block_kernel(SelectArgs a) {
  __shared__ int cnt[2][kWaves];
  const int q = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int w = tid / kWave;
  const int m = a.cap;
  const float* src = a.lv + (int64_t)q * m;
  uint32_t key[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int i = u * kBlock + tid;
    key[u] = i < m ? float_order(src[i]) : 0u;
  }
  uint32_t t = 0;
  if (m >= a.k) {
#pragma unroll 1
    for (int bit = 31; bit >= kTauLowBits; --bit) {
      const uint32_t cand = t | (1u << bit);
      int c = 0;
#pragma unroll
      for (int u = 0; u < U; ++u) c += __popcll(__ballot(key[u] >= cand));
      if (lane == 0) cnt[bit & 1][w] = c;
      __syncthreads();
      int tot = 0;
#pragma unroll
      for (int i = 0; i < kWaves; ++i) tot += cnt[bit & 1][i];
      if (tot >= a.k) t = cand;
    }
  }
  if (tid == 0) a.tau[q] = (m >= a.k) ? order_threshold(t) : -__builtin_inff();
  if (a.qq_out != nullptr && w == 0) {
    float qrow[kQ8RowPer];
    q8_load_row(a.q + (int64_t)q * a.d, a.d, lane, qrow);
    q8_quantize_row(qrow, a.d, a.dq, a.qq_out + (int64_t)q * a.dq, a.qmeta_out + q, lane, a.qf_out, q);
  }
}

// Rescoring: 16 lanes per candidate row, lane l taking the row's 16-byte pieces
// l, l+16, ... (RL of them at most); each group works on RU candidates at once,
// so RL*RU independent loads per lane are in flight.  RL = 4 covers d <= 512,
// RL = 6 d <= 768, RL = 12 (one candidate at a time) d <= 1536.
template <int MODE>
struct RescoreShape {
  static constexpr int RL = MODE == kSelRescoreWide ? 12 : MODE == kSelRescoreMid ? 6 : 4;
  static constexpr int RU = MODE == kSelRescoreWide ? 1 : MODE == kSelRescoreMid ? 2 : 4;
};

// This lane's query pieces for rescore_rows: piece l16 + 16 p of row q.
template <int RL>
__device__ __forceinline__ void load_query_pieces(const SelectArgs& a, int q, half8 (&qv)[RL]) {
  const int l16 = threadIdx.x & 15;
  const int nd = a.d / 8;
  const half8* qr = reinterpret_cast<const half8*>(a.q + (int64_t)q * a.d);
#pragma unroll
  for (int p = 0; p < RL; ++p) {
    const int c = l16 + 16 * p;
    qv[p] = c < nd ? qr[c] : half8{};
  }
}

// Exact fp32 scores (v_dot2_f32_f16) of the rows sids[0..m) against the query
// fragments qv; keys above t are appended to out[0..), *cnt counting them.
// Whole block.
template <int RL, int RU>
__device__ __forceinline__ void rescore_rows(uint64_t* out, int* cnt, const int* sids, int m, uint64_t t,
                                             const half8 (&qv)[RL], const _Float16* x, int d) {
  const int l16 = threadIdx.x & 15;
  const int nd = d / 8;
  for (int c0 = (threadIdx.x >> 4) * RU; c0 < m; c0 += (kBlock / 16) * RU) {
    int idu[RU];
    half8 xv[RU][RL];
#pragma unroll
    for (int u = 0; u < RU; ++u) idu[u] = c0 + u < m ? sids[c0 + u] : -1;
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const half8* xr = reinterpret_cast<const half8*>(x + (int64_t)(idu[u] < 0 ? 0 : idu[u]) * d);
#pragma unroll
      for (int p = 0; p < RL; ++p) {
        const int c = l16 + 16 * p;
        xv[u][p] = (idu[u] >= 0 && c < nd) ? xr[c] : half8{};
      }
    }
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      float acc = 0.f;
#pragma unroll
      for (int p = 0; p < RL; ++p)
#pragma unroll
        for (int j = 0; j < 8; j += 2)
          acc = __builtin_amdgcn_fdot2(half2v{qv[p][j], qv[p][j + 1]}, half2v{xv[u][p][j], xv[u][p][j + 1]}, acc,
                                       false);
#pragma unroll
      for (int off = 8; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
      if (l16 == 0 && idu[u] >= 0) {
        const uint64_t key = make_key(acc, idu[u]);
        if (key > t) out[atomicAdd(cnt, 1)] = key;
      }
    }
  }
}

// The first rescoring pass takes at least this many rows (the top bins holding
// max(k, kFirstPassMin) bounds): for small k its exact k-th best then sits
// high enough that the second pass rarely has rows left, and the search saves
// that pass's round trip of row loads.
constexpr int kFirstPassMin = 32;

// The int8 final stage in one pass over the candidates, when no list
// overflowed and there are at most 2 * kBuf of them: every entry is read once
// into LDS as a (U, corpus row) key (S.keys, then exb); the keys of the top
// bins of a 256-bin histogram of U (m >= max(k, kFirstPassMin) of them when
// there are that many, at most kBlock) are rescored, and the k-th best of their exact keys, kappa, bounds the final
// k-th best key from below (they are real rows); then every other candidate
// whose U reaches score(kappa) is rescored at once (a candidate below it has
// S' <= U < score(kappa) and cannot enter).  The same rows' exact keys as the
// general path below, so the same top k.  Returns false, having written
// nothing, when the top bins hold more than kBlock keys or the second rescoring pass
// more than kBuf - k rows (many equal bounds); the general path then runs.
// Whole block.
template <int RL, int RU>
__device__ __forceinline__ bool final_in_lds(SelShared& S, uint64_t* exb, uint64_t* ex1, int* sids,
                                             const SelectArgs& a, int q, int total) {
  constexpr int PER = 2 * kBuf / kBlock;
  constexpr int G8 = 8;
  __shared__ float mm[2][kWaves];
  __shared__ int cnt[2];  // exact keys; rows in sids
  __shared__ uint64_t red[kWaves];
  const int tid = threadIdx.x;
  const int w = tid / kWave;
  const int lane = tid % kWave;
  const int NL = a.nlists;
  const int k = a.k;
  auto cand = [&](int i) -> uint64_t& { return i < kBuf ? S.keys[i] : exb[i - kBuf]; };
  for (int i = tid; i < kWaves * 256; i += kBlock) (&S.hist[0][0])[i] = 0;
  if (tid == 0) {
    cnt[0] = 0;
    cnt[1] = 0;
  }
  // every entry, 8 per thread at a time (list lookups, then the loads, then
  // the row map when few), as a (U, row) key; key 0 marks an invalid row id.
  // Of thousands of candidates only the rows rescored (hundreds) are mapped to
  // corpus rows, by map_sids (a random 4-byte lookup costs a whole cache
  // line); of a few hundred, all are, on the way (saving map_sids' round trips).
  const bool map_now = total <= 1024;
  // the list of every entry, written by the list's thread into sids (free
  // until the first rescoring pass): one LDS read per entry instead of a binary search
  for (int L = tid; L < NL; L += kBlock)
    for (int i = S.pre[L], e = S.pre[L + 1]; i < e; ++i) sids[i] = L;
  __syncthreads();
  float lo = __builtin_inff(), hi = -__builtin_inff();
  for (int j0 = 0; j0 < PER && j0 * kBlock < total; j0 += G8) {
    int lst[G8];
#pragma unroll
    for (int j = 0; j < G8; ++j) {
      const int gi = (j0 + j) * kBlock + tid;
      lst[j] = gi < total ? sids[gi] : -1;
    }
    int idv[G8];
    float uv[G8];
#pragma unroll
    for (int j = 0; j < G8; ++j) {
      idv[j] = -1;
      uv[j] = 0.f;
      if (lst[j] >= 0) {
        const int64_t off = ((int64_t)q * NL + lst[j]) * a.cap + ((j0 + j) * kBlock + tid - S.pre[lst[j]]);
        idv[j] = a.li[off];
        uv[j] = a.lv[off];
      }
    }
    if (map_now) map_rows(idv, idv, a.perm, (int)a.n);
#pragma unroll
    for (int j = 0; j < G8; ++j) {
      const bool ok = idv[j] >= 0 && idv[j] < a.n;
      if (ok) {
        lo = fminf(lo, uv[j]);
        hi = fmaxf(hi, uv[j]);
      }
      if (lst[j] >= 0) cand((j0 + j) * kBlock + tid) = ok ? make_key(uv[j], idv[j]) : 0ull;
    }
  }
  lo = wave_min_f32(lo);
  hi = wave_max_f32(hi);
  if (lane == 0) {
    mm[0][w] = lo;
    mm[1][w] = hi;
  }
  __syncthreads();
  lo = mm[0][0];
  hi = mm[1][0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) {
    lo = fminf(lo, mm[0][i]);
    hi = fmaxf(hi, mm[1][i]);
  }
  // bin(U) as in block_cut_hist: non-decreasing, in [0, 255] whatever the bounds
  const bool span = hi > lo && __builtin_isfinite(lo) && __builtin_isfinite(hi);
  const float scale = span ? 256.0f / (hi - lo) : 0.0f;
  auto bin = [&](uint64_t kk) {
    const float t = (key_score(kk) - lo) * scale;
    return (int)(t >= 0.0f ? fminf(t, 255.0f) : 0.0f);
  };
  for (int i = tid; i < total; i += kBlock) {
    const uint64_t kk = cand(i);
    if (kk != 0ull) atomicAdd(&S.hist[w][bin(kk)], 1);
  }
  __syncthreads();
  // (bin 0, all keys, when fewer than k1min)
  if (w == 0) hist_cut_bin(S.hist, max(k, kFirstPassMin), &S.digit, &S.above);
  __syncthreads();
  const int bstar = S.digit;
  if (S.above > kBlock) return false;
  // first rescoring pass: the top bins' rows
  for (int i = tid; i < total; i += kBlock) {
    const uint64_t kk = cand(i);
    if (kk != 0ull && bin(kk) >= bstar) sids[atomicAdd(&cnt[1], 1)] = key_id(kk);
  }
  __syncthreads();
  const int m1 = cnt[1];
  map_sids(sids, m1, map_now ? nullptr : a.perm);
  half8 qv[RL];
  load_query_pieces<RL>(a, q, qv);
  rescore_rows<RL, RU>(ex1, &cnt[0], sids, m1, 0ull, qv, a.x, a.d);
  __syncthreads();
  uint64_t kap = 0ull;  // k-th best exact key of the first pass (0: fewer than k rows in all)
  if (m1 > k) {
    block_rank_sort(ex1, m1);  // m1 <= kBlock; the k best first
    kap = ex1[k - 1];
  } else if (m1 == k) {
    kap = block_min_key(ex1, k, red);
  }
  const int k1 = min(m1, k);
  if (tid == 0) cnt[1] = 0;
  __syncthreads();
  // second rescoring pass: every other row whose bound reaches score(kappa)
  if (kap != 0ull) {
    const float umin = key_score(kap);
    for (int i = tid; i < total; i += kBlock) {
      const uint64_t kk = cand(i);
      if (kk != 0ull && bin(kk) < bstar && key_score(kk) >= umin) sids[atomicAdd(&cnt[1], 1)] = key_id(kk);
    }
  }
  __syncthreads();
  const int m2 = cnt[1];
  if (k1 + m2 > kBuf) return false;
  for (int i = tid; i < k1; i += kBlock) exb[i] = ex1[i];  // (the candidates are no longer needed)
  if (tid == 0) cnt[0] = k1;
  map_sids(sids, m2, map_now ? nullptr : a.perm);
  rescore_rows<RL, RU>(exb, &cnt[0], sids, m2, kap, qv, a.x, a.d);
  __syncthreads();
  const int nex = cnt[0];
  block_sort_keys(exb, nex);
  write_keys(exb, a, q, min(nex, k));
  return true;
}

// Threshold of the int8 pre-filter from an int8 sampling pass (scan mode
// kMaxQ8): per query, each of its cap units' largest approximate score A (lv)
// and that row of the companion (li).  A 256-bin histogram of A over its
// [min, max] picks the units of the fewest top bins holding >= k of them (up
// to kBlock are kept: any k real rows will do); their rows are rescored
// exactly, as the final select rescores (fp32 sums of the fp16 products), and
// tau is the k-th best of those scores.  They are k real rows, so tau is at
// most the k-th best score of the final select.  One workgroup per query; U
// units per thread (cap <= U * kBlock).
template <int MODE, int U>
__global__ __launch_bounds__(kBlock) void tau_rescore_kernel(SelectArgs a) {
  constexpr int RL = RescoreShape<MODE>::RL, RU = RescoreShape<MODE>::RU;
  __shared__ int hist[kWaves][256];
  __shared__ float mm[2][kWaves];
  __shared__ int sids[kBlock];
  __shared__ uint64_t ex[kBlock];
  __shared__ int nrow, nex, bstar_s, above_s;
  const int q = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int w = tid / kWave;
  const int m = a.cap;
  const int k = a.k;
  float av[U];
  int row[U];
  float lo = __builtin_inff(), hi = -__builtin_inff();
  const float* src = a.lv + (int64_t)q * m;
  const int* rsrc = a.li + (int64_t)q * m;
#pragma unroll
  for (int u = 0; u < U; ++u) {  // (unconditional loads, clamped: they issue together)
    const int i = u * kBlock + tid;
    const int ic = i < m ? i : m - 1;
    av[u] = src[ic];
    row[u] = rsrc[ic];
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {  // a unit counts when it has a row (A > -inf, row < n)
    const bool ok = u * kBlock + tid < m && av[u] > -__builtin_inff() && row[u] >= 0 && row[u] < a.n;
    if (!ok) av[u] = -__builtin_inff();
    else {
      lo = fminf(lo, av[u]);
      hi = fmaxf(hi, av[u]);
    }
  }
  for (int i = tid; i < kWaves * 256; i += kBlock) (&hist[0][0])[i] = 0;
  if (tid == 0) {
    nrow = 0;
    nex = 0;
  }
  lo = wave_min_f32(lo);
  hi = wave_max_f32(hi);
  if (lane == 0) {
    mm[0][w] = lo;
    mm[1][w] = hi;
  }
  __syncthreads();
  lo = mm[0][0];
  hi = mm[1][0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) {
    lo = fminf(lo, mm[0][i]);
    hi = fmaxf(hi, mm[1][i]);
  }
  // bin(A): non-decreasing, in [0, 255] (as block_cut_hist)
  const bool span = hi > lo && __builtin_isfinite(lo) && __builtin_isfinite(hi);
  const float scale = span ? 256.0f / (hi - lo) : 0.0f;
  auto bin = [&](float v) {
    const float t = (v - lo) * scale;
    return (int)(t >= 0.0f ? fminf(t, 255.0f) : 0.0f);
  };
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (av[u] > -__builtin_inff()) atomicAdd(&hist[w][bin(av[u])], 1);
  __syncthreads();
  if (w == 0) hist_cut_bin(hist, k, &bstar_s, &above_s);
  __syncthreads();
  const int bstar = bstar_s;
  // the rows of the units in the top bins (every unit when fewer than k)
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (av[u] > -__builtin_inff() && bin(av[u]) >= bstar) {
      const int p = atomicAdd(&nrow, 1);
      if (p < kBlock) sids[p] = row[u];
    }
  }
  __syncthreads();
  const int mr = min(nrow, kBlock);
  map_sids(sids, mr, a.perm);
  half8 qv[RL];
  load_query_pieces<RL>(a, q, qv);
  rescore_rows<RL, RU>(ex, &nex, sids, mr, 0ull, qv, a.x, a.d);
  __syncthreads();
  if (mr >= k) block_rank_sort(ex, mr);  // (mr <= kBlock) the k best first
  if (tid == 0) a.tau[q] = mr >= k ? key_score(ex[k - 1]) : -__builtin_inff();
}

// Final stage of the int8 pre-filter: the exact top-k of query blockIdx.x from
// its candidate lists, whose entries are (U, row id) with U the scan's upper
// bound of the row's score.  The scan's bound covers |S - A| plus three times
// the rounding error eps of an fp32 sum of a row's products, so the score S'
// recomputed here (|S' - S| <= eps) satisfies S' <= U.
//
// Phase 1 keeps the k candidates of largest U (keys (U, id)) and rescores
// them; the smallest of their exact keys is a lower bound of the final k-th
// best key, since they are k real rows.  Phase 2 rescores only the other
// candidates whose U reaches the score of the running k-th best key: any
// other has S' <= U below it and cannot enter.  (With ~400 candidates per
// query at 1M rows, k = 10, about 70 rows are rescored instead of all.)
// A list that overflowed in the scan (count > cap) stands for every row of
// its range: those rows skip phase 1 and are all rescored in phase 2, so the
// result stays exact whatever the data.
//
// With a.exact set, rescore_kernel has already replaced the bounds by exact
// scores (small batches, where it spreads the row reads over more workgroups
// than one per query): phase 1 is then a plain selection, and phase 2 only
// rescans overflowed lists.
template <int MODE>
__global__ __launch_bounds__(kBlock) void rescore_select_kernel(SelectArgs a) {
  __shared__ SelShared S;
  constexpr int RL = RescoreShape<MODE>::RL, RU = RescoreShape<MODE>::RU;
  __shared__ int sids[2 * kBuf];                  // rows to rescore
  __shared__ uint64_t ex[kBuf];                   // one-pass form: candidates past kBuf, then exact keys
  __shared__ uint64_t ex1[kBlock];                // one-pass form: exact keys of the first rescoring pass
  __shared__ unsigned ovf[kSelectMaxLists / 32];  // overflowed-list bitmap
  __shared__ uint64_t red[kWaves];
  __shared__ int nrows;
  __shared__ int any_ovf;
  const int tid = threadIdx.x;
  const int q = blockIdx.x;
  const int NL = a.nlists;
  const int k = a.k;
  for (int i = tid; i < (NL + 31) / 32; i += kBlock) ovf[i] = 0u;
  if (tid == 0) any_ovf = 0;
  __syncthreads();
  const int total = list_prefix(S, a, q, true, ovf, &any_ovf);
  if (!a.exact && !any_ovf && total <= 2 * kBuf && final_in_lds<RL, RU>(S, ex, ex1, sids, a, q, total)) return;
  half8 qv[RL];
  load_query_pieces<RL>(a, q, qv);
  auto overflowed = [&](int L) { return ((ovf[L >> 5] >> (L & 31)) & 1u) != 0; };

  // Phase 1: the k largest (U, id) keys of the lists that did not overflow.
  for (int base = 0; base < total; base += kBatch) {
    const uint64_t t = S.thr_key;
    float val[kGather];
    int idv[kGather];
#pragma unroll
    for (int j = 0; j < kGather; ++j) {  // lookups and loads first (see select_kernel)
      const int gi = base + j * kBlock + tid;
      val[j] = 0.f;
      idv[j] = -1;
      if (gi < total) {
        const int L = list_of(S, NL, gi);
        if (!overflowed(L)) {
          const int64_t off = ((int64_t)q * NL + L) * a.cap + (gi - S.pre[L]);
          idv[j] = a.li[off];
          val[j] = a.lv[off];
        }
      }
    }
    map_rows(idv, idv, a.perm, (int)a.n);  // companion rows -> corpus rows
#pragma unroll
    for (int j = 0; j < kGather; ++j) {
      const uint64_t key = make_key(val[j], idv[j]);
      if (idv[j] >= 0 && key > t) S.keys[atomicAdd(&S.nbuf, 1)] = key;
    }
    const bool last = base + kBatch >= total;
    if (a.exact) {
      end_batch(S, k, last);
    } else {
      // bound keys: any m >= k of the largest serve phase 1, so a loose cut
      // (at most kBlock keys after the last one) replaces the radix cut
      __syncthreads();
      const int nb = S.nbuf;
      if (nb > kBuf - kBatch || (last && nb > k)) {
        int m = 0;
        uint64_t cut = block_cut_hist(S, nb, k, last ? kBlock : kBuf - kBatch, red, &m);
        if (m > (last ? kBlock : kBuf - kBatch)) {
          cut = block_keep_top(S, nb, k);
          m = k;
        }
        if (tid == 0) {
          S.nbuf = m;
          S.thr_key = cut - 1;  // keep appending keys >= cut (a real key, > 0)
        }
      }
      __syncthreads();
    }
  }
  // Entries with a bound key below ucut are exactly those phase 1 did not keep.
  uint64_t ucut = 0ull;
  if (!a.exact) {  // (exact lists: the buffer already holds their best k keys)
    const int n1 = S.nbuf;  // <= k, or m <= kBlock after a loose cut
    ucut = block_min_key(S.keys, n1, red);
    for (int i = tid; i < n1; i += kBlock) sids[i] = key_id(S.keys[i]);
    __syncthreads();
    if (tid == 0) {
      S.nbuf = 0;
      S.thr_key = 0ull;
    }
    __syncthreads();
    rescore_rows<RL, RU>(S.keys, &S.nbuf, sids, n1, 0ull, qv, a.x, a.d);
    __syncthreads();
    if (n1 > k) {  // n1 <= kBlock: sort, keep the k best
      block_rank_sort(S.keys, S.nbuf);
      if (tid == 0) {
        S.nbuf = k;
        S.thr_key = S.keys[k - 1];
      }
    } else if (n1 == k) {
      const uint64_t kth = block_min_key(S.keys, S.nbuf, red);
      if (tid == 0) S.thr_key = kth;
    }
    __syncthreads();
  }

  // Phase 2: the remaining candidates that can still enter, and overflow rows.
  for (int base = 0; base < total && (any_ovf || !a.exact); base += kBatch) {
    const uint64_t t = S.thr_key;
    const float umin = t ? key_score(t) : -__builtin_inff();
    if (tid == 0) nrows = 0;
    __syncthreads();
    int idv[kGather];
    float uv[kGather];
    bool fromlist[kGather];
#pragma unroll
    for (int j = 0; j < kGather; ++j) {  // lookups and loads first (see select_kernel)
      const int gi = base + j * kBlock + tid;
      idv[j] = -1;
      uv[j] = 0.f;
      fromlist[j] = false;
      if (gi < total) {
        const int L = list_of(S, NL, gi);
        const int idx = gi - S.pre[L];
        if (overflowed(L)) {  // row idx of the list's range
          const int64_t tile = (int64_t)(L / a.rsplits) * a.tpc + idx / a.wave_rows;
          const int64_t row = tile * a.tile_rows + (int64_t)(L % a.rsplits) * a.wave_rows + idx % a.wave_rows;
          if (tile < a.ntiles && row < a.n) idv[j] = (int)row;
        } else if (!a.exact) {
          const int64_t off = ((int64_t)q * NL + L) * a.cap + idx;
          const int lid = a.li[off];
          uv[j] = a.lv[off];
          if (lid >= 0 && lid < a.n && uv[j] >= umin) {
            idv[j] = lid;
            fromlist[j] = true;
          }
        }
      }
    }
    map_rows(idv, idv, a.perm, (int)a.n);  // companion rows -> corpus rows
#pragma unroll
    for (int j = 0; j < kGather; ++j)  // list entries phase 1 kept are out
      if (fromlist[j] && make_key(uv[j], idv[j]) >= ucut) idv[j] = -1;
#pragma unroll
    for (int j = 0; j < kGather; ++j)
      if (idv[j] >= 0) sids[atomicAdd(&nrows, 1)] = idv[j];
    __syncthreads();
    rescore_rows<RL, RU>(S.keys, &S.nbuf, sids, nrows, t, qv, a.x, a.d);
    end_batch(S, k, base + kBatch >= total);
  }
  write_topk(S, a, q, min(S.nbuf, k));
}

// Exact scores of the int8 pre-filter's candidates, written over their bounds
// in lv: workgroup b takes query b / splits and its lists [s*lpb, (s+1)*lpb),
// s = b % splits.  Overflowed lists (count > cap) are left to the select.
// Then each list is compacted to the candidates that can still be in the top
// k: with tau the k-th best fp32 score of the sampled rows and eps >= the
// rounding error of any fp32 sum of a row's d products (d * 2^-24 * |q| |x|),
// the k-th best exact score over all rows is >= tau - 2 eps, so a candidate
// below that can never be returned.
template <int MODE>
__global__ __launch_bounds__(kBlock) void rescore_kernel(SelectArgs a) {
  constexpr int RL = RescoreShape<MODE>::RL, RU = RescoreShape<MODE>::RU;
  __shared__ int pre[kBlock + 1];
  __shared__ int wsum[kWaves];
  __shared__ int kept[kBlock];      // survivors per list so far
  __shared__ int sid[kBatch];       // a batch's candidates (companion rows, as listed)
  __shared__ int sxr[kBatch];       // ... their corpus rows
  __shared__ short slist[kBatch];   // ... and their lists (local index)
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int l16 = tid & 15;
  const int NL = a.nlists;
  const int splits = (NL + a.lpb - 1) / a.lpb;
  const int q = blockIdx.x / splits;
  const int L0 = (blockIdx.x % splits) * a.lpb;
  const int nl = min(a.lpb, NL - L0);
  int c = 0;
  if (tid < nl) {
    c = a.lcount[(int64_t)q * NL + L0 + tid];
    if (c > a.cap) c = 0;  // overflowed: left to the select
  }
  kept[tid] = 0;
  int v = wave_incl_sum_i32(c);  // inclusive scan of the list counts
  if (lane == kWave - 1) wsum[tid / kWave] = v;
  __syncthreads();
  for (int i = 0; i < tid / kWave; ++i) v += wsum[i];
  pre[tid + 1] = v;
  if (tid == 0) pre[0] = 0;
  __syncthreads();
  const int total = pre[nl];
  float cut = -__builtin_inff();
  if (a.tau_in) {  // tau - 2 eps, eps = gamma |q| max|x| (the sampled rows' norms are <= max|x|)
    const float4 qm = a.qmeta[q];
    cut = a.tau_in[q] - (qm.y + qm.z) * a.xmax[0] * 2.f * a.gamma * (1.0f + 1.0f / 1024.0f);
  }
  const int nd = a.d / 8;
  const half8* qr = reinterpret_cast<const half8*>(a.q + (int64_t)q * a.d);
  half8 qv[RL];
#pragma unroll
  for (int m = 0; m < RL; ++m) {
    const int cc = l16 + 16 * m;
    qv[m] = cc < nd ? qr[cc] : half8{};
  }
  float* lvq = const_cast<float*>(a.lv) + ((int64_t)q * NL + L0) * a.cap;
  int* liq = const_cast<int*>(a.li) + ((int64_t)q * NL + L0) * a.cap;
  for (int base = 0; base < total; base += kBatch) {
    const int cnt = min(kBatch, total - base);
    // every id of the batch is read before any survivor is written back, and a
    // survivor's new slot never passes an unread entry of its list
    int idv[kGather], lov[kGather];
#pragma unroll
    for (int j = 0; j < kGather; ++j) {  // lookups and loads first (see select_kernel)
      const int i = j * kBlock + tid;
      idv[j] = -1;
      lov[j] = 0;
      if (i < cnt) {
        const int gi = base + i;
        int lo = 0, hi = nl;  // largest list with pre[list] <= gi
        while (hi - lo > 1) {
          const int mid = (lo + hi) >> 1;
          if (pre[mid] <= gi) lo = mid; else hi = mid;
        }
        idv[j] = liq[(int64_t)lo * a.cap + (gi - pre[lo])];
        lov[j] = lo;
      }
    }
    int xrv[kGather];
#pragma unroll
    for (int j = 0; j < kGather; ++j)
      if (idv[j] < 0 || idv[j] >= a.n) idv[j] = -1;
    map_rows(idv, xrv, a.perm, (int)a.n);
#pragma unroll
    for (int j = 0; j < kGather; ++j) {
      const int i = j * kBlock + tid;
      if (i < cnt) {
        sid[i] = idv[j];
        sxr[i] = xrv[j];
        slist[i] = (short)lov[j];
      }
    }
    __syncthreads();
    for (int c0 = (tid >> 4) * RU; c0 < cnt; c0 += (kBlock / 16) * RU) {
      int idu[RU], xru[RU];
      half8 xv[RU][RL];
#pragma unroll
      for (int u = 0; u < RU; ++u) {
        idu[u] = c0 + u < cnt ? sid[c0 + u] : -1;
        xru[u] = c0 + u < cnt ? sxr[c0 + u] : -1;
      }
#pragma unroll
      for (int u = 0; u < RU; ++u) {
        const half8* xr = reinterpret_cast<const half8*>(a.x + (int64_t)(idu[u] < 0 ? 0 : xru[u]) * a.d);
#pragma unroll
        for (int m = 0; m < RL; ++m) {
          const int cc = l16 + 16 * m;
          xv[u][m] = (idu[u] >= 0 && cc < nd) ? xr[cc] : half8{};
        }
      }
#pragma unroll
      for (int u = 0; u < RU; ++u) {
        float acc = 0.f;
#pragma unroll
        for (int m = 0; m < RL; ++m)
#pragma unroll
          for (int j = 0; j < 8; j += 2)
            acc = __builtin_amdgcn_fdot2(half2v{qv[m][j], qv[m][j + 1]}, half2v{xv[u][m][j], xv[u][m][j + 1]},
                                         acc, false);
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
        if (l16 == 0 && idu[u] >= 0 && acc >= cut) {
          const int lo = slist[c0 + u];
          const int pos = atomicAdd(&kept[lo], 1);
          lvq[(int64_t)lo * a.cap + pos] = acc;
          liq[(int64_t)lo * a.cap + pos] = idu[u];
        }
      }
    }
    __syncthreads();
  }
  if (tid < nl && a.lcount[(int64_t)q * NL + L0 + tid] <= a.cap)
    const_cast<int*>(a.lcount)[(int64_t)q * NL + L0 + tid] = kept[tid];
}

// Exact top-k of one chunk of one score row: workgroup b takes row b / chunks,
// columns [c*len, min((c+1)*len, n)) with c = b % chunks, and writes its k
// best (value, column) sorted to out[b].  Each thread loads kRowU values per
// round with all loads in flight, then appends the ones above the running k-th
// best key in kBatch-sized steps (wave-aggregated LDS appends).
constexpr int kRowU = 32;

__global__ __launch_bounds__(kBlock) void rowtopk_kernel(RowTopkArgs a) {
  __shared__ RowShared S;
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int b = blockIdx.x;
  const int q = b / a.chunks;
  const int c = b % a.chunks;
  const int64_t start = (int64_t)c * a.len;
  const int cnt = (int)min<int64_t>(a.len, a.n - start);
  const float* src = a.scores + (int64_t)q * a.n + start;
  const int k = a.k;
  if (tid == 0) {
    S.nbuf = 0;
    S.thr_key = 0ull;
  }
  __syncthreads();
  constexpr int kRound = kRowU * kBlock;
  for (int base = 0; base < cnt; base += kRound) {
    float val[kRowU];
#pragma unroll
    for (int u = 0; u < kRowU; ++u) {  // coalesced; a slot past the end re-reads column 0
      const int gi = base + u * kBlock + tid;
      val[u] = src[gi < cnt ? gi : 0];
    }
#pragma unroll
    for (int sub = 0; sub < kRowU / (kBatch / kBlock); ++sub) {
      const uint64_t t = S.thr_key;
#pragma unroll
      for (int j = 0; j < kBatch / kBlock; ++j) {
        const int u = sub * (kBatch / kBlock) + j;
        const int gi = base + u * kBlock + tid;
        const uint64_t key = make_key(val[u], (int)(start + gi));
        const bool pass = gi < cnt && key > t;
        const uint64_t mk = __ballot(pass);
        int pos = 0;
        if (lane == 0 && mk) pos = atomicAdd(&S.nbuf, __popcll(mk));
        pos = __shfl(pos, 0);
        if (pass) S.keys[pos + lanes_below(mk)] = key;
      }
      const bool last = base + (sub + 1) * kBatch >= cnt;
      end_batch<false>(S, k, last);
      if (last) break;
    }
  }
  const int nb = min(S.nbuf, k);
  block_sort_keys(S.keys, nb);
  for (int r = tid; r < k; r += kBlock) {
    const bool ok = r < nb;
    const int64_t o = (int64_t)b * k + r;
    a.out_v[o] = ok ? key_score(S.keys[r]) : -__builtin_inff();
    const int id = ok ? key_id(S.keys[r]) : -1;
    if (a.ids64)
      ((int64_t*)a.out_i)[o] = id;
    else
      ((int*)a.out_i)[o] = id;
  }
}

}  // namespace

hipError_t launch_rowtopk(const RowTopkArgs& a, int blocks, hipStream_t s) {
  if (a.k < 1 || a.k > kSelectMaxK || a.chunks < 1 || a.len < 1 || blocks < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(rowtopk_kernel, dim3(blocks), dim3(kBlock), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_rescore(const SelectArgs& a, int nq, hipStream_t s) {
  if (a.q == nullptr || a.x == nullptr || a.li == nullptr || a.lv == nullptr || a.lcount == nullptr || a.d < 8 ||
      a.d % 8 != 0 || a.d > kMaxD || a.lpb < 1 || a.lpb > kBlock || a.nlists < 1)
    return hipErrorInvalidValue;
  const int64_t grid = (int64_t)nq * ((a.nlists + a.lpb - 1) / a.lpb);
  if (grid < 1 || grid > 0x7fffffff) return hipErrorInvalidValue;
  if (a.d <= 16 * 8 * RescoreShape<kSelRescore>::RL)
    hipLaunchKernelGGL(rescore_kernel<kSelRescore>, dim3((unsigned)grid), dim3(kBlock), 0, s, a);
  else if (a.d <= 16 * 8 * RescoreShape<kSelRescoreMid>::RL)
    hipLaunchKernelGGL(rescore_kernel<kSelRescoreMid>, dim3((unsigned)grid), dim3(kBlock), 0, s, a);
  else
    hipLaunchKernelGGL(rescore_kernel<kSelRescoreWide>, dim3((unsigned)grid), dim3(kBlock), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_select(int mode, const SelectArgs& a, int nq, hipStream_t s) {
  if (a.nlists < 1 || a.nlists > kSelectMaxLists || a.k < 1 || a.k > kSelectMaxK) return hipErrorInvalidValue;
  switch (mode) {
    case kSelFinal:
      hipLaunchKernelGGL(select_kernel<kSelFinal>, dim3(nq), dim3(kBlock), 0, s, a);
      break;
    case kSelTau:
      if (a.qq_out != nullptr &&
          (a.q == nullptr || a.qmeta_out == nullptr || a.d < 8 || a.d % 8 != 0 || a.d > a.dq || a.dq % 8 != 0 ||
           a.dq > kQ8RowPer * kWave || (a.qf_out != nullptr && a.dq % 32 != 0)))
        return hipErrorInvalidValue;
      if (a.nlists == 1 && a.li == nullptr && a.lcount == nullptr && a.cap >= 1 && a.cap <= 8 * kWave) {
        // one list of at most 512 unit maxima per query: the one-wave kernel
        // (measured 6.8 vs 10.8 us at C2 against the 256-thread select)
        hipLaunchKernelGGL(tau_kernel<8>, dim3(nq), dim3(kWave), 0, s, a);
        break;
      }
      if (a.nlists == 1 && a.li == nullptr && a.lcount == nullptr && a.cap > 8 * kBlock && a.cap <= 16 * kBlock) {
        // 2049-4096 unit maxima (k = 100 over 1M rows: 3840): the same search
        // over a workgroup (measured 20.8 vs 23.5 us at 1M x 768, batch 256;
        // the 256-thread select stays faster at 1024 units and one query)
        hipLaunchKernelGGL(tau_block_kernel<16>, dim3(nq), dim3(kBlock), 0, s, a);
        break;
      }
      hipLaunchKernelGGL(select_kernel<kSelTau>, dim3(nq), dim3(kBlock), 0, s, a);
      break;
    case kSelTauRescore: {
      if (a.q == nullptr || a.x == nullptr || a.li == nullptr || a.lv == nullptr || a.tau == nullptr || a.d < 8 ||
          a.d % 8 != 0 || a.d > kMaxD || a.cap < 1 || a.cap > 16 * kBlock || a.k > kBlock)
        return hipErrorInvalidValue;
      const int u = a.cap <= 2 * kBlock ? 2 : a.cap <= 4 * kBlock ? 4 : a.cap <= 8 * kBlock ? 8 : 16;
      const int wc = a.d <= 16 * 8 * RescoreShape<kSelRescore>::RL      ? 0
                     : a.d <= 16 * 8 * RescoreShape<kSelRescoreMid>::RL ? 1
                                                                         : 2;
#define CVS_TAU_RESCORE(MODEW, UU) hipLaunchKernelGGL((tau_rescore_kernel<MODEW, UU>), dim3(nq), dim3(kBlock), 0, s, a)
      if (wc == 0) {
        if (u == 2) CVS_TAU_RESCORE(kSelRescore, 2); else if (u == 4) CVS_TAU_RESCORE(kSelRescore, 4);
        else if (u == 8) CVS_TAU_RESCORE(kSelRescore, 8); else CVS_TAU_RESCORE(kSelRescore, 16);
      } else if (wc == 1) {
        if (u == 2) CVS_TAU_RESCORE(kSelRescoreMid, 2); else if (u == 4) CVS_TAU_RESCORE(kSelRescoreMid, 4);
        else if (u == 8) CVS_TAU_RESCORE(kSelRescoreMid, 8); else CVS_TAU_RESCORE(kSelRescoreMid, 16);
      } else {
        if (u == 2) CVS_TAU_RESCORE(kSelRescoreWide, 2); else if (u == 4) CVS_TAU_RESCORE(kSelRescoreWide, 4);
        else if (u == 8) CVS_TAU_RESCORE(kSelRescoreWide, 8); else CVS_TAU_RESCORE(kSelRescoreWide, 16);
      }
#undef CVS_TAU_RESCORE
      break;
    }
    case kSelRescore:
      if (a.q == nullptr || a.x == nullptr || a.li == nullptr || a.lcount == nullptr || a.d < 8 || a.d % 8 != 0 ||
          a.d > kMaxD || a.wave_rows < 1 || a.rsplits < 1 || a.tile_rows < a.rsplits * a.wave_rows ||
          (int64_t)a.tpc * a.wave_rows > 0x7fffffff)
        return hipErrorInvalidValue;
      if (a.d <= 16 * 8 * RescoreShape<kSelRescore>::RL)
        hipLaunchKernelGGL(rescore_select_kernel<kSelRescore>, dim3(nq), dim3(kBlock), 0, s, a);
      else if (a.d <= 16 * 8 * RescoreShape<kSelRescoreMid>::RL)
        hipLaunchKernelGGL(rescore_select_kernel<kSelRescoreMid>, dim3(nq), dim3(kBlock), 0, s, a);
      else
        hipLaunchKernelGGL(rescore_select_kernel<kSelRescoreWide>, dim3(nq), dim3(kBlock), 0, s, a);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace cvs
