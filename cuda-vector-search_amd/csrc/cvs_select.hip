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
#include "cvs_common.h"
#include "cvs_kernels.h"

namespace cvs {

namespace {

constexpr int kBuf = 4096;    // LDS key buffer
constexpr int kBatch = 2048;  // candidates gathered per round
constexpr int kWaves = kBlock / kWave;

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
__device__ uint64_t block_keep_top(SH& S, int nb, int k) {
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
      int incl = s;
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) {
        const int o = __shfl_up(incl, off);
        if (lane >= off) incl += o;
      }
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
__device__ void block_sort_desc(uint64_t* keys, int N) {
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

template <int TAU_MODE>
__global__ __launch_bounds__(kBlock) void select_kernel(SelectArgs a) {
  __shared__ SelShared S;
  const int tid = threadIdx.x;
  const int q = blockIdx.x;
  const int NL = a.nlists;
  const int k = a.k;

  // Exclusive prefix sum of the list counts.
  const int per = (NL + kBlock - 1) / kBlock;
  const int l0 = tid * per;
  const int l1 = min(NL, l0 + per);
  int sum = 0;
  for (int L = l0; L < l1; ++L) sum += a.lcount ? a.lcount[(int64_t)q * NL + L] : a.cap;
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
    int incl = s;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const int o = __shfl_up(incl, off);
      if (tid >= off) incl += o;
    }
    int run = incl - s;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      S.part[4 * tid + j] = run;
      run += v[j];
    }
    if (tid == kWave - 1) S.pre[NL] = incl;
  }
  __syncthreads();
  {
    int run = S.part[tid];
    for (int L = l0; L < l1; ++L) {
      S.pre[L] = run;
      run += a.lcount ? a.lcount[(int64_t)q * NL + L] : a.cap;
    }
  }
  __syncthreads();
  const int total = S.pre[NL];

  for (int base = 0; base < total; base += kBatch) {
    const uint64_t t = S.thr_key;
    for (int j = 0; j < kBatch / kBlock; ++j) {
      const int gi = base + j * kBlock + tid;
      if (gi < total) {
        int lo = 0, hi = NL;  // largest L with pre[L] <= gi
        while (hi - lo > 1) {
          const int mid = (lo + hi) >> 1;
          if (S.pre[mid] <= gi) lo = mid; else hi = mid;
        }
        const int idx = gi - S.pre[lo];
        const int64_t off = ((int64_t)q * NL + lo) * a.cap + idx;
        const int id = a.li ? a.li[off] : (int)((int64_t)lo * a.cap + idx);
        const uint64_t key = make_key(a.lv[off], id);
        if (key > t) S.keys[atomicAdd(&S.nbuf, 1)] = key;
      }
    }
    __syncthreads();
    const int nb = S.nbuf;
    const bool last = base + kBatch >= total;
    if (nb > kBuf - kBatch || (last && nb > k)) {
      const uint64_t kth = block_keep_top(S, nb, k);
      if (tid == 0) {
        S.nbuf = k;
        S.thr_key = kth;
      }
      __syncthreads();
    }
  }

  const int nb = min(S.nbuf, k);
  if (TAU_MODE) {
    // the k-th best key is the smallest survivor
    if (tid < kWave) {
      uint64_t m = ~0ull;
      for (int i = tid; i < nb; i += kWave) m = min(m, S.keys[i]);
#pragma unroll
      for (int off = kWave / 2; off > 0; off >>= 1) m = min(m, __shfl_xor(m, off));
      if (tid == 0) a.tau[q] = (nb >= k) ? key_score(m) : -__builtin_inff();
    }
  } else {
    int N = 2;
    while (N < nb) N <<= 1;
    for (int i = nb + tid; i < N; i += kBlock) S.keys[i] = 0ull;
    __syncthreads();
    block_sort_desc(S.keys, N);
    for (int r = tid; r < k; r += kBlock) {
      const bool ok = r < nb;
      a.out_v[(int64_t)q * k + r] = ok ? key_score(S.keys[r]) : -__builtin_inff();
      const int id = ok ? key_id(S.keys[r]) : -1;
      if (a.ids64)
        ((int64_t*)a.out_i)[(int64_t)q * k + r] = id;
      else
        ((int*)a.out_i)[(int64_t)q * k + r] = id;
    }
  }
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
      __syncthreads();
      const int nb = S.nbuf;
      const bool last = base + (sub + 1) * kBatch >= cnt;
      if (nb > kBuf - kBatch || (last && nb > k)) {
        const uint64_t kth = block_keep_top(S, nb, k);
        if (tid == 0) {
          S.nbuf = k;
          S.thr_key = kth;
        }
        __syncthreads();
      }
      if (last) break;
    }
  }
  const int nb = min(S.nbuf, k);
  int N = 2;
  while (N < nb) N <<= 1;
  for (int i = nb + tid; i < N; i += kBlock) S.keys[i] = 0ull;
  __syncthreads();
  block_sort_desc(S.keys, N);
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

hipError_t launch_select(int tau_mode, const SelectArgs& a, int nq, hipStream_t s) {
  if (a.nlists < 1 || a.nlists > kSelectMaxLists || a.k < 1 || a.k > kSelectMaxK) return hipErrorInvalidValue;
  if (tau_mode)
    hipLaunchKernelGGL(select_kernel<1>, dim3(nq), dim3(kBlock), 0, s, a);
  else
    hipLaunchKernelGGL(select_kernel<0>, dim3(nq), dim3(kBlock), 0, s, a);
  return hipGetLastError();
}

}  // namespace cvs
