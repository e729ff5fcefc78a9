// Exact top-k selection over candidate lists, one 256-thread workgroup per query.
//
// Replaces the merge of csrc/kernels.cu:373-445.  The reference merges exactly
// k candidates per chunk with one warp and k serial arg-max rounds; here each
// query's candidates (any number per list) are streamed in batches of 1024,
// filtered against the running k-th best key, and the survivors are sorted in
// LDS with a block-wide bitonic network whenever the buffer could overflow.
// Keys order by (score desc, id asc) and are unique, so the k largest keys are
// exactly the top-k and the output comes out sorted like the reference's.
//
// Threshold mode returns only the score of the k-th best key (used to turn the
// sampling pre-pass's unit maxima into per-query thresholds).
#include "cvs_common.h"
#include "cvs_kernels.h"

namespace cvs {

namespace {

constexpr int kBuf = 2048;
constexpr int kBatch = 1024;

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
  __shared__ uint64_t keys[kBuf];
  __shared__ int pre[kSelectMaxLists + 1];
  __shared__ int part[kBlock];
  __shared__ int nbuf;
  __shared__ uint64_t thr_key;

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
  part[tid] = sum;
  if (tid == 0) {
    nbuf = 0;
    thr_key = 0ull;
  }
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int i = 0; i < kBlock; ++i) {
      const int v = part[i];
      part[i] = run;
      run += v;
    }
    pre[NL] = run;
  }
  __syncthreads();
  {
    int run = part[tid];
    for (int L = l0; L < l1; ++L) {
      pre[L] = run;
      run += a.lcount ? a.lcount[(int64_t)q * NL + L] : a.cap;
    }
  }
  __syncthreads();
  const int total = pre[NL];

  for (int base = 0; base < total; base += kBatch) {
    const uint64_t t = thr_key;
    for (int j = 0; j < kBatch / kBlock; ++j) {
      const int gi = base + j * kBlock + tid;
      if (gi < total) {
        // largest L with pre[L] <= gi
        int lo = 0, hi = NL;
        while (hi - lo > 1) {
          const int mid = (lo + hi) >> 1;
          if (pre[mid] <= gi) lo = mid; else hi = mid;
        }
        const int idx = gi - pre[lo];
        const int64_t off = ((int64_t)q * NL + lo) * a.cap + idx;
        const int id = a.li ? a.li[off] : (int)((int64_t)lo * a.cap + idx);
        const uint64_t key = make_key(a.lv[off], id);
        if (key > t) keys[atomicAdd(&nbuf, 1)] = key;
      }
    }
    __syncthreads();
    const int nb = nbuf;
    const bool last = base + kBatch >= total;
    if (nb > kBuf - kBatch || (last && nb > 0)) {
      int N = 2;
      while (N < nb) N <<= 1;
      for (int i = nb + tid; i < N; i += kBlock) keys[i] = 0ull;
      __syncthreads();
      block_sort_desc(keys, N);
      if (tid == 0) {
        if (nb >= k) {
          nbuf = k;
          thr_key = keys[k - 1];
        }
      }
      __syncthreads();
    }
  }

  const int nb = min(nbuf, k);
  if (TAU_MODE) {
    if (tid == 0) a.tau[q] = (nb >= k) ? key_score(keys[k - 1]) : -__builtin_inff();
  } else {
    for (int r = tid; r < k; r += kBlock) {
      const bool ok = r < nb;
      a.out_v[(int64_t)q * k + r] = ok ? key_score(keys[r]) : -__builtin_inff();
      a.out_i[(int64_t)q * k + r] = ok ? key_id(keys[r]) : -1;
    }
  }
}

}  // namespace

hipError_t launch_select(int tau_mode, const SelectArgs& a, int nq, hipStream_t s) {
  if (a.nlists < 1 || a.nlists > kSelectMaxLists || a.k < 1 || a.k > 256) return hipErrorInvalidValue;
  if (tau_mode)
    hipLaunchKernelGGL(select_kernel<1>, dim3(nq), dim3(kBlock), 0, s, a);
  else
    hipLaunchKernelGGL(select_kernel<0>, dim3(nq), dim3(kBlock), 0, s, a);
  return hipGetLastError();
}

}  // namespace cvs
