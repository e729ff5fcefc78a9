// int8 companion of the fp16 corpus and of each query batch, for the int8
// pre-filter of the exact search (no counterpart in the reference, whose only
// corpus format is the fp16 matrix of cuda_vector_search/index.py:56-78).
//
// Rows are quantised symmetrically: a 64-row block of the corpus shares one
// scale s_b = max|x| / 127 over the block, a query row has its own s_q, and
// x~ = rint(x * (127 / max)) in [-127, 127].  The scan then computes
// A = s_q * s_b * sum(q~ x~) with int8 MFMAs (exact int32 sums), and
//
//     |q.x - A| <= |q^|_2 |f|_2 + |e|_2 |x|_2,   q^ = s_q q~, e = q - q^,
//                                                 f = x - s_b x~
//
// (Cauchy-Schwarz on the two residuals), so the exact score of every row lies
// within that slack of A.  The kernels here store, per block, s_b and upper
// bounds of max |f_r|_2 and max |x_r|_2 over its rows, and per query s_q,
// |q^|_2 and |e|_2 (norms rounded up to cover fp32 accumulation).
//
// The companion holds the rows in ascending order of their largest magnitude
// max_j |x_rj| (a stable sort: equal maxima keep the corpus order), so that
// the rows sharing a block, and its scale s_b, have nearly the same maximum:
// |f_r| then tracks each row's own scale instead of the largest of 64 random
// rows (for unit rows of width 768, max |f_r| per block drops by ~23% and the
// slack by ~13%).  perm[r] is the corpus row at companion row r.
#include <rocprim/device/device_radix_sort.hpp>

#include "cvs_common.h"
#include "cvs_kernels.h"
#include "cvs_q8_row.h"

namespace cvs {

namespace {

constexpr float kNormUp = 1.0f + 1.0f / 2048.0f;  // > 1 + d * 2^-24 for d <= 8192, plus sqrt's ulp


// Sort keys: the fp16 bit pattern of max_j |x_rj| (non-negative halves order
// like their bit patterns; NaNs are skipped as fmaxf skips them), 16 lanes per
// row, and the row ids to carry along.
__global__ __launch_bounds__(kBlock) void q8_rowkey_kernel(const _Float16* x, int64_t n, int d, uint16_t* key,
                                                           int* ids) {
  const int64_t row = (int64_t)blockIdx.x * (kBlock / 16) + (threadIdx.x >> 4);
  const int l16 = threadIdx.x & 15;
  float m = 0.f;
  if (row < n) {
    const half8* src = reinterpret_cast<const half8*>(x + row * (int64_t)d);
    for (int p = l16; p < d / 8; p += 16) {
      const half8 v = src[p];
#pragma unroll
      for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf((float)v[j]));
    }
  }
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  if (row < n && l16 == 0) {
    key[row] = __builtin_bit_cast(uint16_t, (_Float16)m);  // m is a half's magnitude: exact
    ids[row] = (int)row;
  }
}

// perm[r] = r for the padding rows r in [n, rows).
__global__ __launch_bounds__(kBlock) void q8_perm_pad_kernel(int* perm, int64_t n, int64_t rows) {
  const int64_t r = n + (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (r < rows) perm[r] = (int)r;
}

// One workgroup per 64-row block of the companion; thread t takes companion
// row t/4 (corpus row perm[t/4]) and the 8-element pieces p = t%4, t%4 + 4,
// ... of it (4 consecutive lanes read 64 contiguous bytes).  Pass 1: block max
// |x|; pass 2 (re-reading the rows, now in cache): quantise, write the int8 row
// and its zero padding, and reduce the row's residual and value norms.
__global__ __launch_bounds__(kBlock) void q8_build_kernel(Q8BuildArgs a) {
  __shared__ float red[kBlock / kWave];
  __shared__ float fmax_s[kBlock / kWave], xmax_s[kBlock / kWave];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int64_t blk = blockIdx.x;
  const int64_t row = blk * 64 + (tid >> 2);
  const int part = tid & 3;
  const bool live = row < a.n;
  const int pieces = a.d / 8;  // 8-element pieces per row
  const int64_t srow = live ? a.perm[row] : 0;
  const half8* src = reinterpret_cast<const half8*>(a.x + srow * (int64_t)a.d);

  float m = 0.f;
  if (live) {
    for (int p = part; p < pieces; p += 4) {
      const half8 v = src[p];
#pragma unroll
      for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf((float)v[j]));
    }
  }
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  if (lane == 0) red[w] = m;
  __syncthreads();
  const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = M / 127.f;
  const float inv = M > 0.f ? 127.f / M : 0.f;

  signed char* dst = a.xq + row * (int64_t)a.dq;
  float ff = 0.f, xx = 0.f;
  for (int p = part; p < pieces; p += 4) {
    half8 v = {};
    if (live) v = src[p];
    int2 packed;
    unsigned lo = 0, hi = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float xv = (float)v[j];
      const signed char c = q8_quant(xv, inv);
      const float f = fmaf(-s, (float)c, xv);
      ff = fmaf(f, f, ff);
      xx = fmaf(xv, xv, xx);
      if (j < 4) lo |= (unsigned)(unsigned char)c << (8 * j);
      else hi |= (unsigned)(unsigned char)c << (8 * (j - 4));
    }
    packed.x = (int)lo;
    packed.y = (int)hi;
    *reinterpret_cast<int2*>(dst + 8 * p) = packed;
  }
  for (int c = a.d + 8 * part; c < a.dq; c += 32) *reinterpret_cast<int2*>(dst + c) = int2{0, 0};
  // row norms: the row's 4 threads are consecutive lanes
  ff += __shfl_xor(ff, 1);
  ff += __shfl_xor(ff, 2);
  xx += __shfl_xor(xx, 1);
  xx += __shfl_xor(xx, 2);
  float fn = sqrtf(ff) * kNormUp, xn = sqrtf(xx) * kNormUp;
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    fn = fmaxf(fn, __shfl_xor(fn, off));
    xn = fmaxf(xn, __shfl_xor(xn, off));
  }
  if (lane == 0) {
    fmax_s[w] = fn;
    xmax_s[w] = xn;
  }
  __syncthreads();
  if (tid == 0) {
    float4 meta;
    meta.x = s;
    meta.y = fmaxf(fmaxf(fmax_s[0], fmax_s[1]), fmaxf(fmax_s[2], fmax_s[3]));
    meta.z = fmaxf(fmaxf(xmax_s[0], xmax_s[1]), fmaxf(xmax_s[2], xmax_s[3]));
    meta.w = 0.f;
    a.bmeta[blk] = meta;
  }
}

// One workgroup: the corpus-wide maximum row norm (max of the blocks' .z).
__global__ __launch_bounds__(kBlock) void q8_xmax_kernel(const float4* bmeta, int64_t nblk, float* xmax) {
  __shared__ float red[kBlock / kWave];
  float m = 0.f;
  for (int64_t b = threadIdx.x; b < nblk; b += kBlock) m = fmaxf(m, bmeta[b].z);
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) *xmax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// One wave per query row; the whole grid also clears a.zero[0, nzero).
__global__ __launch_bounds__(kBlock) void q8_query_kernel(Q8QueryArgs a) {
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < a.nzero; i += (int64_t)gridDim.x * kBlock)
    a.zero[i] = 0ull;
  const int64_t r = (int64_t)blockIdx.x * (kBlock / kWave) + (threadIdx.x >> 6);
  if (r >= a.nq) return;  // whole wave
  q8_query_row(a.q + r * a.d, a.d, a.dq, a.qq + r * a.dq, a.qmeta + r, threadIdx.x & 63, a.qf, r);
}

}  // namespace

// Row order, then the blocks.  The sort's key and id buffers and its scratch
// live in the companion's own int8-row region (rows * dq >= 384 n bytes, far
// more than the ~14 n bytes they take), which q8_build_kernel overwrites only
// after the sort, in stream order: the build allocates nothing.
hipError_t launch_q8_build(const Q8BuildArgs& a, hipStream_t s) {
  if (a.d < 8 || a.d % 8 != 0 || a.dq < a.d || a.dq % 128 != 0 || a.perm == nullptr) return hipErrorInvalidValue;
  const int64_t blocks = (a.n + 63) / 64;
  if (blocks <= 0 || blocks > 0x7fffffff || a.n >= 0x7fffffff) return hipErrorInvalidValue;
  const int64_t n = a.n, rows = blocks * 64;
  size_t sort_bytes = 0;
  hipError_t e = rocprim::radix_sort_pairs(nullptr, sort_bytes, (const uint16_t*)nullptr, (uint16_t*)nullptr,
                                           (const int*)nullptr, (int*)nullptr, (unsigned)n, 0, 15, s);
  if (e != hipSuccess) return e;
  const size_t keys_bytes = ((size_t)n * sizeof(uint16_t) + 255) / 256 * 256;
  const size_t ids_bytes = ((size_t)n * sizeof(int) + 255) / 256 * 256;
  if (2 * keys_bytes + ids_bytes + sort_bytes > (size_t)rows * (size_t)a.dq) return hipErrorInvalidValue;
  char* buf = reinterpret_cast<char*>(a.xq);
  uint16_t* key_in = reinterpret_cast<uint16_t*>(buf);
  uint16_t* key_out = reinterpret_cast<uint16_t*>(buf + keys_bytes);
  int* ids = reinterpret_cast<int*>(buf + 2 * keys_bytes);
  void* tmp = buf + 2 * keys_bytes + ids_bytes;
  const int per = kBlock / 16;
  hipLaunchKernelGGL(q8_rowkey_kernel, dim3((unsigned)((n + per - 1) / per)), dim3(kBlock), 0, s, a.x, n, a.d,
                     key_in, ids);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  e = rocprim::radix_sort_pairs(tmp, sort_bytes, key_in, key_out, ids, a.perm, (unsigned)n, 0, 15, s);
  if (e != hipSuccess) return e;
  if (rows > n)
    hipLaunchKernelGGL(q8_perm_pad_kernel, dim3((unsigned)((rows - n + kBlock - 1) / kBlock)), dim3(kBlock), 0, s,
                       a.perm, n, rows);
  hipLaunchKernelGGL(q8_build_kernel, dim3((unsigned)blocks), dim3(kBlock), 0, s, a);
  hipLaunchKernelGGL(q8_xmax_kernel, dim3(1), dim3(kBlock), 0, s, a.bmeta, blocks, a.xmax);
  return hipGetLastError();
}

hipError_t launch_q8_queries(const Q8QueryArgs& a, hipStream_t s) {
  if (a.d < 8 || a.d % 8 != 0 || a.d > kQ8RowPer * kWave || a.dq < a.d || a.dq > kQ8RowPer * kWave || a.dq % 128 != 0 ||
      a.nzero < 0 || (a.nzero > 0 && a.zero == nullptr))
    return hipErrorInvalidValue;
  const int64_t per = kBlock / kWave;
  const int64_t grid = (a.nq + per - 1) / per;
  if (grid <= 0 || grid > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL(q8_query_kernel, dim3((unsigned)grid), dim3(kBlock), 0, s, a);
  return hipGetLastError();
}

}  // namespace cvs
