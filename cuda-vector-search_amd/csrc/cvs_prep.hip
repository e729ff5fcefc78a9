// Row preparation: L2 normalisation and zero-padding of fp16 rows in one pass.
//
// Replaces the torch sequences of cuda_vector_search/index.py:35-41
// (_normalize_: fp32 row norm clamped at 1e-12, divide, round to fp16) and
// index.py:27-32 (_pad_width: zero columns up to a multiple of 64), which the
// reference runs on every cosine search for the queries (index.py:89-98, about
// ten small kernels per call) and once over the corpus at Index construction
// (index.py:56-78).
//
// One wave per row: the row is read once (fp16 -> fp32), its sum of squares is
// reduced across the wave, and the scaled row is written back as fp16 with the
// padding columns zeroed.  Source and destination may be the same rows (the
// wave reads its whole row before writing it).  Memory-bound: 2*d bytes read
// and 2*width bytes written per row.
#include "cvs_common.h"
#include "cvs_kernels.h"

namespace cvs {

namespace {

constexpr int kMaxPer = 24;  // d <= 1536 = 24 elements per lane held in registers

// WIDE: rows of any width, read twice (sum of squares, then scale and write);
// a lane writes only the columns it read, so in-place rows stay safe.
template <bool WIDE>
__global__ __launch_bounds__(kBlock) void prep_rows_kernel(PrepArgs a) {
  const int lane = lane_id();
  const int64_t row = (int64_t)blockIdx.x * (kBlock / kWave) + (threadIdx.x >> 6);
  if (row >= a.n) return;  // whole wave
  const _Float16* src = a.src + row * a.src_stride;
  _Float16* dst = a.dst + row * a.dst_width;
  float v[WIDE ? 1 : kMaxPer];
  float ss = 0.f;
  if constexpr (WIDE) {
#pragma unroll 4
    for (int c = lane; c < a.d; c += kWave) {
      const float t = (float)src[c];
      ss += t * t;
    }
  } else {
#pragma unroll
    for (int i = 0; i < kMaxPer; ++i) {
      const int c = i * kWave + lane;
      v[i] = c < a.d ? (float)src[c] : 0.f;
      ss += v[i] * v[i];
    }
  }
  float nrm = 1.f;
  if (a.normalize) {  // x / max(||x||, 1e-12), divided per element like the reference
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    nrm = fmaxf(sqrtf(ss), 1e-12f);
  }
  if constexpr (WIDE) {
#pragma unroll 4
    for (int c = lane; c < a.dst_width; c += kWave) {
      const float t = c < a.d ? (float)src[c] : 0.f;
      dst[c] = (_Float16)(a.normalize ? t / nrm : t);
    }
  } else {
#pragma unroll
    for (int i = 0; i < kMaxPer; ++i) {
      const int c = i * kWave + lane;
      if (c < a.dst_width) dst[c] = (_Float16)(c < a.d ? (a.normalize ? v[i] / nrm : v[i]) : 0.f);
    }
  }
}

}  // namespace

hipError_t launch_prep(const PrepArgs& a, hipStream_t s) {
  if (a.d < 1 || a.dst_width < a.d) return hipErrorInvalidValue;
  const int64_t rows_per_block = kBlock / kWave;
  const int64_t grid = (a.n + rows_per_block - 1) / rows_per_block;
  if (grid > 0x7fffffff) return hipErrorInvalidValue;
  if (a.dst_width <= kMaxPer * kWave)
    hipLaunchKernelGGL(prep_rows_kernel<false>, dim3((unsigned)grid), dim3(kBlock), 0, s, a);
  else
    hipLaunchKernelGGL(prep_rows_kernel<true>, dim3((unsigned)grid), dim3(kBlock), 0, s, a);
  return hipGetLastError();
}

}  // namespace cvs
