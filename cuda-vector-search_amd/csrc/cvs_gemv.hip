// Batch-1 GEMV + filter: the bandwidth-bound single-query path.
//
// The reference runs batch-1 queries through its tensor-core kernel with a
// 16-row query block, 15/16 of it padding (csrc/kernels.cu:514, README.md:67-71).
// Here one query is scored with packed-half dot products (v_dot2_f32_f16, fp32
// accumulation) and no matrix-core padding.  Each corpus row is split across 8
// lanes that read 128 contiguous bytes per load (full cache lines), so a wave
// covers 8 rows per load round; UNR rounds are in flight per wave and the query
// stays in VGPRs.  Rows are split into contiguous per-wave ranges (long
// sequential streams per wave).  Scores are filtered against the threshold and
// survivors appended to the wave's candidate list, exactly as in the scan path.
#include "cvs_common.h"
#include "cvs_kernels.h"

namespace cvs {

namespace {

constexpr int kUnr = 2;  // 8-row groups per wave per iteration

__device__ __forceinline__ float dot8(half8 a, half8 b, float acc) {
  acc = __builtin_amdgcn_fdot2(half2v{a[0], a[1]}, half2v{b[0], b[1]}, acc, false);
  acc = __builtin_amdgcn_fdot2(half2v{a[2], a[3]}, half2v{b[2], b[3]}, acc, false);
  acc = __builtin_amdgcn_fdot2(half2v{a[4], a[5]}, half2v{b[4], b[5]}, acc, false);
  acc = __builtin_amdgcn_fdot2(half2v{a[6], a[7]}, half2v{b[6], b[7]}, acc, false);
  return acc;
}

// PMAX = max 128-byte pieces per row handled by one lane (d <= 64*PMAX).
template <int PMAX, int MODE>
__global__ __launch_bounds__(kBlock) void gemv_kernel(GemvArgs a) {
  __shared__ uint64_t sortbuf[MODE == kAppend ? 4 * kMaxCap : 1];
  const int lane = lane_id();
  const int w = threadIdx.x >> 6;
  const int sub = lane & 7;     // 16-byte slot within a 128-byte piece
  const int rg = lane >> 3;     // row within an 8-row group
  const int gw = blockIdx.x * 4 + w;
  const int d = a.d;
  const int np = d >> 6;
  const int64_t n = a.n;

  // Unconditional loads (a piece past d re-reads the last one and is never
  // used): a per-load branch would put each behind a wait for the previous one.
  half8 qv[PMAX];
#pragma unroll
  for (int p = 0; p < PMAX; ++p) qv[p] = *(const half8*)(a.q + min(p, np - 1) * 64 + sub * 8);

  int64_t r_begin, r_end;
  if (MODE == kMax) {
    if (gw >= a.nsample) return;  // whole wave
    const int64_t nblocks = (n + 63) / 64;
    const int64_t blk = ((2 * (int64_t)gw + 1) * nblocks) / (2 * (int64_t)a.nsample);
    r_begin = blk * 64;
    r_end = r_begin + 64 < n ? r_begin + 64 : n;
  } else {
    r_begin = (int64_t)gw * a.rows_per_wave;
    r_end = r_begin + a.rows_per_wave < n ? r_begin + a.rows_per_wave : n;
  }

  float thr = (MODE == kAppend && a.tau) ? a.tau[0] : -__builtin_inff();
  float umax = -__builtin_inff();  // kMax: best score of this lane group's rows
  int count = 0;
  float* lv = nullptr;
  int* li = nullptr;
  if (MODE == kAppend) {
    lv = a.lv + (int64_t)gw * a.cap;
    li = a.li + (int64_t)gw * a.cap;
  }

  for (int64_t r0 = r_begin; r0 < r_end; r0 += 8 * kUnr) {
    half8 xv[kUnr][PMAX];
#pragma unroll
    for (int u = 0; u < kUnr; ++u) {
      int64_t row = r0 + u * 8 + rg;
      if (row >= n) row = n - 1;
      const _Float16* src = a.x + row * d + sub * 8;
#pragma unroll
      for (int p = 0; p < PMAX; ++p)
        if (p < np) xv[u][p] = __builtin_nontemporal_load((const half8*)(src + p * 64));
    }
#pragma unroll
    for (int u = 0; u < kUnr; ++u) {
      float acc = 0.f;
#pragma unroll
      for (int p = 0; p < PMAX; ++p)
        if (p < np) acc = dot8(xv[u][p], qv[p], acc);
      acc += __shfl_xor(acc, 1);
      acc += __shfl_xor(acc, 2);
      acc += __shfl_xor(acc, 4);
      const int64_t row = r0 + u * 8 + rg;
      const bool valid = row < r_end;
      if (MODE == kMax) {
        if (valid) umax = fmaxf(umax, acc);
      } else {
        bool pass = valid && sub == 0 && acc >= thr;
        uint64_t mask = __ballot(pass);
        if (mask) {
          int nnew = __popcll(mask);
          if (count + nnew > a.cap) {
            thr = fmaxf(thr, wave_compact(lv, li, count, a.k, sortbuf + w * kMaxCap));
            count = a.k;
            pass = pass && acc >= thr;
            mask = __ballot(pass);
            nnew = __popcll(mask);
          }
          if (pass) {
            const int pos = count + lanes_below(mask);
            lv[pos] = acc;
            li[pos] = (int)row;
          }
          count += nnew;
        }
      }
    }
  }
  // kMax: sampling unit (block, rg) = the block's rows congruent to rg mod 8, or
  // the whole block when upb == 1; its maximum is the score of one actual row
  // (or -inf past the corpus end).
  if (MODE == kMax) {
    if (a.upb == 1) {  // one unit per block: the maximum over its 8 row classes
      umax = fmaxf(umax, __shfl_xor(umax, 8));
      umax = fmaxf(umax, __shfl_xor(umax, 16));
      umax = fmaxf(umax, __shfl_xor(umax, 32));
      if (lane == 0) a.umax[gw] = umax;
    } else if (sub == 0) {
      a.umax[(int64_t)gw * 8 + rg] = umax;
    }
  }
  if (MODE == kAppend && lane == 0) a.lcount[gw] = count;
}

template <int PMAX>
hipError_t launch_p(const GemvArgs& a, int grid, hipStream_t s) {
  if (a.mode == kAppend)
    hipLaunchKernelGGL((gemv_kernel<PMAX, kAppend>), dim3(grid), dim3(kBlock), 0, s, a);
  else if (a.mode == kMax)
    hipLaunchKernelGGL((gemv_kernel<PMAX, kMax>), dim3(grid), dim3(kBlock), 0, s, a);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemv(int dmax, const GemvArgs& a, int grid, hipStream_t s) {
  if (a.d > dmax) return hipErrorInvalidValue;
  if (dmax <= 384) return launch_p<6>(a, grid, s);
  if (dmax <= 768) return launch_p<12>(a, grid, s);
  if (dmax <= 1536) return launch_p<24>(a, grid, s);
  return hipErrorInvalidValue;
}

}  // namespace cvs
