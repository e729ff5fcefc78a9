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
//
// kAppendQ8 is the same kernel over the int8 companion of the corpus
// (v_dot4_i32_i8, exact int32 sums, 128-byte pieces of 128 int8): rows whose
// score upper bound reaches the threshold are appended, a full list is marked
// overflowed instead of compacted, and the select recomputes exact scores.
// kMaxQ8 samples that way: per unit the largest approximate score
// A = s_q s_b sum(q~ x~) and its row, for the threshold kernel to rescore.
#include "cvs_common.h"
#include "cvs_kernels.h"

namespace cvs {

namespace {

constexpr int kUnr = 2;  // 8-row groups per wave per iteration

// 16 int8 x 16 int8, exact.
__device__ __forceinline__ int dot16_i8(half8 a, half8 b, int acc) {
  const i32x4 x = __builtin_bit_cast(i32x4, a), y = __builtin_bit_cast(i32x4, b);
  acc = __builtin_amdgcn_sdot4(x[0], y[0], acc, false);
  acc = __builtin_amdgcn_sdot4(x[1], y[1], acc, false);
  acc = __builtin_amdgcn_sdot4(x[2], y[2], acc, false);
  acc = __builtin_amdgcn_sdot4(x[3], y[3], acc, false);
  return acc;
}

__device__ __forceinline__ float dot8(half8 a, half8 b, float acc) {
  acc = __builtin_amdgcn_fdot2(half2v{a[0], a[1]}, half2v{b[0], b[1]}, acc, false);
  acc = __builtin_amdgcn_fdot2(half2v{a[2], a[3]}, half2v{b[2], b[3]}, acc, false);
  acc = __builtin_amdgcn_fdot2(half2v{a[4], a[5]}, half2v{b[4], b[5]}, acc, false);
  acc = __builtin_amdgcn_fdot2(half2v{a[6], a[7]}, half2v{b[6], b[7]}, acc, false);
  return acc;
}

// PMAX = max 128-byte pieces per row handled by one lane (d <= 64*PMAX).
// PMAX = 0: rows of any width, taken kWide pieces at a time; the query's pieces
// are re-read per row group (a wave's 8 row groups read the same 128 bytes per
// load, and the whole query stays in the vector L1 / L2).
constexpr int kWide = 8;

template <int PMAX, int MODE>
__global__ __launch_bounds__(kBlock) void gemv_kernel(GemvArgs a) {
  constexpr bool Q8 = (MODE == kAppendQ8 || MODE == kMaxQ8);
  constexpr bool APP = (MODE == kAppend || MODE == kAppendQ8);
  constexpr bool SMAX = (MODE == kMax || MODE == kMaxQ8);
  __shared__ uint64_t sortbuf[MODE == kAppend ? 4 * kMaxCap : 1];
  const int lane = lane_id();
  const int w = threadIdx.x >> 6;
  const int sub = lane & 7;     // 16-byte slot within a 128-byte piece
  const int rg = lane >> 3;     // row within an 8-row group
  const int gw = blockIdx.x * 4 + w;
  const int d = a.d;            // row elements (fp16) or bytes (int8)
  const int np = Q8 ? d >> 7 : d >> 6;  // 128-byte pieces per row
  const int64_t rb = Q8 ? d : 2 * (int64_t)d;  // row bytes
  const int64_t n = a.n;
  const unsigned char* xb = reinterpret_cast<const unsigned char*>(a.x);
  const unsigned char* qb = reinterpret_cast<const unsigned char*>(a.q);

  // Unconditional loads (a piece past d re-reads the last one and is never
  // used): a per-load branch would put each behind a wait for the previous one.
  constexpr bool WIDE = (PMAX == 0);
  static_assert(!WIDE || !Q8, "the int8 companion holds rows of at most 1536 bytes");
  half8 qv[WIDE ? 1 : PMAX];
#pragma unroll
  for (int p = 0; p < PMAX; ++p) qv[p] = *(const half8*)(qb + min(p, np - 1) * 128 + sub * 16);
  float4 qm = float4{0.f, 0.f, 0.f, 0.f};
  if (Q8) qm = a.qmeta[0];

  int64_t r_begin, r_end;
  if (SMAX) {
    if (gw >= a.nsample) return;  // whole wave
    const int64_t nblocks = (n + 63) / 64;
    const int64_t blk = ((2 * (int64_t)gw + 1) * nblocks) / (2 * (int64_t)a.nsample);
    r_begin = blk * 64;
    r_end = r_begin + 64 < n ? r_begin + 64 : n;
  } else {
    r_begin = (int64_t)gw * a.rows_per_wave;
    r_end = r_begin + a.rows_per_wave < n ? r_begin + a.rows_per_wave : n;
  }

  float thr = (APP && a.tau) ? a.tau[0] : -__builtin_inff();
  float umax = -__builtin_inff();  // kMax: best score of this lane group's rows
  int uarg = 0;                    // kMaxQ8: its row
  int count = 0;
  float* lv = nullptr;
  int* li = nullptr;
  if (APP) {
    lv = a.lv + (int64_t)gw * a.cap;
    li = a.li + (int64_t)gw * a.cap;
  }

  for (int64_t r0 = r_begin; r0 < r_end; r0 += 8 * kUnr) {
    half8 xv[kUnr][WIDE ? 1 : PMAX];
    const unsigned char* srcs[kUnr];
#pragma unroll
    for (int u = 0; u < kUnr; ++u) {
      int64_t row = r0 + u * 8 + rg;
      if (row >= n) row = n - 1;
      srcs[u] = xb + row * rb + sub * 16;
#pragma unroll
      for (int p = 0; p < PMAX; ++p)
        if (p < np) xv[u][p] = __builtin_nontemporal_load((const half8*)(srcs[u] + p * 128));
    }
    // WIDE: this lane's partial dot products, kWide pieces at a time
    float wacc[kUnr];
#pragma unroll
    for (int u = 0; u < kUnr; ++u) wacc[u] = 0.f;
    if constexpr (WIDE) {
#pragma unroll 1
      for (int p0 = 0; p0 < np; p0 += kWide) {
        half8 qw[kWide], xw[kUnr][kWide];
#pragma unroll
        for (int p = 0; p < kWide; ++p) {
          const int pp = min(p0 + p, np - 1);  // past the row: re-read the last piece, unused
          qw[p] = *(const half8*)(qb + pp * 128 + sub * 16);
#pragma unroll
          for (int u = 0; u < kUnr; ++u) xw[u][p] = __builtin_nontemporal_load((const half8*)(srcs[u] + pp * 128));
        }
#pragma unroll
        for (int p = 0; p < kWide; ++p)
          if (p0 + p < np)
#pragma unroll
            for (int u = 0; u < kUnr; ++u) wacc[u] = dot8(xw[u][p], qw[p], wacc[u]);
      }
    }
    // kAppendQ8: the 16 rows of this iteration lie in one 64-row block
    // (per-wave ranges start at multiples of 16); its meta comes through the
    // scalar cache.
    float cq = 0.f, slack = 0.f;
    if (Q8) {
      typedef const __attribute__((address_space(4))) float* cfloat_p;
      const int blk = __builtin_amdgcn_readfirstlane((int)(min(r0, n - 1) >> 6));
      const cfloat_p m = (cfloat_p)a.bmeta + 4 * (int64_t)blk;
      const float bs = m[0], bf = m[1], bx = m[2];
      cq = qm.x * bs;
      slack = (fmaf(qm.y, bf, qm.z * bx) + a.gamma * (qm.y + qm.z) * (bf + bx)) * (1.0f + 1.0f / 1048576.0f);
    }
#pragma unroll
    for (int u = 0; u < kUnr; ++u) {
      float acc = 0.f;
      if (Q8) {
        int ia = 0;
#pragma unroll
        for (int p = 0; p < PMAX; ++p)
          if (p < np) ia = dot16_i8(xv[u][p], qv[p], ia);
        ia += __shfl_xor(ia, 1);
        ia += __shfl_xor(ia, 2);
        ia += __shfl_xor(ia, 4);
        // upper bound of the exact score (kMaxQ8: the approximate score itself)
        acc = MODE == kMaxQ8 ? (float)ia * cq : fmaf((float)ia, cq, slack);
      } else {
        if (WIDE) acc = wacc[u];
#pragma unroll
        for (int p = 0; p < PMAX; ++p)
          if (p < np) acc = dot8(xv[u][p], qv[p], acc);
        acc += __shfl_xor(acc, 1);
        acc += __shfl_xor(acc, 2);
        acc += __shfl_xor(acc, 4);
      }
      const int64_t row = r0 + u * 8 + rg;
      const bool valid = row < r_end;
      if (MODE == kMax) {
        if (valid) umax = fmaxf(umax, acc);
      } else if (MODE == kMaxQ8) {
        if (valid && acc > umax) {
          umax = acc;
          uarg = (int)row;
        }
      } else {
        bool pass = valid && sub == 0 && acc >= thr;
        uint64_t mask = __ballot(pass);
        if (mask && Q8) {  // no compaction: a full list overflows (count > cap)
          const int nnew = __popcll(mask);
          if (pass && count + nnew <= a.cap) {
            const int pos = count + lanes_below(mask);
            lv[pos] = acc;
            li[pos] = (int)row;
          }
          count = (count + nnew <= a.cap) ? count + nnew : a.cap + 1;
        } else if (mask) {
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
  if (MODE == kMaxQ8) {  // the same units, each with its row (the first on ties)
    if (a.upb == 1) {
#pragma unroll
      for (int off = 8; off < kWave; off <<= 1) {
        const float om = __shfl_xor(umax, off);
        const int oa = __shfl_xor(uarg, off);
        if (om > umax || (om == umax && oa < uarg)) {
          umax = om;
          uarg = oa;
        }
      }
      if (lane == 0) {
        a.umax[gw] = umax;
        a.uarg[gw] = uarg;
      }
    } else if (sub == 0) {
      a.umax[(int64_t)gw * 8 + rg] = umax;
      a.uarg[(int64_t)gw * 8 + rg] = uarg;
    }
  }
  if (APP && lane == 0) a.lcount[gw] = count;
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

template <int PMAX>
hipError_t launch_q8(const GemvArgs& a, int grid, hipStream_t s) {
  if (a.mode == kMaxQ8)
    hipLaunchKernelGGL((gemv_kernel<PMAX, kMaxQ8>), dim3(grid), dim3(kBlock), 0, s, a);
  else
    hipLaunchKernelGGL((gemv_kernel<PMAX, kAppendQ8>), dim3(grid), dim3(kBlock), 0, s, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemv(const GemvArgs& a, int grid, hipStream_t s) {
  if (a.mode == kAppendQ8 || a.mode == kMaxQ8) {  // d = int8 row bytes
    if (a.qmeta == nullptr || a.bmeta == nullptr) return hipErrorInvalidValue;
    if (a.mode == kAppendQ8 && a.rows_per_wave % 16 != 0) return hipErrorInvalidValue;
    if (a.mode == kMaxQ8 && (a.umax == nullptr || a.uarg == nullptr || a.nsample < 1 || (a.upb != 1 && a.upb != 8) ||
                             a.units != a.nsample * a.upb))
      return hipErrorInvalidValue;
    if (a.d == 384) return launch_q8<3>(a, grid, s);
    if (a.d == 768) return launch_q8<6>(a, grid, s);
    if (a.d == 1536) return launch_q8<12>(a, grid, s);
    return hipErrorInvalidValue;
  }
  if (a.d <= 0 || a.d % 64 != 0) return hipErrorInvalidValue;
  if (a.d <= 384) return launch_p<6>(a, grid, s);
  if (a.d <= 768) return launch_p<12>(a, grid, s);
  if (a.d <= 1536) return launch_p<24>(a, grid, s);
  return launch_p<0>(a, grid, s);
}

}  // namespace cvs
