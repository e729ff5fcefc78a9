// Per-row int8 quantisation of a query, one wave per row (shared by the query
// quantisation kernel and the threshold select, which does it on the way).
// s = max|q| / 127, q~ = clip(rint(q * (127 / max)), -127, 127); meta = (s,
// s |q~|_2, |q - s q~|_2, 0) with the two norms rounded up (fp32 sums of at
// most 1536 terms: relative error < 2^-13, covered by the 2^-11 factor).
#pragma once

#include "cvs_common.h"

namespace cvs {

constexpr int kQ8RowPer = 24;  // d <= 1536 = 24 elements per lane

__device__ __forceinline__ signed char q8_quant(float v, float inv) {
  const float r = rintf(v * inv);
  return (signed char)fminf(127.f, fmaxf(-127.f, r));
}

// The row's elements for this lane: 8 consecutive ones per 512-element group
// g, [512 g + 8 lane, 512 g + 8 lane + 8), zero past d (d % 8 == 0, the row
// 16-byte aligned).  The three 16-byte loads are unconditional (clamped
// inside the row), so they issue together.
__device__ __forceinline__ void q8_load_row(const _Float16* src, int d, int lane, float (&v)[kQ8RowPer]) {
#pragma unroll
  for (int g = 0; g < kQ8RowPer / 8; ++g) {
    const int c = g * 8 * kWave + 8 * lane;
    const half8 h = *(const half8*)(src + (c < d ? c : d - 8));
#pragma unroll
    for (int j = 0; j < 8; ++j) v[8 * g + j] = c < d ? (float)h[j] : 0.f;
  }
}

// Fragment order of the int8 queries, the B operand of the 32x32x32 int8
// MFMA as the scans hold it: bytes [32 ks + 16 kg, +16) of query qi sit at
// this offset, KS = dq / 32 k-steps per row.  A wave's fragments of one
// k-step for 32 consecutive queries (lane = column + 32 kg) are then 1 KiB of
// contiguous memory, where the row layout spreads them over 32 rows.
__device__ __forceinline__ int64_t q8_frag_offset(int64_t qi, int ks, int kg, int KS) {
  return (((qi >> 5) * KS + ks) * 64 + (qi & 31) + 32 * kg) * 16;
}

// Whole wave, on the values q8_load_row loaded; `lane` = lane id.  dst holds
// dq >= d bytes (zero past d; dq % 32 == 0), written 8 bytes per lane; when
// frag is not null the same bytes also go to query qi's places in the
// fragment-ordered copy frag (q8_frag_offset).
__device__ __forceinline__ void q8_quantize_row(const float (&v)[kQ8RowPer], int d, int dq, signed char* dst,
                                                float4* meta, int lane, signed char* frag = nullptr,
                                                int64_t qi = 0) {
  constexpr float kNormUp = 1.0f + 1.0f / 2048.0f;
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < kQ8RowPer; ++i) m = fmaxf(m, fabsf(v[i]));
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  const float s = m / 127.f;
  const float inv = m > 0.f ? 127.f / m : 0.f;
  int sq = 0;  // sum of q~^2, exact (< 1536 * 127^2)
  float ee = 0.f;
#pragma unroll
  for (int g = 0; g < kQ8RowPer / 8; ++g) {
    const int c = g * 8 * kWave + 8 * lane;
    uint64_t packed = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const signed char qc = q8_quant(v[8 * g + j], inv);  // (0 past d: v is 0 there)
      const float e = fmaf(-s, (float)qc, v[8 * g + j]);
      sq += (int)qc * (int)qc;
      ee = fmaf(e, e, ee);
      packed |= (uint64_t)(uint8_t)qc << (8 * j);
    }
    if (c < dq) {
      *(uint64_t*)(dst + c) = packed;
      if (frag != nullptr) *(uint64_t*)(frag + q8_frag_offset(qi, c >> 5, (c >> 4) & 1, dq >> 5) + (c & 15)) = packed;
    }
  }
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    sq += __shfl_xor(sq, off);
    ee += __shfl_xor(ee, off);
  }
  if (lane == 0) {
    float4 mt;
    mt.x = s;
    mt.y = s * sqrtf((float)sq) * kNormUp;
    mt.z = sqrtf(ee) * kNormUp;
    mt.w = 0.f;
    *meta = mt;
  }
}

__device__ __forceinline__ void q8_query_row(const _Float16* src, int d, int dq, signed char* dst, float4* meta,
                                             int lane, signed char* frag, int64_t qi) {
  float v[kQ8RowPer];
  q8_load_row(src, d, lane, v);
  q8_quantize_row(v, d, dq, dst, meta, lane, frag, qi);
}

}  // namespace cvs
