// Shared device helpers for the gfx950 exact top-k engine.
//
// Candidate encoding: a (score, row id) pair is packed into one 64-bit key whose
// unsigned order is the search's total order: score descending, then id
// ascending (the order the reference emits, csrc/kernels.cu:277-279).  Keys are
// unique per query because row ids are, so "the k largest keys" is exactly the
// top-k, ties included.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cvs {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kBlock = 256;  // 4 waves, one per SIMD

// ---- 64-bit search keys ----------------------------------------------------

__device__ __forceinline__ uint32_t float_order(float v) {
  const uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float order_float(uint32_t o) {
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}

// The threshold for an order key found by a bit search truncated above its low
// bits: order_float(t), except that keys below float_order(-FLT_MAX) (those of
// -inf and of the NaNs past it, which a truncated search reaches when the k-th
// largest maximum is -inf) give -inf, a threshold every score passes.  A NaN
// threshold would pass none.
__device__ __forceinline__ float order_threshold(uint32_t t) {
  return t < 0x00800000u ? -__builtin_inff() : order_float(t);
}

__device__ __forceinline__ uint64_t make_key(float v, int id) {
  return ((uint64_t)float_order(v) << 32) | (uint64_t)(~(uint32_t)id);
}

__device__ __forceinline__ float key_score(uint64_t key) { return order_float((uint32_t)(key >> 32)); }
__device__ __forceinline__ int key_id(uint64_t key) { return (int)(~(uint32_t)key); }

// ---- reductions over aligned groups of 8 lanes (DPP, no LDS round trip) ----
// quad_perm [1,0,3,2] and [2,3,0,1] combine each quad; row_half_mirror (lane i
// of an 8-lane half-row reads lane 7-i) then combines the two quads.  Every
// lane of a group must be active.

__device__ __forceinline__ int sum8_i32(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);
  return v;
}

__device__ __forceinline__ uint32_t max8_u32(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
  return v;
}

// Smallest / largest of v over the wave (DPP within rows of 16 lanes, then the
// four rows' results by readlane; every lane must be active): quad_perm
// [1,0,3,2] and [2,3,0,1] combine each quad, row_half_mirror the two quads of a
// half-row, row_mirror the two halves of a row.  fminf / fmaxf: a NaN loses
// to any number.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_f32(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ float wave_min_f32(float v) {
  v = fminf(v, dpp_f32<0xB1>(v));
  v = fminf(v, dpp_f32<0x4E>(v));
  v = fminf(v, dpp_f32<0x141>(v));
  v = fminf(v, dpp_f32<0x140>(v));
  return fminf(fminf(lane_f32(v, 0), lane_f32(v, 16)), fminf(lane_f32(v, 32), lane_f32(v, 48)));
}
__device__ __forceinline__ float wave_max_f32(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x141>(v));
  v = fmaxf(v, dpp_f32<0x140>(v));
  return fmaxf(fmaxf(lane_f32(v, 0), lane_f32(v, 16)), fmaxf(lane_f32(v, 32), lane_f32(v, 48)));
}

// Inclusive prefix sum over the 64 lanes of a wave: row_shr 1, 2, 4 and 8
// within each row of 16 lanes (lanes shifted in from outside the row add 0),
// then row_bcast:15 adds the last lane of rows 0 and 2 to rows 1 and 3, and
// row_bcast:31 that of row 1 (the sum of rows 0-1 by then) to rows 2 and 3.
// Every lane must be active.
__device__ __forceinline__ int wave_incl_sum_i32(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);
  return v;
}

__device__ __forceinline__ uint32_t min8_u32(uint32_t v) {
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
  return v;
}

// ---- s_waitcnt encodings (gfx9 family: vmcnt is 6 bits split 3:0 / 15:14) ----

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (((N >> 4) & 3) << 14) | (7 << 4) | (15 << 8));
}

template <int N>
__device__ __forceinline__ void wait_vmcnt_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (((N >> 4) & 3) << 14) | (7 << 4));
}

// ---- HBM -> LDS DMA ---------------------------------------------------------

// 16 bytes per lane from `src` into LDS at lds_base + 16*lane (one 1 KB block
// per wave), bypassing VGPRs.  Issued through inline asm on purpose: the
// compiler's own LDS-DMA tracking cannot tell the stage buffers apart and
// would insert a full vmcnt(0) wait before every LDS read, serialising the
// pipeline.  Callers therefore own all waits (wait_vmcnt* + s_barrier) before
// reading a block.  `lds_base` must be wave-uniform.  NT marks the load
// non-temporal, for data streamed once per launch (the int8 corpus companion:
// keeping it out of the caches' retained lines leaves them to the fp16 rows
// that rescoring re-reads; 4-12 us less rescoring at 1M rows).  It is slower
// for fp16 scans, whose query groups share corpus lines through L2.  Callers
// load whole 128-byte lines.
template <bool NT>
__device__ __forceinline__ void dma_to_lds_16(const void* src, const void* lds_block) {
  const uint32_t base = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds_block);
  // m0 is restored afterwards: the compiler treats it as reserved.
  uint32_t saved;
  if (NT)
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "global_load_lds_dwordx4 %2, off nt\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(base), "v"(src)
        : "memory");
  else
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "global_load_lds_dwordx4 %2, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(base), "v"(src)
        : "memory");
}

// 16 bytes per lane from sbase + voff (lane's own offset) into LDS at
// lds + 16 * lane.  `sbase` and `lds` must be wave-uniform.  Non-temporal: the
// companion is streamed once per search.
__device__ __forceinline__ void dma16_saddr(uint32_t voff, const void* sbase, uint32_t lds) {
  // (readfirstlane returns int: each half goes through uint32_t, so the low
  // half is zero-extended, never sign-extended into the high half)
  const uint32_t m = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds);
  const uint64_t b = (uint64_t)(uintptr_t)sbase;
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
  const uint64_t sb = ((uint64_t)hi << 32) | (uint64_t)lo;
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "global_load_lds_dwordx4 %2, %3 nt\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(m), "v"(voff), "s"(sb)
      : "memory");
}

// ---- register placement -----------------------------------------------------

// Returns `v` materialised in accumulation registers (AGPRs).  MFMA source
// operands may live in AGPRs on gfx950, so long-lived MFMA inputs (the query
// fragments) are pinned there, leaving the VGPRs to the streaming operands.
// The asm emits no instruction; only the register-class constraint matters.
__device__ __forceinline__ half8 pin_agpr(half8 v) {
  half8 r = v;
  asm volatile("" : "+a"(r));
  return r;
}

typedef int i32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ i32x4 pin_agpr(i32x4 v) {
  i32x4 r = v;
  asm volatile("" : "+a"(r));
  return r;
}

// ---- MFMA scan helpers --------------------------------------------------------

// Wait states between a tile's last MFMA and the epilogue's first VALU read of
// its accumulators.  gfx950 needs passes + 4 for a VALU read of an MFMA's VGPR
// result; with the accumulators in VGPRs (-amdgpu-mfma-vgpr-form) this
// compiler leaves only passes + 3 between them, and the epilogue then reads a
// partial sum (the score matrix intermittently lacked the last k-step).  The
// pad is 2 * passes + 3, tied to the accumulator so that it follows the last
// MFMA; the build checks every MFMA result read of the scan kernels against
// passes + 4 (hazard_check.py).
template <int PASSES, class T>
__device__ __forceinline__ void pad_mfma_result(T& acc) {
  constexpr int WS = 2 * PASSES + 3;
  static_assert(WS > 8 && WS <= 24, "pad of 9..24 wait states");
  if constexpr (WS > 16)
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop %1" : "+v"(acc) : "n"(WS - 17));
  else
    asm volatile("s_nop 7\n\ts_nop %1" : "+v"(acc) : "n"(WS - 9));
}

// Piece permutation of corpus stages in LDS: slot s of a stage row R holds
// 16-byte piece s ^ piece_swz(R), so the 8 (and 16) consecutive rows whose
// equal-index pieces one MFMA fragment's lanes read fall on distinct banks.
__device__ __forceinline__ int piece_swz(int r) { return ((r >> 1) ^ ((r & 1) << 2)) & 7; }

// ---- wave utilities ---------------------------------------------------------

__device__ __forceinline__ int lane_id() { return (int)__lane_id(); }

// Number of set bits of `mask` below this lane.
__device__ __forceinline__ int lanes_below(uint64_t mask) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                        __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

__device__ __forceinline__ float coherent_load(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int coherent_load(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Sorts keys[0..N) descending in LDS; N is a power of two.  Called by one whole
// wave; LDS operations of a wave are performed in issue order, and the
// wavefront fence keeps the compiler from reordering them across stages.
__device__ __forceinline__ void wave_lds_sort_desc(uint64_t* keys, int N) {
  const int lane = lane_id();
#pragma unroll 1
  for (int size = 2; size <= N; size <<= 1) {
#pragma unroll 1
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
#pragma unroll 1
      for (int i = lane; i < (N >> 1); i += kWave) {
        const int lo = ((i & ~(stride - 1)) << 1) | (i & (stride - 1));
        const int hi = lo + stride;
        const bool desc = ((lo & size) == 0);
        const uint64_t a = keys[lo], b = keys[hi];
        if (desc ? (a < b) : (a > b)) {
          keys[lo] = b;
          keys[hi] = a;
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    }
  }
}

// Shrinks one candidate list (owned by the calling wave; `count` entries at
// lv/li) to its k best entries, in place, and returns the score of the k-th
// best: a lower bound on the k-th best score of everything the list has been
// offered, hence a valid filter for later candidates.  `scratch` is this wave's
// private LDS area of at least next_pow2(count) keys.  Called by all 64 lanes
// with identical arguments.  Requires 1 <= k <= count.
__device__ __forceinline__ float wave_compact(float* lv, int* li, int count, int k, uint64_t* scratch) {
  const int lane = lane_id();
  // The list was written by this wave's own global stores: wait for them, and
  // read it back past the (non-coherent) vector L1.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  int N = 2;
  while (N < count) N <<= 1;
#pragma unroll 1
  for (int p = lane; p < N; p += kWave)
    scratch[p] = (p < count) ? make_key(coherent_load(lv + p), coherent_load(li + p)) : 0ull;
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  wave_lds_sort_desc(scratch, N);
#pragma unroll 1
  for (int p = lane; p < k; p += kWave) {
    const uint64_t key = scratch[p];
    lv[p] = key_score(key);
    li[p] = key_id(key);
  }
  const float kth = key_score(scratch[k - 1]);
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  // Retire this rare path's own loads here, so the (hot) caller's loop does not
  // inherit pending VGPR writes and wait on vmcnt(0) in every iteration.
  wait_vmcnt<0>();
  return kth;
}

}  // namespace cvs
