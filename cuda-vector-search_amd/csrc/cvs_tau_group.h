// The int8 pre-filter's threshold computed inside the int8 scan.
//
// tau_rescore_kernel (cvs_select.hip) derives each query's threshold from the
// int8 sampling pass in a launch of its own: a 256-bin histogram of the units'
// approximate maxima A picks the units of the fewest top bins holding >= k of
// them, their rows are rescored exactly (fp32 sums of the fp16 products, the
// final select's arithmetic) and tau is the k-th best of those scores: k real
// rows, so tau is at most the k-th best score of the search.
//
// tau_group() is the same computation for one query by one group of 256
// threads (4 waves) of a larger workgroup, on units the same launch publishes:
// every workgroup of the int8 scan first samples a few tiles of its chunk and
// stores one unit per (query, row half) as a 64-bit word ((row + 1) << 32 |
// bits(A)), with an agent-scope atomic store; waves 0-3 of workgroup b then
// take query b (the grid has at least one workgroup per query), waiting for
// the words of its units (agent-scope atomic loads, coherent across the XCDs'
// L2s).  The threshold is published the same way, one word per query,
// (1 << 32) | bits(tau), and every workgroup waits for the words of its
// queries before its first scanned tile.  Words of 0 mean "not yet": the
// query quantisation, which runs before the scan on the same stream, zeroes
// them.  Bounded waits: a unit still missing after `ticks` (kTauWaitTicks) of the
// 100 MHz constant clock (workgroups of the scan that were not resident
// together, e.g. on a GPU shared with other work) is left out, which leaves
// tau a lower bound of the k-th best score (it is the k-th best of real rows
// either way); a threshold word still 0 gives tau = -inf for that query.
// Both keep the search exact (every row a candidate at worst; lists that fill
// are rescanned by the select), only slower.
#pragma once

#include "cvs_common.h"

namespace cvs {

constexpr uint64_t kTauWaitTicks = 200000;  // 2 ms at 100 MHz

struct TauGroupShared {
  int hist[4][256];
  float mm[2][4];
  int sids[256];
  uint64_t ex[256];
  int nrow, nex, bstar, above;
};

// Query q (q < 0: none, the group only keeps step with the workgroup's
// barriers) from the unit words uw[q * units ..] (A and the companion row
// + 1), the fp16 query row qh + q * d and corpus xh (rows of d halfs, n of
// them), perm (companion row -> corpus row).  gt = thread in the group,
// 0..255; the group's first thread is a multiple of 64.  Every thread of the
// workgroup calls it (it holds workgroup barriers); requires units <= U * 256,
// k <= 256, d <= 8 * 16 * RL.
template <int U, int RL, int RU>
__device__ __forceinline__ void tau_group(TauGroupShared& L, int gt, int q, const unsigned long long* uw, int units,
                                          int k, const _Float16* qh, const _Float16* xh, int64_t n, int d,
                                          const int* perm, unsigned long long* tauw, float* tau_out, uint64_t ticks) {
  const int gl = gt & 63, gw = gt >> 6;
  float av[U];
  int row[U];
  float lo = __builtin_inff(), hi = -__builtin_inff();
#pragma unroll
  for (int u = 0; u < U; ++u) {
    av[u] = -__builtin_inff();
    row[u] = 0;
  }
  if (q >= 0) {
    const unsigned long long* src = uw + (int64_t)q * units;
    unsigned long long v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {  // unconditional clamped loads: they issue together
      const int i = u * 256 + gt;
      v[u] = __hip_atomic_load(&src[i < units ? i : units - 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // the units of workgroups still sampling: wait (bounded) for their words
    auto missing = [&]() {
      bool m = false;
#pragma unroll
      for (int u = 0; u < U; ++u) m |= u * 256 + gt < units && (v[u] >> 32) == 0;
      return m;
    };
    if (__any(missing())) {
      const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
      do {
        __builtin_amdgcn_s_sleep(2);
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int i = u * 256 + gt;
          if (i < units && (v[u] >> 32) == 0)
            v[u] = __hip_atomic_load(&src[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      } while (__any(missing()) && __builtin_amdgcn_s_memrealtime() - t0 <= ticks);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      av[u] = __uint_as_float((unsigned)v[u]);
      row[u] = (int)(v[u] >> 32) - 1;  // -1: missing
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {  // a unit counts when it has a row (A > -inf, row < n)
      const bool ok = u * 256 + gt < units && av[u] > -__builtin_inff() && row[u] >= 0 && row[u] < n;
      if (!ok) {
        av[u] = -__builtin_inff();
      } else {
        lo = fminf(lo, av[u]);
        hi = fmaxf(hi, av[u]);
      }
    }
  }
  for (int i = gt; i < 4 * 256; i += 256) (&L.hist[0][0])[i] = 0;
  if (gt == 0) {
    L.nrow = 0;
    L.nex = 0;
  }
  lo = wave_min_f32(lo);
  hi = wave_max_f32(hi);
  if (gl == 0) {
    L.mm[0][gw] = lo;
    L.mm[1][gw] = hi;
  }
  __syncthreads();
  lo = fminf(fminf(L.mm[0][0], L.mm[0][1]), fminf(L.mm[0][2], L.mm[0][3]));
  hi = fmaxf(fmaxf(L.mm[1][0], L.mm[1][1]), fmaxf(L.mm[1][2], L.mm[1][3]));
  // bin(A): non-decreasing, in [0, 255]
  const bool span = hi > lo && __builtin_isfinite(lo) && __builtin_isfinite(hi);
  const float scale = span ? 256.0f / (hi - lo) : 0.0f;
  auto bin = [&](float v) {
    const float t = (v - lo) * scale;
    return (int)(t >= 0.0f ? fminf(t, 255.0f) : 0.0f);
  };
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (av[u] > -__builtin_inff()) atomicAdd(&L.hist[gw][bin(av[u])], 1);
  __syncthreads();
  if (gw == 0) {  // the highest bin b whose bins >= b hold >= k units (bin 0 when fewer)
    int c[4];
    int sum = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {  // lane gl owns bins 255-4gl-j (descending)
      const int b = 255 - (4 * gl + j);
      c[j] = L.hist[0][b] + L.hist[1][b] + L.hist[2][b] + L.hist[3][b];
      sum += c[j];
    }
    int incl = wave_incl_sum_i32(sum);
    int run = incl - sum;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (run < k && k <= run + c[j]) L.bstar = 255 - (4 * gl + j);
      run += c[j];
    }
    if (gl == 63 && incl < k) L.bstar = 0;
  }
  __syncthreads();
  const int bstar = L.bstar;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (av[u] > -__builtin_inff() && bin(av[u]) >= bstar) {
      const int p = atomicAdd(&L.nrow, 1);
      if (p < 256) L.sids[p] = row[u];
    }
  }
  __syncthreads();
  const int mr = L.nrow < 256 ? L.nrow : 256;
  if (perm != nullptr && gt < mr) L.sids[gt] = perm[L.sids[gt]];  // companion rows -> corpus rows
  __syncthreads();
  // exact scores: 16 lanes per row, RU rows per 16-lane group at a time
  if (q >= 0) {
    const int l16 = gt & 15;
    const int nd = d / 8;
    half8 qv[RL];
    const half8* qr = reinterpret_cast<const half8*>(qh + (int64_t)q * d);
#pragma unroll
    for (int p = 0; p < RL; ++p) {
      const int c = l16 + 16 * p;
      qv[p] = c < nd ? qr[c] : half8{};
    }
    for (int c0 = (gt >> 4) * RU; c0 < mr; c0 += 16 * RU) {
      int idu[RU];
      half8 xv[RU][RL];
#pragma unroll
      for (int u = 0; u < RU; ++u) idu[u] = c0 + u < mr ? L.sids[c0 + u] : -1;
#pragma unroll
      for (int u = 0; u < RU; ++u) {
        const half8* xr = reinterpret_cast<const half8*>(xh + (int64_t)(idu[u] < 0 ? 0 : idu[u]) * d);
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
        if (l16 == 0 && idu[u] >= 0) L.ex[atomicAdd(&L.nex, 1)] = make_key(acc, idu[u]);
      }
    }
  }
  __syncthreads();
  // tau = the k-th largest exact key's score: the key with exactly k - 1 keys
  // above it (keys are unique: distinct rows)
  if (q >= 0) {
    const int m = L.nex;
    if (m < k) {
      if (gt == 0) {
        tau_out[q] = -__builtin_inff();
        __hip_atomic_store(&tauw[q], (1ull << 32) | (unsigned long long)__float_as_uint(-__builtin_inff()),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    } else if (gt < m) {
      const uint64_t mine = L.ex[gt];
      int rank = 0;
#pragma unroll 8
      for (int i = 0; i < m; ++i) rank += L.ex[i] > mine ? 1 : 0;
      if (rank == k - 1) {
        tau_out[q] = key_score(mine);
        __hip_atomic_store(&tauw[q], (1ull << 32) | (unsigned long long)__float_as_uint(key_score(mine)),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

// The published threshold of query q: waits (bounded) for its word.
__device__ __forceinline__ float tau_wait(const unsigned long long* tauw, int q, uint64_t ticks) {
  unsigned long long v = __hip_atomic_load(&tauw[q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if ((v >> 32) == 0) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (((v = __hip_atomic_load(&tauw[q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) >> 32) == 0) {
      __builtin_amdgcn_s_sleep(2);
      if (__builtin_amdgcn_s_memrealtime() - t0 > ticks) return -__builtin_inff();
    }
  }
  return __uint_as_float((unsigned)v);
}

}  // namespace cvs
