// Q-stationary MFMA scan: scores one query group against a run of corpus tiles.
//
// Replaces the score tile + fused top-k of csrc/kernels.cu:123-177 and
// kernels.cu:313-371 (and the score kernel, kernels.cu:285-311), re-designed
// for gfx950:
//
//  * 256 threads = 4 wave64s, one per SIMD (QS <= 4), or 512 threads = 8
//    wave64s, two per SIMD (QS = 8).  Queries are split QS ways across the
//    waves and tile rows RS = 4/QS ways.  Each wave keeps its QW = MS*QB
//    queries as MFMA B fragments in registers (AGPRs) for the whole launch
//    (loaded once), so the corpus is the only operand that streams.
//  * MFMA shape MS = 32 (v_mfma_f32_32x32x16_f16) wherever the query block
//    allows it: on gfx950 it runs at the full dense fp16 rate, twice the
//    throughput of v_mfma_f32_16x16x32_f16, which is kept (MS = 16) for batch
//    <= 16 and for rows wider than 768.
//  * Corpus rows stream HBM -> LDS with global_load_lds_dwordx4 (no VGPR
//    staging), in 64-column (128-byte) stages, each load reading 8 whole
//    128-byte lines; the rows' 16-byte pieces are permuted in LDS so that the
//    ds_read_b128s feeding the MFMAs are free of bank conflicts.  NBUF stages
//    are in flight (40-56 KB per CU); waits are explicit vmcnt counts.
//  * Scores never leave VGPRs.  kAppend filters them against a per-query
//    threshold (from the sampling pre-pass): a lane whose block maximum passes
//    copies its whole row of scores to an LDS staging area (a few ds_writes,
//    independent of how many scores pass); the staging area is flushed into
//    per-wave candidate lists in global memory only when it fills and at the
//    end, and that flush is where lists that overflow get compacted to their
//    k best.  The exact top-k is taken later by the select kernel.  kMax
//    records per-unit maxima for the sampling pre-pass; kStore* writes the full
//    score matrix (Index.scores / twopass).
//
// MFMA layouts (A = corpus rows, B = queries; any consistent k-permutation of
// A and B gives the same dot products, so only the D layout is load-bearing):
//   16x16x32: lane l supplies A[l%16][8(l/16)..+7], B[8(l/16)..+7][l%16] and
//             receives D[4(l/16)+i][l%16], i = 0..3.
//   32x32x16: lane l supplies A[l%32][8(l/32)..+7], B[8(l/32)..+7][l%32] and
//             receives D[8i+4(l/32)+j][l%32], i, j = 0..3 (element 4i+j).
#include <climits>

#include "cvs_common.h"
#include "cvs_kernels.h"
#include "cvs_q8_row.h"
#include "cvs_tau_group.h"

namespace cvs {

namespace {

// Wave-wide maximum and minimum (every lane active): the 8-lane DPP
// reductions, the other half of each 16-lane row by row_mirror, then the
// four rows' lanes 0 through readlane (no LDS round trip).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max8_u32(v);
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
  return max(max((uint32_t)__builtin_amdgcn_readlane((int)v, 0), (uint32_t)__builtin_amdgcn_readlane((int)v, 16)),
             max((uint32_t)__builtin_amdgcn_readlane((int)v, 32), (uint32_t)__builtin_amdgcn_readlane((int)v, 48)));
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  v = min8_u32(v);
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
  return min(min((uint32_t)__builtin_amdgcn_readlane((int)v, 0), (uint32_t)__builtin_amdgcn_readlane((int)v, 16)),
             min((uint32_t)__builtin_amdgcn_readlane((int)v, 32), (uint32_t)__builtin_amdgcn_readlane((int)v, 48)));
}

// Mode kAppendIn, threshold workgroups: query q's threshold by one wave from
// its su_units sampling units (words (1 << 32) | float_order(exact maximum) of
// disjoint row sets; 0 = not yet published), at most 64 * UPL of them.  The
// k-th largest unit key, found by the threshold select's bit search stopped
// above the 12 low bits: a lower bound of the k-th largest unit, hence of the
// query's k-th best score (k distinct rows score at least that much), at most
// 2^-11 of the score below the unit.  Units still missing after `ticks` of the
// 100 MHz clock are left out (fewer units: a lower threshold, still exact);
// fewer than k present give -inf.  Published as (1 << 32) | bits(tau).
template <int UPL>
__device__ __forceinline__ void wave_unit_threshold(const ScanArgs& a, int q, int lane, uint64_t ticks) {
  constexpr int kThrLowBits = 12;
  const int U = a.su_units;
  const unsigned long long* src = a.su_w + (int64_t)q * U;
  unsigned long long v[UPL];
#pragma unroll
  for (int j = 0; j < UPL; ++j) {  // unconditional clamped loads: they issue together
    const int i = lane + kWave * j;
    v[j] = __hip_atomic_load(&src[i < U ? i : U - 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  auto missing = [&]() {
    bool m = false;
#pragma unroll
    for (int j = 0; j < UPL; ++j) m |= lane + kWave * j < U && (v[j] >> 32) == 0;
    return m;
  };
  if (__any(missing())) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    do {
      __builtin_amdgcn_s_sleep(2);
#pragma unroll
      for (int j = 0; j < UPL; ++j) {
        const int i = lane + kWave * j;
        if (i < U && (v[j] >> 32) == 0) v[j] = __hip_atomic_load(&src[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    } while (__any(missing()) && __builtin_amdgcn_s_memrealtime() - t0 <= ticks);
  }
  // (wave-wide counts as the popcounts of ballots: no cross-lane reduction)
  uint32_t key[UPL], hi = 0u, lo = ~0u;
  int have = 0;
#pragma unroll
  for (int j = 0; j < UPL; ++j) {
    const bool h = lane + kWave * j < U && (v[j] >> 32) != 0;
    key[j] = h ? (uint32_t)v[j] : 0u;  // missing: below every unit
    hi = max(hi, key[j]);
    if (h) lo = min(lo, key[j]);
    have += __popcll(__ballot(h));
  }
  hi = wave_max_u32(hi);
  lo = wave_min_u32(lo);
  uint32_t tk = 0u;  // order key 0: threshold -inf
  if (have >= a.k) {
    // tk starts at the bits every present key shares (at most the smallest of
    // them, so at least k keys reach it) and keeps count(key >= tk) >= k
    const uint32_t diff = hi ^ lo;
    const int top = diff ? 31 - __builtin_clz(diff) : -1;
    tk = (top < 0 ? hi : hi & ~((2u << top) - 1u)) & ~((1u << kThrLowBits) - 1u);
    for (int bit = top; bit >= kThrLowBits; --bit) {
      const uint32_t cand = tk | (1u << bit);
      int c = 0;
#pragma unroll
      for (int j = 0; j < UPL; ++j) c += __popcll(__ballot(key[j] >= cand));
      if (c >= a.k) tk = cand;
    }
  }
  const float tv = order_threshold(tk);
  if (lane == 0) {
    if (a.tau_out != nullptr) a.tau_out[q] = tv;
    __hip_atomic_store(&a.tauw[q], (1ull << 32) | (unsigned long long)__float_as_uint(tv), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <int MS>
struct Mfma;

template <>
struct Mfma<16> {
  typedef f32x4 acc_t;
  static constexpr int KSZ = 32;  // k per instruction
  static constexpr int NE = 4;    // accumulator elements per lane
  static constexpr int PASSES = 4;  // 16 cycles on gfx950
  __device__ static acc_t run(half8 a, half8 b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  // row (within the 16-row block) of accumulator element e, minus 4*(lane/16)
  __device__ static constexpr int row(int e) { return e; }
};

template <>
struct Mfma<32> {
  typedef float acc_t __attribute__((ext_vector_type(16)));
  static constexpr int KSZ = 16;
  static constexpr int NE = 16;
  static constexpr int PASSES = 8;  // 32 cycles on gfx950
  __device__ static acc_t run(half8 a, half8 b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  // row (within the 32-row block) of element e = 4i+j, minus 4*(lane/32)
  __device__ static constexpr int row(int e) { return 8 * (e >> 2) + (e & 3); }
};

// int8 pre-filter: v_mfma_i32_32x32x32_i8.  Operands are the same 16 bytes per
// lane as for 32x32x16_f16 (lane l: row l%32, bytes 16(l/32)..+15 of a 32-byte
// k-step), so the kernel's byte addressing is unchanged: it runs on int8 rows
// with d counted in 2-byte units.  Same D layout as Mfma<32>.
struct MfmaI8 {
  typedef int acc_t __attribute__((ext_vector_type(16)));
  static constexpr int KSZ = 16;  // 2-byte units per k-step (32 int8)
  static constexpr int NE = 16;
  static constexpr int PASSES = 8;
  __device__ static acc_t run(half8 a, half8 b, acc_t c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, a), __builtin_bit_cast(i32x4, b),
                                                  c, 0, 0, 0);
  }
  __device__ static constexpr int row(int e) { return Mfma<32>::row(e); }
};

template <int MS, int MODE>
struct MfmaFor {
  typedef Mfma<MS> type;
};
template <>
struct MfmaFor<32, kAppendQ8> {
  typedef MfmaI8 type;
};
template <>
struct MfmaFor<32, kMaxQ8> {
  typedef MfmaI8 type;
};

// FULLW: the row width is exactly KSMAX * KSZ, so the stage count is a
// compile-time constant (per-stage guards on a runtime count split the
// unrolled stage loop into separate blocks and cost ~15% of the scan).
// Stage buffers hold TR rows x 128 bytes (64 halfs), row-major.  A DMA load
// fills 1 KB = 8 rows: lane l fetches a 16-byte piece of row l/8 into slot l%8,
// so every load reads 8 whole 128-byte lines.  Slot s of row R holds piece
// s ^ piece_swz(R): the 8 (and 16) consecutive rows whose equal-index pieces
// the lanes of one fragment read then fall on distinct LDS banks.

template <int MS, int QS, int QB, int RB, int KSMAX, int MODE, bool FULLW>
__global__ __launch_bounds__(scan_waves(QS) * kWave, 1) void scan_kernel(ScanArgs a) {
  constexpr bool Q8 = (MODE == kAppendQ8 || MODE == kMaxQ8);  // int8 rows and queries
  static_assert(!Q8 || MS == 32, "int8 pre-filter uses the 32x32 MFMA");
  static_assert(!Q8 || (MS * RB <= 64 && 64 % (MS * RB) == 0),
                "int8 pre-filter: a wave's rows of a tile must lie in one 64-row block (one meta entry)");
  typedef typename MfmaFor<MS, MODE>::type M;
  typedef typename M::acc_t acc_t;
  constexpr int RS = scan_row_splits(QS);  // row splits
  constexpr int NW = QS * RS;       // waves: 4 (one per SIMD) or 8 (two per SIMD)
  constexpr int NT = NW * kWave;
  constexpr int QW = MS * QB;        // queries per wave
  constexpr int BQ = QS * QW;        // queries per workgroup
  constexpr int RW = MS * RB;        // rows per wave per tile
  constexpr int TR = RS * RW;        // tile rows
  constexpr int KSL = 64 / M::KSZ;   // MFMA k-steps per 128-byte line of a row
  // TS (24 KB stages of the 8-wave int8 scans, 64-row tiles of 3k 128-byte
  // lines per row): a stage is 3 lines of every row of the tile (the whole
  // tile for 384-byte rows, half of it for 768-byte rows), and every 1 KB DMA
  // load reads 8 stage lines, runs of up to 384 consecutive bytes of global
  // memory (measured: HBM -> LDS at 6.5 TB/s against 5.4 TB/s for stages of
  // one 128-byte line per row, whose loads read 8 lines a row apart; the
  // 768-byte-row scan of C4 253.6 -> 237.0 us with two barriers per tile
  // instead of six).  Otherwise a stage is one line (64 columns) of every row.
  constexpr bool TS = FULLW && Q8 && NW == 8 && TR == 64 && (KSMAX / KSL) % 3 == 0;
  constexpr int LPR = TS ? 3 : 1;  // lines per row in a stage
  constexpr int KPS = LPR * KSL;     // MFMA k-steps per stage
  constexpr int TRB = TR / MS;       // MS-row blocks per tile
  constexpr int FC = TR * LPR / 8;   // 1 KB DMA loads (8 lines of 128 bytes) of corpus rows per stage
  static_assert(TRB * KSL * 8 == TR, "an MS-row block is MS lines of 128 bytes");
  // QL (KSMAX == 0, rows of any width): the queries are not held in registers
  // but ride in every stage beside the corpus rows, QA rows of 128 bytes (the
  // query block padded so every wave issues the same number of loads), and the
  // MFMAs read both operands from LDS.
  constexpr bool QL = (KSMAX == 0);
  constexpr int QA = QL ? ((BQ + 8 * NW - 1) / (8 * NW)) * (8 * NW) : 0;
  constexpr int FPS = FC + QA / 8;   // 1 KB DMA loads per stage
  static_assert(FPS % NW == 0, "every wave must issue the same number of stage loads");
  static_assert(!QL || (!FULLW && !Q8), "queries in LDS: fp16 rows of a runtime width");
  constexpr int LPW = FPS / NW;      // stage loads per wave
  constexpr int STAGE = FPS * 1024;
  constexpr int NBUF = ((QS >= 4 ? 56 : 40) * 1024) / STAGE + 2;
  static_assert((NBUF - 2) * LPW < 64 && NBUF >= 3, "vmcnt budget / pipeline depth");
  constexpr int NCMAX = KSMAX / KPS; // 64-column stages per tile (max)
  // One barrier per two stages when every tile has the same, even stage count.
  constexpr bool PAIR = FULLW && (NCMAX % 2 == 0) && NBUF >= 5;
  constexpr int G = kWave / MS;      // lane groups sharing a query column
  constexpr int NV = RB * M::NE;     // scores per lane per query block per tile
  constexpr bool TOPK = (MODE == kTopK);
  constexpr bool SIN = (MODE == kAppendIn);  // fp16 append with its own sampling and thresholds
  // kAppendIn, one wave per SIMD (registers to spare): tiles whose MFMAs run
  // before the thresholds are known, their scores held in registers
  constexpr int DEFER = (SIN && NW == 4) ? 3 : 1;
  constexpr bool APP = (MODE == kAppend || MODE == kAppendQ8 || SIN);
  static_assert(!TOPK || (QB == 1 && MS == 32), "running top-k: one 32-query block per wave");
  constexpr bool SMAX = (MODE == kMax || MODE == kMaxQ8);  // sample passes
  constexpr int STCAP = 64;          // staged entries per wave
  // A staged entry is one lane's NE scores of one (query block, row block): a
  // row of EST floats (NE plus padding to an odd number of 16-byte units, so
  // that ds_write/read_b128 of 16 consecutive entries hit distinct banks).
  constexpr int EST = ((M::NE / 4) | 1) * 4;
  // Pin the query fragments to AGPRs when they dominate the register budget.
  constexpr bool PIN_Q = QB * KSMAX * 4 >= 128 || NW == 8;

  __shared__ __attribute__((aligned(1024))) unsigned char smem[NBUF * STAGE];
  __shared__ int lcnt[RS][BQ];                        // entries in each owned list
  __shared__ uint32_t thr_k[TOPK ? BQ : 1];           // kTopK: the workgroup's per-query k-th best so far (order key)
  __shared__ float thr_s[APP ? RS : 1][BQ];           // per-query filter threshold
  __shared__ float mred[MODE == kMax ? RS : 1][BQ];    // kMax, agg 2: maxima of the row splits
  __shared__ __attribute__((aligned(16))) float st_val[APP ? NW : 1][APP ? STCAP * EST : 1];  // staged entries
  __shared__ int st_meta[APP ? NW : 1][APP ? 2 * STCAP : 1];  // (query, first row) per entry
  __shared__ uint64_t sortbuf[(MODE == kAppend || SIN) ? NW * kMaxCap : 1];  // compaction scratch (int8 lists never compact)
  // kStore*: each wave's [QW queries][RW rows] score tile, written out one query
  // row at a time by consecutive lanes (coalesced); rows padded by 4 elements.
  constexpr bool STORE = (MODE == kStoreF32 || MODE == kStoreF16);
  constexpr int SROW = RW + 4;
  __shared__ __attribute__((aligned(16))) float stg[STORE ? NW : 1][STORE ? QW * SROW : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int qs = w % QS;
  const int rs = w / QS;
  // kAppendIn: bound of each cross-workgroup wait (100 MHz ticks; 0 only in
  // tests, where every wait not satisfied at once gives up), and the grid's
  // workgroups past the scan's chunks: each wave takes one query's threshold.
  const uint64_t wait_ticks = a.no_wait ? 0 : kTauWaitTicks;
  if constexpr (SIN) {
    if ((int)blockIdx.x >= a.groups * a.nchunks) {
      const int q = ((int)blockIdx.x - a.groups * a.nchunks) * NW + w;
      if (q < a.nq) {  // (8-wave kernels: at most 512 units, so that the registers suffice)
        if (NW == 8 || a.su_units <= kWave * 8)
          wave_unit_threshold<8>(a, q, lane, wait_ticks);
        else if (a.su_units <= kWave * 16)
          wave_unit_threshold<16>(a, q, lane, wait_ticks);
        else
          wave_unit_threshold<32>(a, q, lane, wait_ticks);
      }
      return;
    }
  }
  const int col = lane % MS;  // query column of this lane / A-fragment row
  const int kg = lane / MS;   // k-group of this lane (0..G-1)

  // Workgroup -> (query group, chunk).  With xcd_pair, consecutive workgroups on
  // one XCD (ids i, i+8, ...) take the query groups of one chunk so that its
  // corpus rows are fetched from HBM once and re-read from that XCD's L2.
  int grp, chunk;
  {
    const int id = blockIdx.x;
    if (a.xcd_pair) {  // (kMax: chunk = sampling workgroup, nsample % 8 == 0)
      const int slot = id >> 3;
      grp = slot % a.groups;
      chunk = (slot / a.groups) * 8 + (id & 7);
    } else {
      grp = id % a.groups;
      chunk = id / a.groups;
    }
  }
  int64_t t_begin, t_end;
  if (SMAX) {  // spt consecutive tiles centred on an evenly spread position
    const int64_t centre = ((2 * (int64_t)chunk + 1) * a.ntiles) / (2 * (int64_t)a.nsample);
    t_begin = centre - a.spt / 2;
    if (t_begin > a.ntiles - a.spt) t_begin = a.ntiles - a.spt;
    if (t_begin < 0) t_begin = 0;
    t_end = t_begin + a.spt;
  } else {
    t_begin = (int64_t)chunk * a.tpc;
    t_end = t_begin + a.tpc < a.ntiles ? t_begin + a.tpc : a.ntiles;
  }

  const int d = a.d;
  const int nc = FULLW ? NCMAX : (d >> 6);
  const int64_t n = a.n;
  const int qwave0 = grp * BQ + qs * QW;

  // Stage issue cursor (runs NBUF-1 stages ahead of the compute cursor).  Stages
  // past the end of this workgroup's range load a clamped, valid row so every
  // wave always has the same number of loads in flight.
  int64_t it_t = t_begin;
  int it_c = 0;
  int it_buf = 0;
  // Per-lane source of each of this wave's stage loads (row, and the address
  // of its first 64-column stage), advanced incrementally.
  const _Float16* src[LPW];
  int64_t src_row[LPW];
  int poff[LPW];  // this lane's 16-byte piece of its row, in halfs
  bool qload[LPW];  // QL: this (wave-uniform) load fetches query rows, the same every tile
#pragma unroll
  for (int j = 0; j < LPW; ++j) {
    const int f = w + NW * j;
    qload[j] = QL && f >= FC;
    if (qload[j]) {  // query-area row ql: query grp*BQ + ql (padding rows re-read the last query)
      const int ql = (f - FC) * 8 + (lane >> 3);
      poff[j] = ((lane & 7) ^ piece_swz(ql)) * 8;
      src_row[j] = -1;  // never clamped
      src[j] = a.q + (int64_t)min(grp * BQ + ql, a.nq - 1) * d + poff[j];
    } else {
      // line L of the stage: row L / LPR of the tile, its line L % LPR
      const int L = f * 8 + (lane >> 3);
      const int rl = L / LPR;
      poff[j] = (L % LPR) * 64 + ((lane & 7) ^ piece_swz(rl)) * 8;
      src_row[j] = t_begin * TR + rl;
      src[j] = a.x + src_row[j] * d + poff[j];
    }
  }
  // TS: the int8 companion holds whole 64-row blocks, so a tile's rows are
  // TR * row-bytes contiguous bytes that all exist (rows past n are padding,
  // never reported): each load is a scalar tile base plus a constant lane
  // offset, without the per-load address registers and clamps below.
  uint32_t voff_ts[TS ? LPW : 1];
  if constexpr (TS) {
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
      const int L = (w + NW * j) * 8 + (lane >> 3);
      const int rl = L / LPR;
      voff_ts[j] = (uint32_t)(rl * 2 * d + (L % LPR) * 128 + (((lane & 7) ^ piece_swz(rl)) << 4));
    }
  }
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)smem);
  auto issue_next = [&]() {
    if constexpr (TS) {
      const int64_t tt = it_t < a.ntiles ? it_t : a.ntiles - 1;
      const unsigned char* base =
          reinterpret_cast<const unsigned char*>(a.x) + tt * (TR * 2 * (int64_t)d) + it_c * (LPR * 128);
      const uint32_t lds = lds0 + (uint32_t)(it_buf * STAGE + w * 1024);
#pragma unroll
      for (int j = 0; j < LPW; ++j) dma16_saddr(voff_ts[j], base, lds + (uint32_t)(j * NW * 1024));
      if (++it_c == nc) {
        it_c = 0;
        ++it_t;
      }
      if (++it_buf == NBUF) it_buf = 0;
      return;
    }
    unsigned char* buf = smem + it_buf * STAGE;
    const bool whole = (it_t + 1) * TR <= n;  // every row of this tile exists
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
      const int f = w + NW * j;
      const _Float16* p = src[j] + it_c * (64 * LPR);
      if (!whole && src_row[j] >= n) p = a.x + (n - 1) * d + it_c * (64 * LPR) + poff[j];
      dma_to_lds_16<Q8>(p, buf + f * 1024);
    }
    if (++it_c == nc) {
      it_c = 0;
      ++it_t;
#pragma unroll
      for (int j = 0; j < LPW; ++j) {
        if (!qload[j]) {
          src[j] += (int64_t)TR * d;
          src_row[j] += TR;
        }
      }
    }
    if (++it_buf == NBUF) it_buf = 0;
  };
  issue_next();  // stage 0 first: its latency overlaps the query loads'

  // Query fragments (B operand), resident for the whole launch.  The loads are
  // unconditional so that they issue back to back (a per-load lane mask puts
  // each behind a wait for the previous one): a column past nq loads query
  // nq-1 (its scores are never reported: its threshold is +inf and kMax skips
  // it), a k-step past d loads the last one (the stage loop never uses it).
  half8 qf[QB][QL ? 1 : KSMAX];
  if constexpr (!QL) {
    half8 ld[QB][KSMAX];
    const int ksl = d / M::KSZ - 1;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int qi = min(qwave0 + qb * MS + col, a.nq - 1);
#pragma unroll
      for (int ks = 0; ks < KSMAX; ++ks) {
        if constexpr (Q8)  // full-width int8 rows (KSMAX k-steps): the fragment-ordered copy, 1 KiB per load
          ld[qb][ks] = *(const half8*)(a.qf + q8_frag_offset(qi, ks, kg, KSMAX));
        else if constexpr (SIN)  // the fp16 fragment-ordered copy, the same layout
          ld[qb][ks] = *(const half8*)(reinterpret_cast<const char*>(a.qfh) + q8_frag_offset(qi, ks, kg, KSMAX));
        else
          ld[qb][ks] = *(const half8*)(a.q + (int64_t)qi * d + min(ks, ksl) * M::KSZ + kg * 8);
      }
    }
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int ks = 0; ks < KSMAX; ++ks) qf[qb][ks] = ld[qb][ks];  // pinned after the prologue wait
  }

  float thr[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int qi = qwave0 + qb * MS + col;
    thr[qb] = (qi >= a.nq) ? __builtin_inff() : (a.tau ? a.tau[qi] : -__builtin_inff());
  }
  // kAppendQ8: this lane's queries' (s_q, |q^|, |e|), for the score bound.
  float4 qm[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    if (Q8) qm[qb] = a.qmeta[min(qwave0 + qb * MS + col, a.nq - 1)];
    else qm[qb] = float4{0.f, 0.f, 0.f, 0.f};
  }
  // kAppend from sampling maxima (small batches): each query's threshold is the
  // k-th largest of its units_in <= 64 maxima, found by 8 lanes of 8 maxima
  // each (below, once the prologue's loads have retired).  The maxima load here
  // beside the other prologue loads: unconditionally, from clamped addresses, so
  // that they issue back to back.
  constexpr bool TIN = (MODE == kAppend) && (BQ <= NT / 8);
  const bool thr_in = TIN && a.umax_in != nullptr;
  float kraw[TIN ? 8 : 1];
  if constexpr (TIN) {
    if (thr_in) {
      const int qi = min(grp * BQ + min(tid >> 3, BQ - 1), a.nq - 1);
      const float* src = a.umax_in + (int64_t)qi * a.units_in;
#pragma unroll
      for (int j = 0; j < 8; ++j) kraw[j] = src[min((tid & 7) + 8 * j, a.units_in - 1)];
    }
  }
  if (APP || TOPK) {
    for (int i = tid; i < RS * BQ; i += NT) {
      (&lcnt[0][0])[i] = 0;
      const int qi = grp * BQ + i % BQ;
      if (!thr_in) (&thr_s[0][0])[i] = (qi >= a.nq) ? __builtin_inff() : (a.tau ? a.tau[qi] : -__builtin_inff());
    }
  }
  // kTopK: this lane's running top-k of each query block in the last k of
  // TK slots, descending (the first TK - k slots are parked at +inf, so the
  // k-th best is always the last slot; real slots not yet filled hold -inf
  // and row -1), and the workgroup's threshold: the largest k-th best of any
  // lane holding the query, a lower bound of the workgroup's own k-th best
  // (that lane has k scores at or above it).
  constexpr int TK = TOPK ? 16 : 1;
  float tkv[QB][TK];
  int tki[QB][TK];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb)
#pragma unroll
    for (int j = 0; j < TK; ++j) {
      tkv[qb][j] = j < TK - a.k ? __builtin_inff() : -__builtin_inff();
      tki[qb][j] = -1;
    }
  if constexpr (TOPK) {
    for (int i = tid; i < RS * BQ; i += NT) (&lcnt[0][0])[i] = 0;
    for (int i = tid; i < BQ; i += NT) thr_k[i] = float_order(-__builtin_inff());
  }
  int st_n = 0;  // wave-uniform count of staged lane-rows
  float umx[QB];  // kMax / kMaxQ8 with agg: this lane's unit maxima over all sampled tiles
  int uag[QB];    // kMaxQ8 with agg: their rows
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    umx[qb] = -__builtin_inff();
    uag[qb] = 0;
  }

  // Appends the passing scores of this wave's staged entries to its global
  // candidate lists.  A list that fills up is compacted to its k best entries
  // (raising that query's threshold) and the remaining scores are retried.
  auto flush = [&]() {
    const int list = chunk * RS + rs;
#pragma unroll 1
    for (int base = 0; base < st_n; base += kWave) {
      const int er = base + lane;
      const bool have = er < st_n;
      const int ers = have ? er : 0;
      const int ql = have ? st_meta[w][2 * er] : 0;
      const int rbase = have ? st_meta[w][2 * er + 1] : 0;
      float ev[M::NE];
#pragma unroll
      for (int c = 0; c < M::NE / 4; ++c) {
        const f32x4 t = *(const f32x4*)(&st_val[w][ers * EST + 4 * c]);
        ev[4 * c] = t[0];
        ev[4 * c + 1] = t[1];
        ev[4 * c + 2] = t[2];
        ev[4 * c + 3] = t[3];
      }
      const int64_t lbase = ((int64_t)(grp * BQ + ql) * a.nlists + list) * a.cap;
      unsigned todo = 0;  // scores of this entry not yet appended
      if (have) {
        const float tq = thr_s[rs][ql];
#pragma unroll
        for (int e = 0; e < M::NE; ++e)  // (rows past n of the last tile are -inf: never appended)
          todo |= (ev[e] >= tq && rbase + M::row(e) < n ? 1u : 0u) << e;
      }
#pragma unroll 1
      while (true) {
        const int cnt = __popc(todo);
        const int pos = cnt ? atomicAdd(&lcnt[rs][ql], cnt) : 0;
        const int room = a.cap - pos;
        int put = 0;
#pragma unroll
        for (int e = 0; e < M::NE; ++e) {
          if (((todo >> e) & 1u) && put < room) {
            a.lv[lbase + pos + put] = ev[e];
            a.li[lbase + pos + put] = rbase + M::row(e);
            todo &= ~(1u << e);
            ++put;
          }
        }
        // int8 pre-filter: a full list is not compacted (its entries are only
        // bounds); the surplus is dropped and the count, now above cap, marks
        // the list as overflowed so that the select rescans its whole range.
        if constexpr (Q8) break;
        uint64_t om = __ballot(todo != 0);
        if (!om) break;
#pragma unroll 1
        while (om) {
          const int ql0 = __shfl(ql, __ffsll((unsigned long long)om) - 1);
          const int64_t base0 = ((int64_t)(grp * BQ + ql0) * a.nlists + list) * a.cap;
          const float prev = thr_s[rs][ql0];
          if (lane == 0) lcnt[rs][ql0] = a.cap;  // positions [0, cap) are all written
          const float nt = fmaxf(prev, wave_compact(a.lv + base0, a.li + base0, a.cap, a.k,
                                                    sortbuf + w * kMaxCap));
          if (lane == 0) {
            lcnt[rs][ql0] = a.k;
            thr_s[rs][ql0] = nt;
          }
          om &= ~__ballot(ql == ql0);
        }
        // drop the scores that no longer pass the raised threshold
        if (todo) {
          const float tq = thr_s[rs][ql];
#pragma unroll
          for (int e = 0; e < M::NE; ++e)
            if (ev[e] < tq) todo &= ~(1u << e);
        }
      }
    }
    st_n = 0;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) thr[qb] = thr_s[rs][qs * QW + qb * MS + col];
  };

  // kMax for the int8 pre-filter: the sampling pass also quantises the batch's
  // queries (query i on wave i / #workgroups of workgroup i % #workgroups, so
  // each workgroup takes at most one more query than any other), its row loads
  // overlapping the prologue's stage loads; the threshold select that follows
  // then only selects.
  if constexpr (MODE == kMax) {
    if (a.qq_out != nullptr) {
      for (int qi = blockIdx.x + w * gridDim.x; qi < a.nq; qi += NW * gridDim.x) {
        float v[kQ8RowPer];
        q8_load_row(a.q + (int64_t)qi * d, d, lane, v);
        q8_quantize_row(v, d, a.dq, a.qq_out + (int64_t)qi * a.dq, a.qmeta_out + qi, lane, a.qf_out, qi);
      }
    }
  }

  // Retire the query/threshold loads (and stage 0, issued before them) with one
  // wait before the loop (otherwise the compiler's wait-count analysis carries
  // them around the loop back-edge and waits on vmcnt(0) at every stage), and
  // only then issue the other prologue stages: a load the compiler tracks,
  // waited on after stage loads were issued, would wait for all of them too
  // (vmcnt counts every vector memory load in issue order), which kept the
  // first tile behind the last prologue stage instead of the first (C1: 38.1 ->
  // 37.5 us per search, C5 69.3 -> 68.5 us).  The query fragments are pinned to
  // AGPRs only here: pinning uses a fragment, so before the wait it put a wait
  // per fragment ahead of the loads that follow them, a second round trip
  // (C5 66.4 -> 65.1 us, C2 -0.3 us).
  wait_vmcnt<0>();
  if constexpr (!QL && PIN_Q) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int ks = 0; ks < KSMAX; ++ks) qf[qb][ks] = pin_agpr(qf[qb][ks]);
  }
#pragma unroll
  for (int i = 1; i < NBUF - 1; ++i) issue_next();

  // The thresholds from sampling maxima: the threshold select's bit search
  // (count the maxima >= each candidate, summed over the 8 lanes by DPP),
  // started below the bits that the smallest and the largest maximum share
  // (the k-th largest lies between them) and stopped above the low
  // kThrLowBits bits, which leaves a valid lower bound at most 2^-11 of the
  // score below the exact k-th.  Written to LDS; every lane reads its
  // queries' after the prologue's barrier.
  if constexpr (TIN) {
    if (thr_in && (tid >> 3) < BQ) {  // whole waves: BQ is a multiple of 8
      constexpr int kThrLowBits = 12;
      const int ql = tid >> 3, g8 = tid & 7;
      const int qi = grp * BQ + ql;
#pragma unroll
      for (int j = 0; j < 8; ++j) asm volatile("" : "+v"(kraw[j]));  // keeps the uses (and their wait) here
      uint32_t key[8], hi = 0u, lo = ~0u;
#pragma unroll
      for (int j = 0; j < 8; ++j) {  // maxima past units_in: key 0, and no part in lo
        const uint32_t m = 0u - (uint32_t)(g8 + 8 * j < a.units_in);
        key[j] = float_order(kraw[j]) & m;
        hi = max(hi, key[j]);
        lo = min(lo, key[j] | ~m);
      }
      hi = max8_u32(hi);
      lo = min8_u32(lo);
      uint32_t tk = 0u;
      if (a.units_in >= a.k) {
        const uint32_t diff = hi ^ lo;
        const int top = diff ? 31 - __builtin_clz(diff) : -1;  // highest bit in which they differ
        tk = (top < 0 ? hi : hi & ~((2u << top) - 1u)) & ~((1u << kThrLowBits) - 1u);
        for (int bit = top; bit >= kThrLowBits; --bit) {
          const uint32_t cand = tk | (1u << bit);
          int c = 0;
#pragma unroll
          for (int j = 0; j < 8; ++j) c += key[j] >= cand ? 1 : 0;
          if (sum8_i32(c) >= a.k) tk = cand;
        }
      }
      const float tv = qi >= a.nq ? __builtin_inff() : (a.units_in >= a.k ? order_threshold(tk) : -__builtin_inff());
      if (g8 == 0)
#pragma unroll
        for (int r = 0; r < RS; ++r) thr_s[r][ql] = tv;
    }
  }

  // A fragments of one stage (KPS k-steps x RB row blocks), read from LDS one
  // stage ahead of the MFMAs that consume them.
  // A fragment of k-step kk, row block rb: row R = (rs*RB + rb)*MS + col, its
  // line kk / KSL, piece (kk % KSL)*G + kg, at (R*LPR + line)*128 +
  // ((piece ^ piece_swz(R)) << 4); piece_swz(R) depends on R mod 16 = col mod
  // 16 only, so one lane offset per k-step serves every rb.
  // (one lane offset per piece of a line; the line's 128-byte step is an
  // immediate offset of the read)
  int aoff[KSL];
#pragma unroll
  for (int kk = 0; kk < KSL; ++kk)
    aoff[kk] = (rs * RB * MS + col) * LPR * 128 + (((kk * G + kg) ^ piece_swz(col)) << 4);
  constexpr int RBOFF = MS * LPR * 128;  // LDS bytes between row blocks
  auto a_at = [&](int kk) { return aoff[kk % KSL] + (kk / KSL) * 128; };
  auto read_stage = [&](int buf_idx, half8 (&f)[KPS][RB]) {
    const unsigned char* buf = smem + buf_idx * STAGE;
#pragma unroll
    for (int kk = 0; kk < KPS; ++kk)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
        f[kk][rb] = *(const half8*)(buf + a_at(kk) + rb * RBOFF);
  };
  // QL: B fragment of k-step kk, query block qb: query-area row
  // Rq = qs*QW + qb*MS + col (after the TR corpus rows), same piece rule.
  // (Unused, and dropped by the compiler, when the queries sit in registers.)
  int boff[KPS];
#pragma unroll
  for (int kk = 0; kk < KPS; ++kk)
    boff[kk] = (TR + qs * QW + col) * 128 + (((kk * G + kg) ^ piece_swz(col)) << 4);
  auto read_qstage = [&](int buf_idx, half8 (&f)[KPS][QB]) {
    const unsigned char* buf = smem + buf_idx * STAGE;
#pragma unroll
    for (int kk = 0; kk < KPS; ++kk)
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) f[kk][qb] = *(const half8*)(buf + boff[kk] + qb * MS * 128);
  };
  // 8-wave full-width tiles (256 registers per wave) read the A fragments of
  // one k-step LA k-steps ahead into a ring of SL = LA + 1 slots (slot g % SL
  // holds k-step g) instead of a whole stage ahead: 24 instead of 64 VGPRs of
  // fragments.  Without it the 8-wave kernels spill, and the scratch reloads in
  // the tile loop wait on vmcnt(0), draining the stage pipeline (C2 scan 239 us
  // vs 192 us).  It syncs once per stage (paired sync would refill a buffer
  // still being read); 4-wave kernels keep the stage-ahead scheme (4% faster).
  constexpr int KT = NCMAX * KPS;  // k-steps per tile
  constexpr int LA = 2, SL = LA + 1;
  constexpr bool KRING = FULLW && NW == 8 && (KT % SL == 0);
  half8 ab[KRING ? 1 : 2][KPS][RB];  // stage s in ab[s & 1] (static within a tile), stage s+1 prefetched
  half8 bb[QL ? 2 : 1][KPS][QB];     // QL: the queries' B fragments, staged like ab
  half8 fr[KRING ? SL : 1][RB];
  auto read_ks = [&](int buf_idx, int kk, half8 (&f)[RB]) {
    const unsigned char* buf = smem + buf_idx * STAGE;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) f[rb] = *(const half8*)(buf + a_at(kk) + rb * RBOFF);
  };
  wait_vmcnt_lgkm0<(NBUF - 2) * LPW>();  // first stage landed (this wave)
  __builtin_amdgcn_s_barrier();           // ... and for every wave
  if (thr_in) {  // thresholds from sampling maxima, found above
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) thr[qb] = thr_s[rs][qs * QW + qb * MS + col];
  }
  if (KRING) {
#pragma unroll
    for (int g = 0; g < LA; ++g) read_ks(0, g, fr[g]);
  } else {
    read_stage(0, ab[0]);
    if constexpr (QL) read_qstage(0, bb[0]);
  }
  int cur_buf = 0;
  // QL: one stage of a runtime-length tile.  Same sync as the register-query
  // kernels: wait until the next stage has landed for every wave (the barrier
  // also retires every read of the buffer issue_next() refills), read its A
  // and B fragments, then run this stage's MFMAs on the ones read before.
  auto ql_stage = [&](half8 (&ca)[KPS][RB], half8 (&cb)[KPS][QB], half8 (&na)[KPS][RB],
                      half8 (&nb)[KPS][QB], auto& acc) {
    wait_vmcnt_lgkm0<(NBUF - 3) * LPW>();
    __builtin_amdgcn_s_barrier();
    issue_next();
    const int nxt = (cur_buf + 1 == NBUF) ? 0 : cur_buf + 1;
    read_stage(nxt, na);
    read_qstage(nxt, nb);
#pragma unroll
    for (int kk = 0; kk < KPS; ++kk)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) acc[qb][rb] = M::run(ca[kk][rb], cb[kk][qb], acc[qb][rb]);
    cur_buf = nxt;
  };

  // One tile's MFMAs into acc; the stage pipeline advances by one tile.
  auto tile_mfma = [&](acc_t (&acc)[QB][RB]) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int e = 0; e < M::NE; ++e) acc[qb][rb][e] = 0.f;

    if (KRING) {
#pragma unroll
      for (int c = 0; c < NCMAX; ++c) {
        // per-stage sync: stage c+1 has landed for every wave, and every read
        // of stage c-1's buffer is retired before issue_next() refills it
        wait_vmcnt_lgkm0<(NBUF - 3) * LPW>();
        __builtin_amdgcn_s_barrier();
        issue_next();
        const int nxt = (cur_buf + 1 == NBUF) ? 0 : cur_buf + 1;
#pragma unroll
        for (int kk = 0; kk < KPS; ++kk) {
          const int g = c * KPS + kk;
          if (kk + LA < KPS) read_ks(cur_buf, kk + LA, fr[(g + LA) % SL]);
          else read_ks(nxt, kk + LA - KPS, fr[(g + LA) % SL]);
#pragma unroll
          for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) acc[qb][rb] = M::run(fr[g % SL][rb], qf[qb][g], acc[qb][rb]);
        }
        cur_buf = nxt;
      }
    }
#pragma unroll
    for (int c = 0; c < NCMAX; ++c) {
      if (!KRING && c < nc) {
        // Stage s is in ab[c & 1].  Per-stage sync: wait until stage s+1 has
        // landed for every wave; the barrier also retires all reads of stage
        // s-1's buffer, which issue_next() refills with stage s+NBUF-1.  Paired
        // sync (even s only): wait for stages s+1 and s+2, then refill the
        // buffers of stages s-1 and s with stages s+NBUF-1 and s+NBUF.
        if (!PAIR) {
          wait_vmcnt_lgkm0<(NBUF - 3) * LPW>();
          __builtin_amdgcn_s_barrier();
          issue_next();
        } else if ((c & 1) == 0) {
          wait_vmcnt_lgkm0<(NBUF - 4) * LPW>();
          __builtin_amdgcn_s_barrier();
          issue_next();
          issue_next();
        }
        const int nxt = (cur_buf + 1 == NBUF) ? 0 : cur_buf + 1;
        read_stage(nxt, ab[(c + 1) & 1]);
#pragma unroll
        for (int kk = 0; kk < KPS; ++kk)
#pragma unroll
          for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int qb = 0; qb < QB; ++qb)
              acc[qb][rb] = M::run(ab[c & 1][kk][rb], qf[qb][KPS * c + kk], acc[qb][rb]);
        cur_buf = nxt;
      }
    }
    if constexpr (QL) {
      // stages in pairs, so that the fragment buffers are indexed statically
#pragma unroll 1
      for (int c = 0; c < nc; c += 2) {
        ql_stage(ab[0], bb[0], ab[1], bb[1], acc);
        if (c + 1 < nc) ql_stage(ab[1], bb[1], ab[0], bb[0], acc);
      }
      if (nc & 1) {  // the next tile's first stage sits in ab[1] / bb[1]
#pragma unroll
        for (int kk = 0; kk < KPS; ++kk) {
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) ab[0][kk][rb] = ab[1][kk][rb];
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) bb[0][kk][qb] = bb[1][kk][qb];
        }
      }
    }
    if (!QL && !KRING && (nc & 1)) {  // the next tile's first stage sits in ab[1]
#pragma unroll
      for (int kk = 0; kk < KPS; ++kk)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) ab[0][kk][rb] = ab[1][kk][rb];
    }
    // The epilogue's first VALU reads of the accumulators can follow the
    // tile's last MFMA within a few instructions (across the partial-tile
    // branch): pad its result latency (pad_mfma_result); the empty asm
    // statements order every accumulator read after the padding.
    pad_mfma_result<M::PASSES>(acc[QB - 1][RB - 1]);
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) asm volatile("" : "+v"(acc[qb][rb]));
  };

  // kAppendIn: the first tile is this workgroup's sample.  publish_units
  // stores its units: the largest exact score of each query (rows past n left
  // out) over the whole tile (one unit per workgroup, when there are 2k
  // workgroups) or over each row split's rows (each lane group's without row
  // splits), for the threshold workgroups.  wait_thresholds then reads the
  // thresholds of the group's queries (bounded waits), which replace the
  // initial -inf before any candidate is staged.
  auto publish_units = [&](int64_t t, acc_t (&acc)[QB][RB]) {
    const int64_t rowb = t * TR + rs * RW + 4 * kg;
    const bool partial = (t * TR + TR > n);
    const bool one = a.su_units == a.nchunks;
    auto put_unit = [&](int qi, int u, float um) {
      if (qi < a.nq)
        __hip_atomic_store(&a.su_w[(int64_t)qi * a.su_units + u],
                           (1ull << 32) | (unsigned long long)float_order(um), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    };
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      float um = -__builtin_inff();
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int e = 0; e < M::NE; ++e)
          if (!partial || rowb + rb * MS + M::row(e) < n) um = fmaxf(um, acc[qb][rb][e]);
      if (RS > 1 || one) um = fmaxf(um, __shfl_xor(um, 32));  // both lane groups
      const int ql = qs * QW + qb * MS + col;
      if (kg == 0 && one && RS > 1)
        thr_s[rs][ql] = um;  // (the row splits' maxima meet below)
      else if (RS == 1 && !one)
        put_unit(grp * BQ + ql, chunk * G + kg, um);
      else if (kg == 0)
        put_unit(grp * BQ + ql, one ? chunk : chunk * RS + rs, um);
    }
    if (one && RS > 1) {
      __syncthreads();
      for (int i = tid; i < BQ; i += NT) {  // (each thread rewrites only its own entries below)
        float um = thr_s[0][i];
#pragma unroll
        for (int r = 1; r < RS; ++r) um = fmaxf(um, thr_s[r][i]);
        put_unit(grp * BQ + i, chunk, um);
      }
    }
  };
  auto wait_thresholds = [&]() {
    for (int i = tid; i < BQ; i += NT) {
      const int qi = grp * BQ + i;
      const float tv = qi >= a.nq ? __builtin_inff() : tau_wait(a.tauw, qi, wait_ticks);
#pragma unroll
      for (int r = 0; r < RS; ++r) thr_s[r][i] = tv;
    }
    __syncthreads();
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) thr[qb] = thr_s[rs][qs * QW + qb * MS + col];
  };

  // The epilogue of tile t from its scores acc.
  auto tile_epilogue = [&](int64_t t, acc_t (&acc)[QB][RB]) {
    // ---- epilogue: acc[qb][rb][e] = score(query qwave0 + MS*qb + col,
    //                                        row rowb + MS*rb + M::row(e))
    const int64_t rowb = t * TR + rs * RW + 4 * kg;
    // kAppendQ8: the meta of the 64-row block holding this wave's rows, read
    // through the scalar cache (a vector load here would make the compiler wait
    // for every outstanding stage load before using it).
    float4 bm = float4{0.f, 0.f, 0.f, 0.f};
    if (Q8) {
      typedef const __attribute__((address_space(4))) float* cfloat_p;
      // (a wave whose rows all lie past n, in the last tile, reads the last block)
      const int64_t first = min(t * TR + rs * RW, n - 1);
      const int blk = __builtin_amdgcn_readfirstlane((int)(first >> 6));
      const cfloat_p m = (cfloat_p)a.bmeta + 4 * (int64_t)blk;
      bm = float4{m[0], m[1], m[2], m[3]};
    }
    const bool partial = (t * TR + TR > n);
    // kAppend / kAppendQ8: stage row block rb of query block qb (block maximum
    // m) for every lane whose maximum passes; val(e) is the lane's score e.
    auto stage = [&](int qb, int rb, float m, auto val) {
      uint64_t mk = __ballot(m >= thr[qb]);
      if (mk) {
        if (st_n + __popcll(mk) > STCAP) {
          flush();
          mk = __ballot(m >= thr[qb]);
        }
        if (m >= thr[qb]) {
          const int p = st_n + lanes_below(mk);
#pragma unroll
          for (int c = 0; c < M::NE / 4; ++c)
            *(f32x4*)(&st_val[w][p * EST + 4 * c]) = f32x4{val(4 * c), val(4 * c + 1), val(4 * c + 2), val(4 * c + 3)};
          st_meta[w][2 * p] = qs * QW + qb * MS + col;
          st_meta[w][2 * p + 1] = (int)rowb + rb * MS;
        }
        st_n += __popcll(mk);
      }
    };
    if constexpr (SIN && DEFER == 1) {
      if (t == t_begin) {
        publish_units(t, acc);
        wait_thresholds();
      }
    }
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int qi = qwave0 + qb * MS + col;
      if constexpr (MODE == kMaxQ8) {
        // the largest approximate score A = cq * acc of this lane's rows (cq >=
        // 0: that of the largest int32 sum) and its row (the first on ties)
        if (partial) {  // rows past n of the corpus's last tile: never the maximum
          const int64_t left = n - rowb;
#pragma unroll
          for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int e = 0; e < M::NE; ++e)
              if (rb * MS + M::row(e) >= left) acc[qb][rb][e] = INT_MIN;
        }
        int mi = acc[qb][0][0], mr = M::row(0);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int e = 0; e < M::NE; ++e)
            if (acc[qb][rb][e] > mi) {
              mi = acc[qb][rb][e];
              mr = rb * MS + M::row(e);
            }
        const float av = mi == INT_MIN ? -__builtin_inff() : (float)mi * (qm[qb].x * bm.x);
        const int row = (int)rowb + mr;
        if (a.agg) {
          if (av > umx[qb]) {
            umx[qb] = av;
            uag[qb] = row;
          }
        } else if (qi < a.nq) {
          const int64_t u = (int64_t)qi * a.units + ((chunk * a.spt + (t - t_begin)) * RS + rs) * G + kg;
          a.umax[u] = av;
          a.uarg[u] = row;
        }
      } else if constexpr (Q8) {
        // Upper bound of each exact score: A + slack with A = cq * acc and
        // cq >= 0, so the largest bound of a row block is that of its largest
        // int32 sum (conversion and fma round monotonically): the filter needs
        // one conversion per block, the rest only for staged blocks.
        const float cq = qm[qb].x * bm.x;
        const float slack = (fmaf(qm[qb].y, bm.y, qm[qb].z * bm.z) +
                             a.gamma * (qm[qb].y + qm[qb].z) * (bm.y + bm.z)) * (1.0f + 1.0f / 1048576.0f);
        if (partial) {  // only the corpus's last tile has rows past n: not in the block maximum
          const int64_t left = n - rowb;
#pragma unroll
          for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int e = 0; e < M::NE; ++e)
              if (rb * MS + M::row(e) >= left) acc[qb][rb][e] = INT_MIN;
        }
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          int mi = acc[qb][rb][0];
#pragma unroll
          for (int e = 1; e < M::NE; ++e) mi = max(mi, acc[qb][rb][e]);
          stage(qb, rb, fmaf((float)mi, cq, slack), [&](int e) { return fmaf((float)acc[qb][rb][e], cq, slack); });
        }
      } else {
        float v[NV];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int e = 0; e < M::NE; ++e) v[rb * M::NE + e] = acc[qb][rb][e];
        if (partial) {  // only the corpus's last tile has rows past n
          const int64_t left = n - rowb;
#pragma unroll
          for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int e = 0; e < M::NE; ++e)
              if (rb * MS + M::row(e) >= left) v[rb * M::NE + e] = -__builtin_inff();
        }

        if (STORE) {  // into this wave's LDS tile: [query qb*MS + col][row rb*MS + 4kg + row(e)]
          const int qo = (qb * MS + col) * SROW + 4 * kg;
#pragma unroll
          for (int j = 0; j < NV; j += 4) {  // elements 4c..4c+3 are 4 consecutive rows
            const int r = (j / M::NE) * MS + M::row(j % M::NE);
            if (MODE == kStoreF32)
              *(f32x4*)(&stg[w][qo + r]) = f32x4{v[j], v[j + 1], v[j + 2], v[j + 3]};
            else
              *(half4*)((_Float16*)stg[w] + qo + r) =
                  half4{(_Float16)v[j], (_Float16)v[j + 1], (_Float16)v[j + 2], (_Float16)v[j + 3]};
          }
        } else if constexpr (TOPK) {
          // Each of the lane's scores above its own k-th best and not below the
          // workgroup's threshold enters its list (a med3 insertion network; equal
          // scores keep the earlier, smaller row first).  Rows arrive in
          // ascending order per lane.  A score position no lane inserts is skipped.
          const float tw = order_float(thr_k[qs * QW + qb * MS + col]);
#pragma unroll
          for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int e = 0; e < M::NE; ++e) {
              const float sc = v[rb * M::NE + e];
              const bool ins = sc > tkv[qb][TK - 1] && sc >= tw && qi < a.nq;
              if (__ballot(ins)) {
                if (ins) {
                  const int r = (int)rowb + rb * MS + M::row(e);
#pragma unroll
                  for (int j = TK - 1; j >= 1; --j) {
                    const bool up = sc > tkv[qb][j - 1], here = sc > tkv[qb][j];
                    tki[qb][j] = up ? tki[qb][j - 1] : (here ? r : tki[qb][j]);
                    tkv[qb][j] = __builtin_amdgcn_fmed3f(tkv[qb][j - 1], tkv[qb][j], sc);
                  }
                  tki[qb][0] = sc > tkv[qb][0] ? r : tki[qb][0];
                  tkv[qb][0] = fmaxf(tkv[qb][0], sc);
                }
              }
            }
          if (qi < a.nq) atomicMax(&thr_k[qs * QW + qb * MS + col], float_order(tkv[qb][TK - 1]));
        } else if (MODE == kMax) {
          float m = v[0];
#pragma unroll
          for (int j = 1; j < NV; ++j) m = fmaxf(m, v[j]);
          if (a.agg)
            umx[qb] = fmaxf(umx[qb], m);
          else if (qi < a.nq)
            a.umax[(int64_t)qi * a.units + ((chunk * a.spt + (t - t_begin)) * RS + rs) * G + kg] = m;
        } else {  // kAppend: stage each row block whose maximum passes
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) {
            float m = v[rb * M::NE];
#pragma unroll
            for (int e = 1; e < M::NE; ++e) m = fmaxf(m, v[rb * M::NE + e]);
            stage(qb, rb, m, [&](int e) { return v[rb * M::NE + e]; });
          }
        }
      }
    }
    if (STORE) {  // write the tile out: each query's RW rows by RW/4 consecutive lanes, 4 rows each
      constexpr int LPQ = RW / 4;      // lanes per query
      constexpr int QPI = kWave / LPQ; // queries per store instruction
      static_assert(QW % QPI == 0, "store read-out shape");
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      const int r4 = 4 * (lane % LPQ);
      const int64_t row = t * TR + rs * RW + r4;
      // 16-byte (fp32) / 8-byte (fp16) stores need 4 | n (row starts aligned) and 4 whole rows
      const bool vec = (n % 4 == 0) && (row + 4 <= n);
#pragma unroll 4
      for (int qq = lane / LPQ; qq < QW; qq += QPI) {
        const int qi = qwave0 + qq;
        if (qi < a.nq) {
          const int so = qq * SROW + r4;
          if (MODE == kStoreF32) {
            const f32x4 x4 = *(const f32x4*)(&stg[w][so]);
            float* o = (float*)a.out + (int64_t)qi * n + row;
            if (vec) {
              *(f32x4*)o = x4;
            } else {
#pragma unroll
              for (int i = 0; i < 4; ++i)
                if (row + i < n) o[i] = x4[i];
            }
          } else {
            const half4 x4 = *(const half4*)((const _Float16*)stg[w] + so);
            _Float16* o = (_Float16*)a.out + (int64_t)qi * n + row;
            if (vec) {
              *(half4*)o = x4;
            } else {
#pragma unroll
              for (int i = 0; i < 4; ++i)
                if (row + i < n) o[i] = x4[i];
            }
          }
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    }
  };

  int64_t t_first = t_begin;
  if constexpr (SIN && DEFER > 1) {
    // The first DEFER tiles' MFMAs run before the thresholds are known (the
    // first tile's units published as soon as its scores are in), their
    // scores held in registers; then their epilogues.  The MFMAs of tiles 2..
    // DEFER fill the wait for the thresholds.
    acc_t accd[DEFER][QB][RB];
    const int64_t nd = t_end - t_begin < DEFER ? t_end - t_begin : DEFER;
#pragma unroll
    for (int dd = 0; dd < DEFER; ++dd) {
      if (dd < nd) {
        tile_mfma(accd[dd]);
        if (dd == 0) publish_units(t_begin, accd[0]);
      }
    }
    if (nd > 0) wait_thresholds();
#pragma unroll
    for (int dd = 0; dd < DEFER; ++dd)
      if (dd < nd) tile_epilogue(t_begin + dd, accd[dd]);
    t_first = t_begin + nd;
  }
  for (int64_t t = t_first; t < t_end; ++t) {
    acc_t acc[QB][RB];
    tile_mfma(acc);
    tile_epilogue(t, acc);
  }
  if (APP && st_n > 0) flush();
  if constexpr (TOPK) {
    // every lane's entries not below the workgroup's final threshold (real
    // rows only) into its wave's list of the query
    __syncthreads();
    const int list = chunk * RS + rs;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int ql = qs * QW + qb * MS + col;
      const int qi = grp * BQ + ql;
      const float tw = order_float(thr_k[ql]);
      int c = 0;
#pragma unroll
      for (int j = 0; j < TK; ++j) c += (tki[qb][j] >= 0 && tkv[qb][j] >= tw) ? 1 : 0;
      if (qi < a.nq && c > 0) {
        const int pos = atomicAdd(&lcnt[rs][ql], c);
        const int64_t lbase = ((int64_t)qi * a.nlists + list) * a.cap;
        int put = 0;
#pragma unroll
        for (int j = 0; j < TK; ++j) {
          if (tki[qb][j] >= 0 && tkv[qb][j] >= tw) {
            if (pos + put < a.cap) {
              a.lv[lbase + pos + put] = tkv[qb][j];
              a.li[lbase + pos + put] = tki[qb][j];
            }
            ++put;
          }
        }
      }
    }
  }
  if (SMAX && a.agg == 1) {
    // kMaxQ8 with perm: the units' corpus rows (perm of their companion rows;
    // the lookups overlap the drain below), so that the threshold needs no
    // lookup of its own
    int urow[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) urow[qb] = (MODE == kMaxQ8 && a.perm != nullptr) ? a.perm[uag[qb]] : uag[qb];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int qi = qwave0 + qb * MS + col;
      if (qi < a.nq) {
        const int64_t u = (int64_t)qi * a.units + (chunk * RS + rs) * G + kg;
        a.umax[u] = umx[qb];
        if (MODE == kMaxQ8) a.uarg[u] = urow[qb];
      }
    }
  }

  // Drain the trailing (dummy) stage loads before this workgroup's LDS can be
  // handed to another one, and make all list counts final.
  wait_vmcnt_lgkm0<0>();
  __builtin_amdgcn_s_barrier();
  if constexpr (MODE == kMax) {
    if (a.agg == 2) {  // one unit per workgroup: the maxima of its lane groups and row splits
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        float m = umx[qb];
#pragma unroll
        for (int off = MS; off < kWave; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
        if (kg == 0) mred[rs][qs * QW + qb * MS + col] = m;
      }
      __syncthreads();
      for (int i = tid; i < BQ; i += NT) {
        const int qi = grp * BQ + i;
        float m = mred[0][i];
#pragma unroll
        for (int r = 1; r < RS; ++r) m = fmaxf(m, mred[r][i]);
        if (qi < a.nq) a.umax[(int64_t)qi * a.units + chunk] = m;
      }
    }
  }
  if (APP || TOPK) {
    for (int i = tid; i < RS * BQ; i += NT) {
      const int r = i / BQ;
      const int ql = i % BQ;
      const int qi = grp * BQ + ql;
      if (qi < a.nq) a.lcount[(int64_t)qi * a.nlists + chunk * RS + r] = lcnt[r][ql];
    }
  }
}

// int8 pre-filter: full-width rows only (the int8 row bytes are padded to 32 * KS).
template <int MS, int QS, int QB, int RB, int KS>
hipError_t launch_one_q8(int mode, const ScanArgs& a, int grid, hipStream_t s) {
  if (a.d != KS * MfmaI8::KSZ || a.qf == nullptr || a.qmeta == nullptr || a.bmeta == nullptr) return hipErrorInvalidValue;
  if (mode == kMaxQ8) {
    if (a.umax == nullptr || a.uarg == nullptr || a.nsample < 1 || a.spt < 1 || a.agg < 0 || a.agg > 1)
      return hipErrorInvalidValue;
    hipLaunchKernelGGL((scan_kernel<MS, QS, QB, RB, KS, kMaxQ8, true>), dim3(grid), dim3(scan_waves(QS) * kWave), 0, s, a);
  } else {
    hipLaunchKernelGGL((scan_kernel<MS, QS, QB, RB, KS, kAppendQ8, true>), dim3(grid), dim3(scan_waves(QS) * kWave), 0, s,
                       a);
  }
  return hipGetLastError();
}

// One mode of one configuration: the full-width kernel when the row width is
// exactly KS k-steps, else the runtime-width one (the only one for KS = 0).
template <int MS, int QS, int QB, int RB, int KS, int MODE>
void launch_mode(bool full, const ScanArgs& a, int grid, hipStream_t s) {
  if constexpr (KS > 0) {
    if (full) {
      hipLaunchKernelGGL((scan_kernel<MS, QS, QB, RB, KS, MODE, true>), dim3(grid), dim3(scan_waves(QS) * kWave), 0, s, a);
      return;
    }
  }
  hipLaunchKernelGGL((scan_kernel<MS, QS, QB, RB, KS, MODE, false>), dim3(grid), dim3(scan_waves(QS) * kWave), 0, s, a);
}

template <int MS, int QS, int QB, int RB, int KS>
hipError_t launch_one(int mode, const ScanArgs& a, int grid, hipStream_t s) {
  const bool full = KS > 0 && (a.d == KS * Mfma<MS>::KSZ);
  if (KS > 0 && a.d > KS * Mfma<MS>::KSZ) return hipErrorInvalidValue;
  switch (mode) {
    case kAppend:
      launch_mode<MS, QS, QB, RB, KS, kAppend>(full, a, grid, s);
      break;
    case kMax:
      launch_mode<MS, QS, QB, RB, KS, kMax>(full, a, grid, s);
      break;
    case kStoreF32:
      launch_mode<MS, QS, QB, RB, KS, kStoreF32>(full, a, grid, s);
      break;
    case kStoreF16:
      launch_mode<MS, QS, QB, RB, KS, kStoreF16>(full, a, grid, s);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// The instantiated configurations: (MS, QS, QB, RB, KSMAX).  KSMAX * KSZ is the
// widest row each one accepts (KSZ = 32 for MS = 16, 16 for MS = 32); KSMAX = 0
// takes rows of any width (multiple of 64), with the queries staged through LDS
// beside the corpus rows instead of held in registers.
#define CVS_SCAN_CONFIGS(X) \
  X(16, 1, 1, 1, 12)        \
  X(16, 1, 1, 1, 24)        \
  X(16, 1, 1, 1, 48)        \
  X(16, 2, 1, 1, 48)        \
  X(16, 4, 1, 2, 48)        \
  X(32, 1, 1, 1, 24)        \
  X(32, 1, 1, 1, 48)        \
  X(32, 1, 2, 1, 24)        \
  X(32, 2, 1, 1, 48)        \
  X(32, 4, 1, 2, 24)        \
  X(32, 4, 1, 2, 48)        \
  X(32, 8, 1, 2, 24)        \
  X(16, 1, 1, 1, 0)         \
  X(32, 1, 1, 1, 0)         \
  X(32, 2, 1, 1, 0)         \
  X(32, 4, 1, 2, 0)

// int8 pre-filter configurations (KS in 32-byte k-steps: 12, 24, 48 = int8 rows
// of 384, 768, 1536 bytes).
#define CVS_SCAN_Q8_CONFIGS(X) \
  X(32, 1, 1, 1, 12)           \
  X(32, 1, 1, 1, 24)           \
  X(32, 1, 1, 1, 48)           \
  X(32, 1, 2, 1, 12)           \
  X(32, 1, 2, 1, 24)           \
  X(32, 4, 1, 2, 12)           \
  X(32, 4, 1, 2, 24)           \
  X(32, 4, 1, 2, 48)           \
  X(32, 8, 1, 2, 12)           \
  X(32, 8, 1, 2, 24)

}  // namespace

bool scan_topk_available(const ScanCfg& c, int64_t d, int64_t k) {
  return c.ms == 32 && c.qs == 1 && c.qb == 1 && c.rb == 1 && c.ksmax == 24 && d <= 384 && k >= 1 && k <= 16;
}

hipError_t launch_scan_topk(const ScanCfg& c, const ScanArgs& a, int grid, hipStream_t s) {
  if (!scan_topk_available(c, a.d, a.k) || a.cap < 2 * 16 || a.nlists != a.nchunks * c.rs()) return hipErrorInvalidValue;
  launch_mode<32, 1, 1, 1, 24, kTopK>(a.d == 24 * 16, a, grid, s);
  return hipGetLastError();
}

// Mode kAppendIn: the full-width d = 384 configurations, one query group.
#define CVS_SCAN_IN_CONFIGS(X) \
  X(32, 1, 1, 1, 24)           \
  X(32, 1, 2, 1, 24)           \
  X(32, 4, 1, 2, 24)           \
  X(32, 8, 1, 2, 24)

bool scan_in_available(const ScanCfg& c, int64_t d) {
#define CVS_HAS_IN(MS, QS, QB, RB, KS) \
  if (c.ms == MS && c.qs == QS && c.qb == QB && c.rb == RB && c.ksmax == KS) return d == KS * Mfma<MS>::KSZ;
  CVS_SCAN_IN_CONFIGS(CVS_HAS_IN)
#undef CVS_HAS_IN
  return false;
}

hipError_t launch_scan_in(const ScanCfg& c, const ScanArgs& a, int grid, hipStream_t s) {
  const int nw = scan_waves(c.qs);
  if (!scan_in_available(c, a.d) || a.groups != 1 || a.tau != nullptr || a.umax_in != nullptr ||
      a.tauw == nullptr || a.su_w == nullptr || a.qfh == nullptr ||
      (a.su_units != a.nchunks && a.su_units != a.nchunks * (c.rs() > 1 ? c.rs() : kWave / c.ms)) ||
      a.su_units > kWave * (nw == 8 ? 8 : 32) || a.nlists != a.nchunks * c.rs() || a.k < 1 || a.k > 256 ||
      grid != a.nchunks + (a.nq + nw - 1) / nw)
    return hipErrorInvalidValue;
#define CVS_LAUNCH_IN(MS, QS, QB, RB, KS)                                     \
  if (c.ms == MS && c.qs == QS && c.qb == QB && c.rb == RB && c.ksmax == KS) { \
    hipLaunchKernelGGL((scan_kernel<MS, QS, QB, RB, KS, kAppendIn, true>), dim3(grid), dim3(nw * kWave), 0, s, a); \
    return hipGetLastError();                                                  \
  }
  CVS_SCAN_IN_CONFIGS(CVS_LAUNCH_IN)
#undef CVS_LAUNCH_IN
  return hipErrorInvalidValue;
}

namespace {
// Thread i clears word i and copies 16-byte fragment piece i: piece o of the
// copy is lane o % 64 of (32-query block, k-step) o / 64, i.e. 8 halfs of
// query 32 * block + (lane % 32) at dims 16 * k-step + 8 * (lane / 32).
__global__ __launch_bounds__(kBlock) void scan_in_prep_kernel(const _Float16* q, int nq, int d, _Float16* qfh,
                                                              unsigned long long* words, int64_t nwords) {
  const int ks_per_row = d / 16;
  const int64_t npieces = (int64_t)((nq + 31) / 32) * ks_per_row * kWave;
  const int64_t total = nwords > npieces ? nwords : npieces;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < total; i += (int64_t)gridDim.x * kBlock) {
    if (i < nwords) words[i] = 0ull;
    if (i < npieces) {
      const int lane = (int)(i % kWave);
      const int64_t t = i / kWave;
      const int ks = (int)(t % ks_per_row);
      const int qi = (int)(t / ks_per_row) * 32 + (lane & 31);
      half8 v = {};
      if (qi < nq) v = *(const half8*)(q + (int64_t)qi * d + ks * 16 + (lane >> 5) * 8);
      *(half8*)(qfh + i * 8) = v;
    }
  }
}
}  // namespace

hipError_t launch_scan_in_prep(const _Float16* q, int nq, int d, _Float16* qfh, unsigned long long* words, int64_t nwords,
                               hipStream_t s) {
  if (q == nullptr || qfh == nullptr || words == nullptr || nq < 1 || d < 16 || d % 16 != 0 || nwords < 0)
    return hipErrorInvalidValue;
  const int64_t npieces = (int64_t)((nq + 31) / 32) * (d / 16) * kWave;
  const int64_t total = nwords > npieces ? nwords : npieces;
  const int64_t need = (total + kBlock - 1) / kBlock;
  const int64_t blocks = need < 512 ? need : 512;
  hipLaunchKernelGGL(scan_in_prep_kernel, dim3((unsigned)blocks), dim3(kBlock), 0, s, q, nq, d, qfh, words, nwords);
  return hipGetLastError();
}

bool scan_cfg_available(const ScanCfg& c, int mode) {
  if (mode == kAppendQ8 || mode == kMaxQ8) {
#define CVS_HAS_Q8(MS, QS, QB, RB, KS) \
  if (c.ms == MS && c.qs == QS && c.qb == QB && c.rb == RB && c.ksmax == KS) return true;
    CVS_SCAN_Q8_CONFIGS(CVS_HAS_Q8)
#undef CVS_HAS_Q8
    return false;
  }
  if (mode < kAppend || mode > kStoreF16) return false;
#define CVS_HAS(MS, QS, QB, RB, KS) \
  if (c.ms == MS && c.qs == QS && c.qb == QB && c.rb == RB && c.ksmax == KS) return true;
  CVS_SCAN_CONFIGS(CVS_HAS)
#undef CVS_HAS
  return false;
}

hipError_t launch_scan(const ScanCfg& c, int mode, const ScanArgs& a, int grid, hipStream_t s) {
  if (mode == kAppendQ8 || mode == kMaxQ8) {
#define CVS_LAUNCH_Q8(MS, QS, QB, RB, KS)                                      \
  if (c.ms == MS && c.qs == QS && c.qb == QB && c.rb == RB && c.ksmax == KS) \
    return launch_one_q8<MS, QS, QB, RB, KS>(mode, a, grid, s);
    CVS_SCAN_Q8_CONFIGS(CVS_LAUNCH_Q8)
#undef CVS_LAUNCH_Q8
    return hipErrorInvalidValue;
  }
#define CVS_LAUNCH(MS, QS, QB, RB, KS)                                              \
  if (c.ms == MS && c.qs == QS && c.qb == QB && c.rb == RB && c.ksmax == KS) \
    return launch_one<MS, QS, QB, RB, KS>(mode, a, grid, s);
  CVS_SCAN_CONFIGS(CVS_LAUNCH)
#undef CVS_LAUNCH
  return hipErrorInvalidValue;
}

}  // namespace cvs
