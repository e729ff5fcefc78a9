// int8 pre-filter scan for 384-byte int8 rows at 256 queries per workgroup
// (fp16 widths up to 384, batches above 128: the 1M x 384, batch 256 class).
//
// Same contract as scan_kernel<32, 8, 1, 2, 12, kAppendQ8, true> in
// cvs_scan.hip, which it replaces for these shapes: one workgroup per (group
// of 256 queries, corpus chunk); int8 scores of 64-row tiles on
// v_mfma_i32_32x32x32_i8; the rigorous upper bound U of each exact score; rows
// with U >= the query's threshold appended to the (query, chunk) candidate
// list, whose count runs past its capacity when it fills (the select then
// rescans the chunk).  What differs is the hot loop:
//
//  * 8 wave64s, two per SIMD, as 4 query groups of 64 x 2 row halves of 32.
//    Each wave reads only its 32 rows of a tile from LDS and feeds each A
//    fragment to two MFMAs (its two 32-query blocks): half the LDS fragment
//    reads of 8 waves x 32 queries over all 64 rows.  Query fragments stay in
//    AGPRs (2 x 12 x 16 bytes per lane), loaded from the quantisation's
//    fragment-ordered copy (1 KiB of contiguous memory per wave and k-step).
//  * A tile is one 24 KB stage (64 rows x 384 bytes) and one 64-row block of
//    the companion (one block-meta entry).  The companion is padded to whole
//    64-row blocks, so no DMA load needs a bounds clamp: each of a wave's 3
//    loads per stage is global_load_lds_dwordx4 from a scalar 64-bit tile base
//    plus a constant 32-bit lane offset (no per-load vector address
//    arithmetic); stages past the workgroup's own tiles are not loaded.
//  * The tile's block meta comes through the scalar cache, loaded one tile
//    ahead and consumed after the next mid-tile wait.
//  * Sampling and thresholds in the same launch (tauw not null): each
//    workgroup first runs the chunk's first spt tiles through the same MFMAs
//    keeping, per (query, row half), the largest approximate score A and its
//    row; publishes these units; computes one query's threshold from every
//    workgroup's units (cvs_tau_group.h) while its ring already holds the
//    first scanned tiles; then scans the whole chunk.  One launch replaces
//    the sampling pass, its threshold select and their two launch gaps, and
//    the sampled tiles' MFMAs run at the scan's rate.
//
// Stage layout (as the generic kernel's whole-tile stages): row R of a tile at
// R * 384 bytes, three 128-byte lines, slot s of a line holding 16-byte piece
// s ^ piece_swz(R).  DMA load f (0..23) fills stage bytes [1024 f, 1024 f +
// 1024): lane l writes slot l % 8 of line L = 8 f + l / 8 (row L / 3), so every
// load reads 8 consecutive 128-byte lines of global memory.
#include <climits>

#include "cvs_common.h"
#include "cvs_kernels.h"
#include "cvs_q8_row.h"
#include "cvs_tau_group.h"

namespace cvs {

namespace {

constexpr int kQ8Row = 384;                // int8 row bytes
constexpr int kQ8Ks = kQ8Row / 32;          // 32-byte MFMA k-steps per row
constexpr int kQ8Tile = 64;                 // rows per tile = rows per block-meta entry
constexpr int kQ8Stage = kQ8Tile * kQ8Row;  // 24 KB
constexpr int kQ8Nbuf = 4;                  // stages in the ring (two in flight during a tile)
constexpr int kQ8Waves = 8;
constexpr int kQ8Bq = 256;                  // queries per workgroup
constexpr int kQ8Lpw = kQ8Stage / 1024 / kQ8Waves;  // DMA loads per wave per stage
constexpr int kQ8Stcap = 64;                // staged entries per wave
constexpr int kQ8LateKs = 4;                // k-step of the tile barrier of row half 1's waves
// A staged entry is one lane's 16 int32 sums of one (query block, tile) and
// (query in group, first row, cq, slack): 80 bytes, an odd count of 16-byte
// units, so the ds_write_b128s of 16 consecutive entries hit distinct banks.
constexpr int kQ8Est = 20;
static_assert(kQ8Lpw * kQ8Waves * 1024 == kQ8Stage, "a stage is whole 1 KB loads, the same count per wave");
static_assert(kQ8Ks % 3 == 0, "the 3-slot fragment ring needs the k-steps of a tile in multiples of 3");
static_assert(kQ8LateKs < kQ8Ks - 2, "row half 1's tile barrier comes before its first read of the next stage");

typedef int i32x16 __attribute__((ext_vector_type(16)));

// Row (within a 32-row block) of accumulator element e of lane l, minus 4 * (l / 32):
// v_mfma_i32_32x32x32_i8 gives lane l D[8i + 4(l/32) + j][l % 32] in element 4i + j.
__device__ __forceinline__ constexpr int acc_row(int e) { return 8 * (e >> 2) + (e & 3); }

__global__ __launch_bounds__(kQ8Waves * kWave, 1) void q8scan384_kernel(ScanArgs a) {
  __shared__ __attribute__((aligned(1024))) unsigned char smem[kQ8Nbuf * kQ8Stage];
  __shared__ int lcnt[kQ8Bq];    // entries appended to each query's list of this chunk
  __shared__ float thr_s[kQ8Bq];  // per-query threshold
  __shared__ __attribute__((aligned(16))) int st_ent[kQ8Waves][kQ8Stcap * kQ8Est];  // staged entries

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int qgw = w & 3;   // this wave's 64 queries: [64 qgw, 64 qgw + 64) of the group
  const int half = w >> 2;  // this wave's rows of every tile: [32 half, 32 half + 32)
  const int col = lane & 31;
  const int kg = lane >> 5;

  int grp, chunk;  // workgroup -> (query group, chunk), as scan_kernel
  {
    const int id = blockIdx.x;
    if (a.xcd_pair) {
      const int slot = id >> 3;
      grp = slot % a.groups;
      chunk = (slot / a.groups) * 8 + (id & 7);
    } else {
      grp = id % a.groups;
      chunk = id / a.groups;
    }
  }
  const int64_t n = a.n;
  const int64_t t_begin = (int64_t)chunk * a.tpc;
  const int64_t t_end = t_begin + a.tpc < a.ntiles ? t_begin + a.tpc : a.ntiles;
  const int64_t t_last = a.ntiles - 1;
  const unsigned char* xq = reinterpret_cast<const unsigned char*>(a.x);
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)smem);

  // ---- stage issue (3 loads per wave), NBUF - 1 stages ahead of the compute ----
  uint32_t voff[kQ8Lpw];
#pragma unroll
  for (int j = 0; j < kQ8Lpw; ++j) {
    const int L = (w + kQ8Waves * j) * 8 + (lane >> 3);  // stage line of this lane's piece
    voff[j] = (uint32_t)(L * 128 + (((lane & 7) ^ piece_swz(L / 3)) << 4));
  }
  // The workgroup's tile sequence.  With sampling in the scan (a.tauw not
  // null): the first spt tiles of its chunk, sampled, then every tile of the
  // chunk, scanned (the sampled ones again, now against the thresholds);
  // otherwise the chunk's tiles, scanned.  Workgroups past the scan's chunks
  // (the grid extends to one workgroup per query) only compute their query's
  // threshold.
  const bool fused = a.tauw != nullptr;
  // bound of each cross-workgroup wait (100 MHz ticks); 0 only in tests: every
  // wait not satisfied at once gives up, which exercises the exact fallbacks
  const uint64_t wait_ticks = a.no_wait ? 0 : kTauWaitTicks;
  const bool tau_only = fused && (int)blockIdx.x >= a.groups * a.nchunks;
  const int64_t ntl = (tau_only || t_end <= t_begin) ? 0 : t_end - t_begin;
  const int spt = fused ? (int)(a.spt < ntl ? a.spt : ntl) : 0;
  const int64_t npos = spt + ntl;
  auto tile_at = [&](int64_t p) -> int64_t { return t_begin + (p < spt ? p : p - spt); };
  int64_t it_p = 0;
  int it_buf = 0;
  // Positions past the sequence are not loaded (the tile loop's waits account
  // for it): prefetching them would read another chunk's tiles, ~5% of the
  // corpus again over a launch, and the final drain would wait for them.
  auto issue_next = [&]() {
    if (it_p < npos) {
      const unsigned char* base = xq + tile_at(it_p) * kQ8Stage;
      const uint32_t lds = lds0 + (uint32_t)(it_buf * kQ8Stage + w * 1024);
#pragma unroll
      for (int j = 0; j < kQ8Lpw; ++j) dma16_saddr(voff[j], base, lds + (uint32_t)(j * kQ8Waves * 1024));
    }
    ++it_p;
    it_buf = (it_buf + 1 == kQ8Nbuf) ? 0 : it_buf + 1;
  };
  // ---- this lane's two queries: fragments (AGPRs), thresholds, bound terms ----
  i32x4 qf[2][kQ8Ks];
  float thr[2];
  float4 qm[2];
  auto load_queries = [&]() {
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const int qi = grp * kQ8Bq + qgw * 64 + qb * 32 + col;
      const int qc = min(qi, a.nq - 1);  // columns past nq load the last query; their threshold is +inf
      i32x4 ld[kQ8Ks];
#pragma unroll
      for (int ks = 0; ks < kQ8Ks; ++ks) ld[ks] = *(const i32x4*)(a.qf + q8_frag_offset(qc, ks, kg, kQ8Ks));
#pragma unroll
      for (int ks = 0; ks < kQ8Ks; ++ks) qf[qb][ks] = pin_agpr(ld[ks]);
      thr[qb] = (qi >= a.nq) ? __builtin_inff() : (a.tau ? a.tau[qi] : -__builtin_inff());
      qm[qb] = a.qmeta[qc];
    }
  };
  // Query blockIdx.x's threshold (waves 0-3; waves 4-7 keep step with the
  // group's barriers), in the staging area, which holds no entries then.
  static_assert(2 * sizeof(TauGroupShared) <= sizeof(st_ent), "threshold scratch in the staging area");
  TauGroupShared* tg = reinterpret_cast<TauGroupShared*>(&st_ent[0][0]);
  auto threshold = [&]() {
    const int qt = (w < 4 && (int)blockIdx.x < a.nq) ? (int)blockIdx.x : -1;
    tau_group<2, 4, 4>(tg[w >> 2], tid & 255, qt, a.su_w, a.su_units, a.k, a.qh, a.xh, n, a.dh, a.perm, a.tauw,
                       a.tau_out, wait_ticks);
  };
  if (tau_only) {
    threshold();
    return;
  }
  issue_next();  // stage 0 first; stages 1 and 2 once it and the queries are in
  load_queries();

  for (int i = tid; i < kQ8Bq; i += kQ8Waves * kWave) {
    const int qi = grp * kQ8Bq + i;
    lcnt[i] = 0;
    if (!fused) thr_s[i] = (qi >= a.nq) ? __builtin_inff() : (a.tau ? a.tau[qi] : -__builtin_inff());
  }
  int st_n = 0;  // wave-uniform count of staged entries

  // Appends the rows of this wave's staged entries whose bound reaches their
  // query's threshold to the (query, chunk) lists.  The bounds are computed
  // here (the same fmaf(sum, cq, slack) as the block maxima's), off the tile
  // loop.  No compaction (entries are bounds): the surplus of a full list is
  // dropped and its count, now above cap, marks it overflowed.  Both row
  // halves of a query share its list and count.
  auto flush = [&]() {
#pragma unroll 1
    for (int base = 0; base < st_n; base += kWave) {
      const int er = base + lane;
      const bool have = er < st_n;
      const int* ent = &st_ent[w][(have ? er : 0) * kQ8Est];
      const i32x4 mt = *(const i32x4*)(ent + 16);
      const int ql = have ? mt[0] : 0;
      const int rbase = have ? mt[1] : 0;
      const float cq = __int_as_float(mt[2]), slack = __int_as_float(mt[3]);
      float ev[16];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const i32x4 t = *(const i32x4*)(ent + 4 * c);
#pragma unroll
        for (int i = 0; i < 4; ++i) ev[4 * c + i] = fmaf((float)t[i], cq, slack);
      }
      const int64_t lbase = ((int64_t)(grp * kQ8Bq + ql) * a.nlists + chunk) * a.cap;
      unsigned todo = 0;
      if (have) {
        const float tq = thr_s[ql];
#pragma unroll
        for (int e = 0; e < 16; ++e) todo |= (ev[e] >= tq && rbase + acc_row(e) < n ? 1u : 0u) << e;
      }
      const int cnt = __popc(todo);
      const int pos = cnt ? atomicAdd(&lcnt[ql], cnt) : 0;
      const int room = a.cap - pos;
      // The passing rows in ascending order, one per lane and round (rarely
      // more than one per lane): bound and row from the entry's own sum in LDS.
      int put = 0;
      while (__any(todo != 0u)) {
        if (todo != 0u) {
          const int e = __builtin_ctz(todo);
          todo &= todo - 1u;
          if (put < room) {
            a.lv[lbase + pos + put] = fmaf((float)ent[e], cq, slack);
            a.li[lbase + pos + put] = rbase + acc_row(e);
          }
          ++put;
        }
      }
    }
    st_n = 0;
  };

  // Retire the query and threshold loads and stage 0 before the loop (so the
  // loop's waits count only stage loads), then issue stages 1 and 2 and start:
  // the launch's first burst of HBM reads is one stage instead of three (back-to-back
  // C2 searches 1.2 us faster on average over five interleaved A/Bs).
  wait_vmcnt_lgkm0<0>();
#pragma unroll
  for (int i = 1; i < kQ8Nbuf - 1; ++i) issue_next();
  __builtin_amdgcn_s_barrier();

  // LDS offsets of this lane's A fragment pieces: k-step ks of row
  // R = 32 half + col is piece 2 (ks % 4) + kg of line ks / 4, in slot
  // piece ^ piece_swz(R) (piece_swz(R) = piece_swz(col): R mod 16 = col mod 16).
  uint32_t aoff[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk)
    aoff[kk] = (uint32_t)((32 * half + col) * kQ8Row + (((2 * kk + kg) ^ piece_swz(col)) << 4));
  auto frag = [&](int buf, int ks) -> i32x4 {
    return *(const i32x4*)(smem + buf * kQ8Stage + aoff[ks & 3] + (ks >> 2) * 128);
  };
  // Fragments of k-step g live in slot g % 3, read two k-steps ahead.
  i32x4 fr[3];
  fr[0] = frag(0, 0);
  fr[1] = frag(0, 1);
  int cur = 0;

  // block meta of the first tile; later tiles' are loaded one tile ahead
  typedef const __attribute__((address_space(4))) float* cfloat_p;
  const cfloat_p meta = (cfloat_p)a.bmeta;
  float4 bm_next;
  {
    const cfloat_p m = meta + 4 * (t_begin < t_last ? t_begin : t_last);
    bm_next = float4{m[0], m[1], m[2], m[3]};
  }
  // sampling: this lane's largest approximate score A = cq * sum of its rows
  // (per query block) and its companion row, over the sampled tiles
  float umx[2] = {-__builtin_inff(), -__builtin_inff()};
  int uag[2] = {0, 0};
  // One unit per (query, row half): the better of the two lane groups' (the
  // lower row on ties), published as (row + 1) << 32 | bits(A).
  auto publish_units = [&]() {
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const float ov = __shfl_xor(umx[qb], 32);
      const int orow = __shfl_xor(uag[qb], 32);
      if (ov > umx[qb] || (ov == umx[qb] && orow < uag[qb])) {
        umx[qb] = ov;
        uag[qb] = orow;
      }
      const int qi = grp * kQ8Bq + qgw * 64 + qb * 32 + col;
      if (kg == 0 && qi < a.nq)
        __hip_atomic_store(&a.su_w[(int64_t)qi * a.su_units + 2 * chunk + half],
                           ((unsigned long long)(uag[qb] + 1) << 32) | __float_as_uint(umx[qb]), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
  };

  // One tile of the sequence: its block meta (loaded a tile ahead) and its
  // MFMAs, which also read the next position's first fragments.  The waves of
  // row half 0 take the tile's barrier two k-steps before its end, those of
  // row half 1 kQ8LateKs k-steps into it: the two waves of a SIMD (one of each
  // half: wave w and w + 4) then reach their epilogues half a tile apart, and
  // each one's epilogue runs beside the other's MFMAs instead of both leaving
  // the matrix core idle at once.  Every wave still takes one barrier per tile.
  auto tile_mfma = [&](int64_t p, float4& bm, i32x16& acc0, i32x16& acc1) {
    const int64_t t = tile_at(p);
    bm = bm_next;
    {
      const int64_t tn = p + 1 < npos ? tile_at(p + 1) : t;
      const cfloat_p m = meta + 4 * (tn < t_last ? tn : t_last);
      bm_next = float4{m[0], m[1], m[2], m[3]};
    }
    const int nxt = (cur + 1 == kQ8Nbuf) ? 0 : cur + 1;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      acc0[e] = 0;
      acc1[e] = 0;
    }
#pragma unroll
    for (int ks = 0; ks < kQ8Ks; ++ks) {
      if ((ks == kQ8Ks - 2 && half == 0) || (ks == kQ8LateKs && half == 1)) {
        // The fragments read from k-step kQ8Ks - 2 on are position p+1's (the
        // current stage's were published by the previous tile's barrier, so
        // the MFMAs above overlap the waves' arrival here).  Stage p+1 has
        // landed for every wave, and every read of the buffer that
        // issue_next() refills (stage p-1's) has retired: row half 1's waves
        // are kQ8LateKs k-steps into stage p, whose reads do not touch p-1's
        // buffer, and the buffer refilled at the next barrier (stage p's) is
        // read by no wave after its k-step kQ8Ks - 1 of this tile.  Stage p+2's loads may still be
        // in flight, when it exists: near the end there is nothing after
        // stage p+1 to leave outstanding.  (Exact for a ring of 4: one stage,
        // p+2, may be outstanding, and it exists exactly when p + 2 < npos.)
        static_assert(kQ8Nbuf == 4, "the end-of-range wait counts assume a ring of 4 stages");
        if (p + 2 < npos)
          wait_vmcnt_lgkm0<(kQ8Nbuf - 3) * kQ8Lpw>();
        else
          wait_vmcnt_lgkm0<0>();
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");  // no LDS read moves above the barrier
        issue_next();
      }
      if (ks + 2 < kQ8Ks)
        fr[(ks + 2) % 3] = frag(cur, ks + 2);
      else
        fr[(ks + 2) % 3] = frag(nxt, ks + 2 - kQ8Ks);
      acc0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(fr[ks % 3], qf[0][ks], acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(fr[ks % 3], qf[1][ks], acc1, 0, 0, 0);
    }
    cur = nxt;
  };
  // acc{qb}[e] = int8 score of query 64 qgw + 32 qb + col, row rowb +
  // acc_row(e); rows past n (only in the corpus's last tile) get INT_MIN.
  auto tile_rows = [&](int64_t p, i32x16& acc0, i32x16& acc1) -> int64_t {
    pad_mfma_result<8>(acc1);
    asm volatile("" : "+v"(acc0));
    asm volatile("" : "+v"(acc1));
    const int64_t t = tile_at(p);
    const int64_t rowb = t * kQ8Tile + 32 * half + 4 * kg;
    if (t * kQ8Tile + kQ8Tile > n) {
      const int64_t left = n - rowb;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        if (acc_row(e) >= left) {
          acc0[e] = INT_MIN;
          acc1[e] = INT_MIN;
        }
      }
    }
    return rowb;
  };

  // ---- sampled tiles: the lane's largest sum of each (its first row on ties) ----
#pragma unroll 1
  for (int64_t p = 0; p < spt; ++p) {
    float4 bm;
    i32x16 acc0, acc1;
    tile_mfma(p, bm, acc0, acc1);
    const int64_t rowb = tile_rows(p, acc0, acc1);
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const i32x16& acc = qb ? acc1 : acc0;
      int mi = acc[0], me = 0;
#pragma unroll
      for (int e = 1; e < 16; ++e)
        if (acc[e] > mi) {
          mi = acc[e];
          me = e;
        }
      const float av = mi == INT_MIN ? -__builtin_inff() : (float)mi * (qm[qb].x * bm.x);
      if (av > umx[qb]) {
        umx[qb] = av;
        uag[qb] = (int)rowb + acc_row(me);
      }
    }
  }
  if (fused) {
    publish_units();
    threshold();  // waits for every workgroup's units of query blockIdx.x
  }

  // ---- scanned tiles ----
#pragma unroll 1
  for (int64_t p = spt; p < npos; ++p) {
    float4 bm;
    i32x16 acc0, acc1;
    tile_mfma(p, bm, acc0, acc1);
    if (fused && p == spt) {
      // the thresholds (this workgroup's and the others'), waited for while
      // the first scanned tile's MFMAs run
      for (int i = tid; i < kQ8Bq; i += kQ8Waves * kWave) {
        const int qi = grp * kQ8Bq + i;
        thr_s[i] = qi >= a.nq ? __builtin_inff() : tau_wait(a.tauw, qi, wait_ticks);
      }
      __syncthreads();
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) thr[qb] = thr_s[qgw * 64 + qb * 32 + col];
    }
    const int64_t rowb = tile_rows(p, acc0, acc1);
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const i32x16& acc = qb ? acc1 : acc0;
      // U = cq * A + slack with cq >= 0: the largest bound of the lane's 16 rows
      // is that of its largest int32 sum (conversion and fma round monotonically)
      const float cq = qm[qb].x * bm.x;
      const float slack = (fmaf(qm[qb].y, bm.y, qm[qb].z * bm.z) +
                           a.gamma * (qm[qb].y + qm[qb].z) * (bm.y + bm.z)) * (1.0f + 1.0f / 1048576.0f);
      int mi = acc[0];
#pragma unroll
      for (int e = 1; e < 16; ++e) mi = max(mi, acc[e]);
      const float m = fmaf((float)mi, cq, slack);
      uint64_t mk = __ballot(m >= thr[qb]);
      if (mk) {
        if (st_n + __popcll(mk) > kQ8Stcap) flush();
        if (m >= thr[qb]) {
          int* ent = &st_ent[w][(st_n + lanes_below(mk)) * kQ8Est];
#pragma unroll
          for (int c = 0; c < 4; ++c)
            *(i32x4*)(ent + 4 * c) = i32x4{acc[4 * c], acc[4 * c + 1], acc[4 * c + 2], acc[4 * c + 3]};
          *(i32x4*)(ent + 16) = i32x4{qgw * 64 + qb * 32 + col, (int)rowb, __float_as_int(cq), __float_as_int(slack)};
        }
        st_n += __popcll(mk);
      }
    }
  }
  if (st_n > 0) flush();

  // Drain the trailing stage loads before this workgroup's LDS is handed to
  // another, and make the list counts final.
  wait_vmcnt_lgkm0<0>();
  __builtin_amdgcn_s_barrier();
  for (int i = tid; i < kQ8Bq; i += kQ8Waves * kWave) {
    const int qi = grp * kQ8Bq + i;
    if (qi < a.nq) a.lcount[(int64_t)qi * a.nlists + chunk] = lcnt[i];
  }
}

}  // namespace

bool q8scan384_fits(const ScanArgs& a) {
  if (a.tauw != nullptr &&
      (a.tau != nullptr || a.tau_out == nullptr || a.su_w == nullptr || a.su_units != 2 * a.nchunks ||
       a.su_units > 2 * 256 || a.spt < 1 || a.qh == nullptr || a.xh == nullptr || a.dh < 8 || a.dh % 8 != 0 ||
       a.dh > 8 * 16 * 4 || a.k < 1 || a.k > 256 || a.groups != 1))
    return false;
  return a.d * 2 == kQ8Row && a.qf != nullptr && a.qmeta != nullptr && a.bmeta != nullptr && a.nlists == a.nchunks;
}

hipError_t launch_q8scan384(const ScanArgs& a, int grid, hipStream_t s) {
  if (!q8scan384_fits(a)) return hipErrorInvalidValue;
  // with sampling in the scan, workgroup q computes query q's threshold
  if (a.tauw != nullptr && (grid < a.nq || grid < a.nchunks)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(q8scan384_kernel, dim3(grid), dim3(kQ8Waves * kWave), 0, s, a);
  return hipGetLastError();
}

}  // namespace cvs
