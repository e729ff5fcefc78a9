// Q-stationary MFMA scan: scores one query group against a run of corpus tiles.
//
// Replaces the score tile + fused top-k of csrc/kernels.cu:123-177 and
// kernels.cu:313-371 (and the score kernel, kernels.cu:285-311), re-designed
// for gfx950:
//
//  * 256 threads = 4 wave64s, one per SIMD.  Queries are split QS ways across
//    the waves and tile rows RS = 4/QS ways.  Each wave keeps its QW = 16*QB
//    queries as MFMA B fragments in VGPRs for the whole launch (loaded once), so
//    the corpus is the only operand that streams.
//  * Corpus rows stream HBM -> LDS with global_load_lds_dwordx4 (no VGPR
//    staging), in 64-column stages.  Each 1 KB block of a stage is exactly one
//    MFMA A fragment (16 rows x 32 columns) in lane order, so the ds_read_b128
//    that feeds v_mfma_f32_16x16x32_f16 is contiguous and conflict free.
//    NBUF stages are in flight (about 56 KB per CU); waits are explicit vmcnt
//    counts because the compiler does not track LDS-DMA dependencies.
//  * Scores never leave VGPRs.  kAppend filters them against a per-query
//    threshold and appends survivors to per-wave candidate lists (exact top-k
//    is taken later by the select kernel); kMax records per-unit maxima for the
//    sampling pre-pass that produces those thresholds; kStore* writes the full
//    score matrix (Index.scores / twopass).
//
// MFMA layout used (v_mfma_f32_16x16x32_f16, A = 16x32 corpus rows, B = 32x16
// queries): lane l supplies A[l%16][8*(l/16)..+7] and B[8*(l/16)..+7][l%16] and
// receives D[4*(l/16)+i][l%16], i = 0..3.  Any consistent k-permutation of A
// and B gives the same dot products, so only the D layout is load-bearing.
#include "cvs_common.h"
#include "cvs_kernels.h"

namespace cvs {

namespace {

template <int QS, int QB, int RB, int KSMAX, int MODE>
__global__ __launch_bounds__(kBlock, 1) void scan_kernel(ScanArgs a) {
  constexpr int RS = 4 / QS;
  constexpr int QW = 16 * QB;
  constexpr int BQ = QS * QW;
  constexpr int TRB = RS * RB;      // 16-row blocks per tile
  constexpr int TR = TRB * 16;      // tile rows
  constexpr int FPS = TRB * 2;      // A fragments per 64-column stage
  static_assert(FPS % 4 == 0, "every wave must issue the same number of stage loads");
  constexpr int LPW = FPS / 4;      // stage loads per wave
  constexpr int STAGE = FPS * 1024;
  constexpr int NBUF = (56 * 1024) / STAGE + 1;
  static_assert((NBUF - 2) * LPW < 64, "vmcnt budget");
  constexpr int NCMAX = KSMAX / 2;  // 64-column stages per tile (max)

  __shared__ __attribute__((aligned(1024))) unsigned char smem[NBUF * STAGE];
  __shared__ int lcnt[RS][BQ];
  // Per-wave sort area for the (rare) list compaction; capacity <= kMaxCap.
  __shared__ uint64_t sortbuf[MODE == kAppend ? 4 * kMaxCap : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int qs = w % QS;
  const int rs = w / QS;
  const int c16 = lane & 15;
  const int g = lane >> 4;

  // Workgroup -> (query group, chunk).  With xcd_pair, consecutive workgroups on
  // one XCD (ids i, i+8, ...) take the query groups of one chunk so that its
  // corpus rows are fetched from HBM once and re-read from that XCD's L2.
  int grp, chunk;
  {
    const int id = blockIdx.x;
    if (MODE != kMax && a.xcd_pair) {
      const int slot = id >> 3;
      grp = slot % a.groups;
      chunk = (slot / a.groups) * 8 + (id & 7);
    } else {
      grp = id % a.groups;
      chunk = id / a.groups;
    }
  }
  int64_t t_begin, t_end;
  if (MODE == kMax) {
    t_begin = ((2 * (int64_t)chunk + 1) * a.ntiles) / (2 * (int64_t)a.nsample);
    t_end = t_begin + 1;
  } else {
    t_begin = (int64_t)chunk * a.tpc;
    t_end = t_begin + a.tpc < a.ntiles ? t_begin + a.tpc : a.ntiles;
  }

  const int d = a.d;
  const int nc = d >> 6;
  const int64_t n = a.n;
  const int qwave0 = grp * BQ + qs * QW;

  // Query fragments (B operand), resident for the whole launch.
  half8 qf[QB][KSMAX];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int qi = qwave0 + qb * 16 + c16;
#pragma unroll
    for (int ks = 0; ks < KSMAX; ++ks) {
      half8 v = {0, 0, 0, 0, 0, 0, 0, 0};
      if (qi < a.nq && ks * 32 < d) v = *(const half8*)(a.q + (int64_t)qi * d + ks * 32 + g * 8);
      qf[qb][ks] = v;
    }
  }

  float thr[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int qi = qwave0 + qb * 16 + c16;
    thr[qb] = (qi >= a.nq) ? __builtin_inff() : (a.tau ? a.tau[qi] : -__builtin_inff());
  }
  if (MODE == kAppend) {
    for (int i = tid; i < RS * BQ; i += kBlock) (&lcnt[0][0])[i] = 0;
  }

  // Stage issue cursor (runs NBUF-1 stages ahead of the compute cursor).  Stages
  // past the end of this workgroup's range load a clamped, valid row so every
  // wave always has the same number of loads in flight.
  int64_t it_t = t_begin;
  int it_c = 0;
  int it_buf = 0;
  auto issue_next = [&]() {
    unsigned char* buf = smem + it_buf * STAGE;
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
      const int f = w + 4 * j;
      const int rbt = f % TRB;
      const int kk = f / TRB;
      int64_t row = it_t * TR + rbt * 16 + c16;
      if (row >= n) row = n - 1;
      const _Float16* src = a.x + row * d + it_c * 64 + kk * 32 + g * 8;
      __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(buf + f * 1024),
                                       16, 0, 0);
    }
    if (++it_c == nc) {
      it_c = 0;
      ++it_t;
    }
    if (++it_buf == NBUF) it_buf = 0;
  };

#pragma unroll
  for (int i = 0; i < NBUF - 1; ++i) issue_next();

  int cur_buf = 0;
  for (int64_t t = t_begin; t < t_end; ++t) {
    f32x4 acc[QB][RB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) acc[qb][rb] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int c = 0; c < NCMAX; ++c) {
      if (c < nc) {
        // This wave's loads for the current stage have landed; the barrier makes
        // every wave's loads visible and retires all reads of the buffer that
        // issue_next() is about to overwrite.
        wait_vmcnt_lgkm0<(NBUF - 2) * LPW>();
        __builtin_amdgcn_s_barrier();
        issue_next();
        const unsigned char* buf = smem + cur_buf * STAGE;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          half8 af[RB];
#pragma unroll
          for (int rb = 0; rb < RB; ++rb)
            af[rb] = *(const half8*)(buf + (kk * TRB + rs * RB + rb) * 1024 + lane * 16);
#pragma unroll
          for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int qb = 0; qb < QB; ++qb)
              acc[qb][rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[rb], qf[qb][2 * c + kk],
                                                                   acc[qb][rb], 0, 0, 0);
        }
        if (++cur_buf == NBUF) cur_buf = 0;
      }
    }

    // ---- epilogue: acc[qb][rb][i] = score(query qwave0+16qb+c16, row rowb+16rb+i)
    const int64_t rowb = t * TR + (rs * RB) * 16 + g * 4;
    const bool partial = (t * TR + TR > n);
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int qi = qwave0 + qb * 16 + c16;
      float v[RB * 4];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float s = acc[qb][rb][i];
          if (partial && rowb + rb * 16 + i >= n) s = -__builtin_inff();
          v[rb * 4 + i] = s;
        }

      if (MODE == kStoreF32 || MODE == kStoreF16) {
        if (qi < a.nq) {
#pragma unroll
          for (int j = 0; j < RB * 4; ++j) {
            const int64_t row = rowb + (j / 4) * 16 + (j % 4);
            if (row < n) {
              if (MODE == kStoreF32)
                ((float*)a.out)[(int64_t)qi * n + row] = v[j];
              else
                ((_Float16*)a.out)[(int64_t)qi * n + row] = (_Float16)v[j];
            }
          }
        }
      } else if (MODE == kMax) {
        float m = v[0];
#pragma unroll
        for (int j = 1; j < RB * 4; ++j) m = fmaxf(m, v[j]);
        if (qi < a.nq) a.umax[(int64_t)qi * a.units + chunk * (RS * 4) + rs * 4 + g] = m;
      } else {  // kAppend
        float m = v[0];
#pragma unroll
        for (int j = 1; j < RB * 4; ++j) m = fmaxf(m, v[j]);
        if (__ballot(m >= thr[qb]) != 0ull) {
          const int ql = qs * QW + qb * 16 + c16;
          const int list = chunk * RS + rs;
          int my = 0;
#pragma unroll
          for (int j = 0; j < RB * 4; ++j) my += (v[j] >= thr[qb]) ? 1 : 0;
          int tot = my + __shfl_xor(my, 16);
          tot += __shfl_xor(tot, 32);
          const bool need = (qi < a.nq) && (lcnt[rs][ql] + tot > a.cap);
          uint64_t needm = __ballot(need);
          while (needm) {
            const int cq = (__ffsll((unsigned long long)needm) - 1) & 15;
            const int ql0 = qs * QW + qb * 16 + cq;
            const int64_t base0 = ((int64_t)(grp * BQ + ql0) * a.nlists + list) * a.cap;
            const int count0 = lcnt[rs][ql0];
            const float nt = wave_compact(a.lv + base0, a.li + base0, count0, a.k, sortbuf + w * kMaxCap);
            if (lane == 0) lcnt[rs][ql0] = a.k;
            if (c16 == cq) thr[qb] = fmaxf(thr[qb], nt);
            needm &= ~(0x0001000100010001ull << cq);
          }
          my = 0;
#pragma unroll
          for (int j = 0; j < RB * 4; ++j) my += (v[j] >= thr[qb]) ? 1 : 0;
          if (my > 0 && qi < a.nq) {
            int pos = atomicAdd(&lcnt[rs][ql], my);
            const int64_t base = ((int64_t)qi * a.nlists + list) * a.cap;
            float* lv = a.lv + base;
            int* li = a.li + base;
#pragma unroll
            for (int j = 0; j < RB * 4; ++j) {
              if (v[j] >= thr[qb]) {
                lv[pos] = v[j];
                li[pos] = (int)(rowb + (j / 4) * 16 + (j % 4));
                ++pos;
              }
            }
          }
        }
      }
    }
  }

  // Drain the trailing (dummy) stage loads before this workgroup's LDS can be
  // handed to another one, and make all list counts final.
  wait_vmcnt_lgkm0<0>();
  __builtin_amdgcn_s_barrier();
  if (MODE == kAppend) {
    for (int i = tid; i < RS * BQ; i += kBlock) {
      const int r = i / BQ;
      const int ql = i % BQ;
      const int qi = grp * BQ + ql;
      if (qi < a.nq) a.lcount[(int64_t)qi * a.nlists + chunk * RS + r] = lcnt[r][ql];
    }
  }
}

struct CfgKey {
  int qs, qb, rb, ksmax;
};

template <int QS, int QB, int RB, int KS>
hipError_t launch_one(int mode, const ScanArgs& a, int grid, hipStream_t s) {
  switch (mode) {
    case kAppend:
      hipLaunchKernelGGL((scan_kernel<QS, QB, RB, KS, kAppend>), dim3(grid), dim3(kBlock), 0, s, a);
      break;
    case kMax:
      hipLaunchKernelGGL((scan_kernel<QS, QB, RB, KS, kMax>), dim3(grid), dim3(kBlock), 0, s, a);
      break;
    case kStoreF32:
      hipLaunchKernelGGL((scan_kernel<QS, QB, RB, KS, kStoreF32>), dim3(grid), dim3(kBlock), 0, s, a);
      break;
    case kStoreF16:
      hipLaunchKernelGGL((scan_kernel<QS, QB, RB, KS, kStoreF16>), dim3(grid), dim3(kBlock), 0, s, a);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// The instantiated configurations: (QS, QB, RB, KSMAX).
#define CVS_SCAN_CONFIGS(X) \
  X(1, 1, 1, 12)            \
  X(1, 1, 1, 24)            \
  X(1, 1, 1, 48)            \
  X(1, 2, 1, 12)            \
  X(1, 2, 1, 24)            \
  X(2, 1, 1, 48)            \
  X(1, 4, 1, 12)            \
  X(4, 1, 2, 24)            \
  X(4, 1, 2, 48)            \
  X(4, 2, 2, 12)            \
  X(4, 2, 2, 24)            \
  X(4, 4, 4, 12)

}  // namespace

bool scan_cfg_available(const ScanCfg& c, int mode) {
  if (mode < kAppend || mode > kStoreF16) return false;
#define CVS_HAS(QS, QB, RB, KS) \
  if (c.qs == QS && c.qb == QB && c.rb == RB && c.ksmax == KS) return true;
  CVS_SCAN_CONFIGS(CVS_HAS)
#undef CVS_HAS
  return false;
}

hipError_t launch_scan(const ScanCfg& c, int mode, const ScanArgs& a, int grid, hipStream_t s) {
#define CVS_LAUNCH(QS, QB, RB, KS) \
  if (c.qs == QS && c.qb == QB && c.rb == RB && c.ksmax == KS) return launch_one<QS, QB, RB, KS>(mode, a, grid, s);
  CVS_SCAN_CONFIGS(CVS_LAUNCH)
#undef CVS_LAUNCH
  return hipErrorInvalidValue;
}

}  // namespace cvs
