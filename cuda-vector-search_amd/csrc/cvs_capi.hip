// C-ABI of libcvs_hip.so: planning, validation and launch sequencing.
//
// Replaces the pybind11 host half of csrc/kernels.cu:451-592 (check_matrix,
// check_pair, scores, slots_per_lane, fused_topk, PYBIND11_MODULE).  Every entry
// point takes raw device pointers, sizes, a device index and a hipStream_t, and
// allocates nothing: the caller owns outputs and the workspace (sized by
// cvs_fused_plan).  Launches are asynchronous on the given stream; nothing here
// synchronises.  Errors are reported as a non-zero status plus a thread-local
// message (cvs_last_error), mirroring the reference's TORCH_CHECK messages.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "cvs.h"
#include "cvs_kernels.h"

using namespace cvs;

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(CVS_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

struct DevInfo {
  bool ready = false;
  bool gfx950 = false;
  int cus = 0;
  char arch[64] = {0};
};

constexpr int kMaxDevices = 64;
DevInfo g_dev[kMaxDevices];
std::mutex g_dev_mu;

int dev_info(int device, DevInfo* out) {
  if (device < 0 || device >= kMaxDevices) return fail(CVS_ERR_INVALID, "invalid device index %d", device);
  std::lock_guard<std::mutex> lock(g_dev_mu);
  DevInfo& di = g_dev[device];
  if (!di.ready) {
    hipDeviceProp_t prop;
    hipError_t e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
    di.cus = prop.multiProcessorCount;
    std::snprintf(di.arch, sizeof di.arch, "%s", prop.gcnArchName);
    di.gfx950 = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0;
    di.ready = true;
  }
  *out = di;
  return CVS_OK;
}

// Switches to `device` for the lifetime of the guard (the reference's CUDAGuard).
struct DeviceGuard {
  int prev = -1;
  bool switched = false;
  hipError_t err = hipSuccess;
  explicit DeviceGuard(int device) {
    err = hipGetDevice(&prev);
    if (err == hipSuccess && prev != device) {
      err = hipSetDevice(device);
      switched = (err == hipSuccess);
    }
  }
  ~DeviceGuard() {
    if (switched) (void)hipSetDevice(prev);
  }
};

int check_inputs(const void* q, const void* x, int64_t nq, int64_t n, int64_t d) {
  if (d <= 0 || d % 64 != 0) return fail(CVS_ERR_INVALID, "width must be a multiple of 64 (zero-pad it)");
  if (d >= INT_MAX / 2) return fail(CVS_ERR_INVALID, "width %lld is too large", (long long)d);
  if (n < 0 || n >= INT_MAX) return fail(CVS_ERR_INVALID, "corpus must have fewer than 2^31 rows");
  if (nq < 0 || nq >= INT_MAX) return fail(CVS_ERR_INVALID, "too many queries");
  if (nq > 0 && (q == nullptr || reinterpret_cast<uintptr_t>(q) % 16 != 0))
    return fail(CVS_ERR_INVALID, "queries must be 16-byte aligned");
  if (n > 0 && (x == nullptr || reinterpret_cast<uintptr_t>(x) % 16 != 0))
    return fail(CVS_ERR_INVALID, "corpus must be 16-byte aligned");
  return CVS_OK;
}

// Widest row whose query fragments the scan holds in registers.
constexpr int64_t kRegWidth = 1536;

int ks_bucket(int64_t d) { return d <= 384 ? 12 : d <= 768 ? 24 : 48; }

// Scan configuration for a query block of `bq` queries at width d (false if
// none).  32x32x16 MFMA (full-rate on gfx950) whenever the queries of a wave
// fit in registers with it; 16x16x32 for bq = 16 and for rows wider than 768.
// bq = 256 at d <= 384 runs 8 waves (32 queries each, two per SIMD), so that
// one wave's candidate epilogue and barrier waits overlap the other's MFMAs
// (measured 7% faster than 4 waves of 64 queries).  The auto plan uses it at
// d = 384 only: narrower rows run the runtime-width kernel, which spills at 256
// registers per wave and is ~2x slower than two groups of 128 queries.  Rows
// wider than kRegWidth take the ksmax = 0 kernels: both MFMA operands come from
// LDS, the queries riding in every stage beside the corpus rows, so any width
// that is a multiple of 64 works (bq <= 128).
bool cfg_for(int64_t bq, int64_t d, ScanCfg* c) {
  if (d > kRegWidth) {
    switch (bq) {
      case 16: *c = {16, 1, 1, 1, 0}; return true;
      case 32: *c = {32, 1, 1, 1, 0}; return true;
      case 64: *c = {32, 2, 1, 1, 0}; return true;
      case 128: *c = {32, 4, 1, 2, 0}; return true;
      default: return false;
    }
  }
  switch (bq) {
    case 16:
      *c = {16, 1, 1, 1, ks_bucket(d)};
      return true;
    case 32:
      if (d <= 384) { *c = {32, 1, 1, 1, 24}; return true; }
      if (d <= 768) { *c = {32, 1, 1, 1, 48}; return true; }
      *c = {16, 2, 1, 1, 48};
      return true;
    case 64:
      if (d <= 384) { *c = {32, 1, 2, 1, 24}; return true; }
      if (d <= 768) { *c = {32, 2, 1, 1, 48}; return true; }
      *c = {16, 4, 1, 2, 48};
      return true;
    case 128:
      if (d <= 384) { *c = {32, 4, 1, 2, 24}; return true; }
      if (d <= 768) { *c = {32, 4, 1, 2, 48}; return true; }
      return false;
    case 256:
      if (d <= 384) { *c = {32, 8, 1, 2, 24}; return true; }  // 8 waves, 2 per SIMD
      return false;
    default:
      return false;
  }
}

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
int64_t pow2_at_least(int64_t v) {
  int64_t p = 1;
  while (p < v) p <<= 1;
  return p;
}
int64_t align_up(int64_t v, int64_t a) { return ceil_div(v, a) * a; }

// Reference's register-state rule (kernels.cu:499,518), kept for forced plans.
int slots_per_lane(int64_t k) { return k <= 32 ? 1 : k <= 64 ? 2 : k <= 128 ? 4 : 8; }

struct Plan {
  bool gemv = false;
  ScanCfg cfg{};
  int64_t bq = 0;       // reported plan[0]
  int64_t groups = 1;
  int64_t chunks = 1;   // reported plan[1]
  int64_t tile_rows = 0, ntiles = 0, tpc = 0;
  int xcd_pair = 0;
  int64_t nlists = 0, cap = 0;
  // gemv
  int64_t gemv_grid = 0, rows_per_wave = 0;
  // sampling pre-pass
  bool prepass = false;
  bool tau_in_scan = false;  // one sampling maximum per workgroup, thresholds found by the scan
  bool topk = false;         // CVS_FLAG_REGISTER_TOPK: running top-k in registers, no pre-pass
  // sampling and thresholds inside the scan (mode kAppendIn) instead of the
  // pre-pass and its threshold select: su_units units per query, the grid's
  // sin_grid workgroups are the chunks and then the threshold workgroups
  bool sin = false;
  int64_t su_units = 0, sin_grid = 0;
  int64_t nsample = 0, spt = 1, units = 0;
  int agg = 0;
  int upb = 8;  // gemv sampling units per block
  // workspace
  int64_t off_lv = 0, off_li = 0, off_cnt = 0, off_tau = 0, off_umax = 0, off_tauw = 0, off_qfh = 0, ws_bytes = 0;
};

// sample_div: the sampling pre-pass scores about 1/sample_div of the tiles (the
// int8 pre-filter samples more densely: every candidate it keeps costs a
// random row read, so a tighter threshold pays for itself).
int make_plan(int64_t nq, int64_t n, int64_t d, int64_t k, int64_t bq, int64_t chunks, int flags,
              int cus, Plan* p, int64_t sample_div = 16, bool allow_tau_in_scan = true) {
  if (k < 1 || k > 256) return fail(CVS_ERR_INVALID, "fused_topk supports 1 <= k <= 256");
  if (k > n) return fail(CVS_ERR_INVALID, "k must not exceed the corpus size");
  if (bq < 0) return fail(CVS_ERR_INVALID, "bq must be 0 (auto) or one of 16, 32, 64, 128, 256");
  const bool forced_bq = bq > 0;
  if (forced_bq) {
    if (bq != 16 && bq != 32 && bq != 64 && bq != 128 && bq != 256)
      return fail(CVS_ERR_INVALID, "bq must be 16, 32, 64, 128 or 256");
    if (bq * slots_per_lane(k) > 256) return fail(CVS_ERR_INVALID, "bq * ceil(k/32) must be <= 256");
  }
  Plan P;
  P.gemv = (nq == 1 && !forced_bq && !(flags & CVS_FLAG_NO_GEMV));
  if (P.gemv) {
    int64_t waves = chunks > 0 ? chunks : (int64_t)cus * 16;
    waves = std::max<int64_t>(1, std::min<int64_t>({waves, kSelectMaxLists, ceil_div(n, 16)}));
    P.gemv_grid = ceil_div(waves, 4);
    waves = P.gemv_grid * 4;
    P.rows_per_wave = align_up(ceil_div(n, waves), 16);
    P.bq = 1;
    P.chunks = waves;
    P.nlists = waves;
    P.cap = std::max<int64_t>(128, pow2_at_least(k + 8));
    const int64_t nblocks = ceil_div(n, 64);
    // sampled 64-row blocks, 8 units (row classes mod 8) each
    const int64_t s = std::min<int64_t>(8192 / sample_div, std::max<int64_t>(nblocks / sample_div, ceil_div(2 * k, 8)));
    P.prepass = !(flags & CVS_FLAG_NO_PREPASS) &&
                (((flags & CVS_FLAG_FORCE_PREPASS) && s <= nblocks) || (s >= 4 && s <= nblocks / 8));
    if (P.prepass) {
      P.nsample = s;
      P.upb = (s >= 32 * k) ? 1 : 8;  // whole-block units when they are plentiful
      P.units = s * P.upb;
    }
  } else {
    if (!forced_bq) {
      bq = nq <= 16 ? 16 : nq <= 32 ? 32 : nq <= 64 ? 64 : (nq <= 128 || d != 384) ? 128 : 256;
      if ((flags & CVS_FLAG_REGISTER_TOPK) && nq <= 32) bq = 32;  // (the register top-k's 32-query block)
      ScanCfg tmp;
      while (!cfg_for(bq, d, &tmp)) bq >>= 1;
    }
    if (!cfg_for(bq, d, &P.cfg)) return fail(CVS_ERR_INVALID, "bq=%lld is not supported at width %lld", (long long)bq, (long long)d);
    P.bq = bq;
    P.groups = ceil_div(std::max<int64_t>(nq, 1), bq);
    P.tile_rows = P.cfg.tile_rows();
    P.ntiles = ceil_div(n, P.tile_rows);
    const int64_t rs = P.cfg.rs();
    const int64_t max_chunks = std::min<int64_t>({P.ntiles, 65535, kSelectMaxLists / rs});
    int64_t c;
    if (chunks > 0) {
      c = std::max<int64_t>(1, std::min<int64_t>(chunks, max_chunks));
      P.tpc = ceil_div(P.ntiles, c);
      c = ceil_div(P.ntiles, P.tpc);
    } else {
      c = std::max<int64_t>(1, ceil_div(cus, P.groups));
      c = std::min<int64_t>(c, std::max<int64_t>(1, P.ntiles / 2));
      c = std::min<int64_t>(c, max_chunks);
      if (P.groups > 1 && c >= 8) {
        // keep the XCD-aware mapping exact: chunk count a multiple of the 8 XCDs
        c = std::min<int64_t>(align_up(c, 8), (max_chunks / 8) * 8);
        P.tpc = ceil_div(P.ntiles, c);
      } else {
        P.tpc = ceil_div(P.ntiles, c);
        c = ceil_div(P.ntiles, P.tpc);
      }
    }
    P.chunks = c;
    P.xcd_pair = (P.groups > 1 && c % 8 == 0) ? 1 : 0;
    P.nlists = c * rs;
    P.cap = std::max<int64_t>(128, pow2_at_least(k + 64));
    // Sampling pre-pass: about 1/16 of the tiles, and at least 8k/upt of them
    // but at most a quarter (its threshold is the k-th best of ~upt*s unit
    // maxima, so the expected number of candidates that pass it is about
    // k * ntiles / s), run by at most one workgroup per CU, each on spt
    // consecutive tiles.
    const int64_t upt = P.cfg.units_per_tile();  // sampling units per tile
    int64_t s = std::min<int64_t>(16384 / sample_div, std::max<int64_t>(P.ntiles / sample_div, ceil_div(8 * k, upt)));
    s = std::min<int64_t>(s, (flags & CVS_FLAG_FORCE_PREPASS) ? P.ntiles : P.ntiles / 4);
    P.prepass = !(flags & CVS_FLAG_NO_PREPASS) &&
                (((flags & CVS_FLAG_FORCE_PREPASS) && s >= 1) || (s >= 4 && s * upt >= 2 * k));
    if (P.prepass) {
      const int64_t wgs = std::max<int64_t>(1, std::min<int64_t>(s, cus / P.groups));
      P.spt = std::max<int64_t>(1, s / wgs);
      P.nsample = wgs;
      // One unit per (workgroup, row split, lane group) when that still leaves
      // >= 32k units (the top k scores then almost never share a unit, so the
      // threshold is as tight as per-tile units give, from fewer values).
      P.agg = (P.spt > 1 && wgs * upt >= 32 * k) ? 1 : 0;
      P.units = wgs * (P.agg ? 1 : P.spt) * upt;
      // A single query group of at most 32 queries whose sample fits 64
      // workgroups (small corpora, small batches: all latency): up to 64
      // sampled tiles, one each, one maximum per (query, workgroup), and the
      // scan finds the k-th largest of them itself, which saves the threshold
      // select's launch.  With >= 2k workgroups about 1.15k..1.4k rows of the
      // sample pass that threshold (k when every row were its own unit).
      const int64_t s_in = std::min<int64_t>({64, (int64_t)cus, (flags & CVS_FLAG_FORCE_PREPASS) ? P.ntiles : P.ntiles / 4});
      P.tau_in_scan = allow_tau_in_scan && P.groups == 1 && bq <= 32 && s <= 64 && s_in >= 2 * k;
      if (P.tau_in_scan) {
        P.nsample = std::max<int64_t>(s, s_in);
        P.spt = 1;
        P.agg = 2;
        P.units = P.nsample;
      }
      // Sampling inside the scan (d = 384, one query group): every scanning
      // workgroup's first tile is its sample (units below), and ceil(nq / waves) more workgroups take
      // the thresholds from them, one query per wave.  Every workgroup waits
      // for others, so the whole grid must fit the GPU at once (one per CU);
      // at least 2k units per query.  Replaces the pre-pass, its threshold
      // select and their launches (small corpora: all latency).
      // Fewer chunks make room for the threshold workgroups when that costs at
      // most one more tile per workgroup (an automatic chunk count only).
      const int64_t nw = scan_waves(P.cfg.qs);
      const int64_t twg = ceil_div(nq, nw);
      int64_t c2 = P.chunks, tpc2 = P.tpc;
      if (chunks == 0 && c2 + twg > cus && cus > twg) {
        tpc2 = ceil_div(P.ntiles, cus - twg);
        c2 = ceil_div(P.ntiles, tpc2);
      }
      // one unit per (query, workgroup) when that leaves 8k of them (C1: 196
      // units for k = 10 take the threshold waves' search 1.3 us less than 784
      // per row split), else one per row split, per lane group without row
      // splits (C5: 448 units for k = 100, 2.2 us faster than 224 per workgroup:
      // the looser threshold costs more in candidates than the search saves)
      const int64_t su = c2 >= 8 * k ? c2 : c2 * (P.cfg.rs() > 1 ? P.cfg.rs() : 64 / P.cfg.ms);
      if (allow_tau_in_scan && P.groups == 1 && scan_in_available(P.cfg, d) &&
          !(flags & (CVS_FLAG_TAU_LAUNCH | CVS_FLAG_FORCE_PREPASS)) && c2 + twg <= cus && tpc2 <= P.tpc + 1 &&
          su >= 2 * k && su <= 64 * (nw == 8 ? 8 : 32)) {
        P.sin = true;
        P.tau_in_scan = false;
        P.chunks = c2;
        P.tpc = tpc2;
        P.nlists = c2 * P.cfg.rs();
        P.su_units = su;
        P.sin_grid = c2 + twg;
      }
    }
  }
  if (flags & CVS_FLAG_REGISTER_TOPK) {
    if (P.gemv || !scan_topk_available(P.cfg, d, k))
      return fail(CVS_ERR_INVALID, "the register top-k scan covers batches of 2..32 at widths <= 384 and k <= 16");
    P.topk = true;
    P.prepass = false;
    P.tau_in_scan = false;
    P.sin = false;
  }
  if (P.cap > kMaxCap) return fail(CVS_ERR_INVALID, "internal: list capacity %lld too large", (long long)P.cap);
  const int64_t lists = std::max<int64_t>(nq, 1) * P.nlists;
  int64_t off = 0;
  P.off_lv = off;
  off = align_up(off + lists * P.cap * 4, 256);
  P.off_li = off;
  off = align_up(off + lists * P.cap * 4, 256);
  P.off_cnt = off;
  off = align_up(off + lists * 4, 256);
  P.off_tau = off;
  off = align_up(off + std::max<int64_t>(nq, 1) * 4, 256);
  P.off_umax = off;
  if (P.prepass && !P.sin) off = align_up(off + std::max<int64_t>(nq, 1) * P.units * 4, 256);
  P.off_tauw = off;  // kAppendIn: threshold words, then unit words (cleared before the scan)
  if (P.sin) off = align_up(off + std::max<int64_t>(nq, 1) * (1 + P.su_units) * 8, 256);
  P.off_qfh = off;  // kAppendIn: the queries in fragment order (whole 32-query blocks)
  if (P.sin) off = align_up(off + align_up(std::max<int64_t>(nq, 1), 32) * d * 2, 256);
  P.ws_bytes = off;
  *p = P;
  return CVS_OK;
}

}  // namespace

extern "C" {

int cvs_version(void) { return CVS_VERSION; }

const char* cvs_last_error(void) { return g_err.c_str(); }

int cvs_device_supported(int device) {
  DevInfo di;
  if (dev_info(device, &di) != CVS_OK) return 0;
  return di.gfx950 ? 1 : 0;
}

int cvs_fused_plan(int64_t nq, int64_t n, int64_t d, int64_t k, int64_t bq, int64_t chunks,
                   int flags, int device, int64_t* plan_out, int64_t* workspace_bytes) {
  DevInfo di;
  int rc = dev_info(device, &di);
  if (rc != CVS_OK) return rc;
  if (d <= 0 || d % 64 != 0) return fail(CVS_ERR_INVALID, "width must be a multiple of 64 (zero-pad it)");
  if (d >= INT_MAX / 2) return fail(CVS_ERR_INVALID, "width %lld is too large", (long long)d);
  Plan P;
  rc = make_plan(nq, n, d, k, bq, chunks, flags, di.cus, &P);
  if (rc != CVS_OK) return rc;
  if (plan_out) {
    plan_out[0] = P.bq;
    plan_out[1] = P.chunks;
  }
  if (workspace_bytes) *workspace_bytes = P.ws_bytes;
  return CVS_OK;
}

}  // extern "C"

namespace {

// Records marks[i] after pipeline stage i-1 when marks != nullptr (marks[0]
// before the first launch).  Stages: 0 sample pass, 1 threshold select, 2 scan
// or GEMV, 3 final select; skipped stages get back-to-back marks.
int run_fused(const void* q, const void* x, int64_t nq, int64_t n, int64_t d, int64_t k, int64_t bq,
              int64_t chunks, int flags, void* workspace, int64_t workspace_bytes, float* out_v,
              void* out_i, int64_t* plan_out, int device, void* stream, hipEvent_t* marks) {
  DevInfo di;
  int rc = dev_info(device, &di);
  if (rc != CVS_OK) return rc;
  if (!di.gfx950) return fail(CVS_ERR_INVALID, "libcvs_hip targets gfx950 (MI355X); device %d is %s", device, di.arch);
  rc = check_inputs(q, x, nq, n, d);
  if (rc != CVS_OK) return rc;
  Plan P;
  rc = make_plan(nq, n, d, k, bq, chunks, flags, di.cus, &P);
  if (rc != CVS_OK) return rc;
  if (plan_out) {
    plan_out[0] = P.bq;
    plan_out[1] = P.chunks;
  }
  if (nq == 0) return CVS_OK;
  if (out_v == nullptr || out_i == nullptr) return fail(CVS_ERR_INVALID, "output pointers must not be null");
  if (workspace == nullptr || workspace_bytes < P.ws_bytes)
    return fail(CVS_ERR_INVALID, "workspace too small: need %lld bytes, got %lld", (long long)P.ws_bytes,
                (long long)workspace_bytes);
  if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0) return fail(CVS_ERR_INVALID, "workspace must be 256-byte aligned");

  DeviceGuard guard(device);
  if (guard.err != hipSuccess) return hip_fail(guard.err, "hipSetDevice");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  auto mark = [&](int i) {
    if (marks) (void)hipEventRecord(marks[i], s);
  };
  mark(0);
  char* ws = static_cast<char*>(workspace);
  float* lv = reinterpret_cast<float*>(ws + P.off_lv);
  int* li = reinterpret_cast<int*>(ws + P.off_li);
  int* cnt = reinterpret_cast<int*>(ws + P.off_cnt);
  float* tau = reinterpret_cast<float*>(ws + P.off_tau);
  float* umax = reinterpret_cast<float*>(ws + P.off_umax);
  const _Float16* qh = static_cast<const _Float16*>(q);
  const _Float16* xh = static_cast<const _Float16*>(x);
  hipError_t e;

  if (P.gemv) {
    GemvArgs g{};
    g.q = qh;
    g.x = xh;
    g.n = n;
    g.d = (int)d;
    g.rows_per_wave = P.rows_per_wave;
    g.k = (int)k;
    g.cap = (int)P.cap;
    if (P.prepass) {
      GemvArgs pg = g;
      pg.mode = kMax;
      pg.umax = umax;
      pg.nsample = (int)P.nsample;
      pg.upb = P.upb;
      pg.units = (int)P.units;
      e = launch_gemv(pg, (int)ceil_div(P.nsample, 4), s);
      if (e != hipSuccess) return hip_fail(e, "gemv sample pass launch");
      SelectArgs sa{};
      sa.lv = umax;
      sa.nlists = 1;
      sa.cap = (int)P.units;
      sa.k = (int)k;
      sa.tau = tau;
      mark(1);
      e = launch_select(1, sa, 1, s);
      if (e != hipSuccess) return hip_fail(e, "threshold select launch");
      mark(2);
      g.tau = tau;
    } else {
      mark(1);
      mark(2);
    }
    g.mode = kAppend;
    g.lv = lv;
    g.li = li;
    g.lcount = cnt;
    g.nlists = (int)P.nlists;
    e = launch_gemv(g, (int)P.gemv_grid, s);
    if (e != hipSuccess) return hip_fail(e, "gemv launch");
    mark(3);
  } else {
    ScanArgs a{};
    a.q = qh;
    a.x = xh;
    a.n = n;
    a.nq = (int)nq;
    a.d = (int)d;
    a.groups = (int)P.groups;
    a.nchunks = (int)P.chunks;
    a.ntiles = P.ntiles;
    a.tpc = P.tpc;
    a.xcd_pair = P.xcd_pair;
    a.k = (int)k;
    a.cap = (int)P.cap;
    if (P.sin) {  // sampling and thresholds inside the scan: clear their words, copy the queries in fragment order
      unsigned long long* tauw = reinterpret_cast<unsigned long long*>(ws + P.off_tauw);
      _Float16* qfh = reinterpret_cast<_Float16*>(ws + P.off_qfh);
      e = launch_scan_in_prep(qh, (int)nq, (int)d, qfh, tauw, nq * (1 + P.su_units), s);
      if (e != hipSuccess) return hip_fail(e, "scan prep launch");
      a.qfh = qfh;
      a.tauw = tauw;
      a.tau_out = tau;
      a.su_w = tauw + nq;
      a.su_units = (int)P.su_units;
      a.no_wait = (flags & CVS_FLAG_TAU_NOWAIT) ? 1 : 0;
      mark(1);
      mark(2);
    } else if (P.prepass) {
      ScanArgs pa = a;
      pa.umax = umax;
      pa.nsample = (int)P.nsample;
      pa.spt = (int)P.spt;
      pa.agg = P.agg;
      // two query groups of one sampled chunk on one XCD: its rows come from HBM once
      pa.xcd_pair = (P.groups > 1 && P.nsample % 8 == 0) ? 1 : 0;
      pa.units = (int)P.units;
      e = launch_scan(P.cfg, kMax, pa, (int)(P.groups * P.nsample), s);
      if (e != hipSuccess) return hip_fail(e, "sample pass launch");
      mark(1);
      if (P.tau_in_scan) {  // the scan takes the k-th largest of each query's maxima itself
        a.umax_in = umax;
        a.units_in = (int)P.units;
      } else {
        SelectArgs sa{};
        sa.lv = umax;
        sa.nlists = 1;
        sa.cap = (int)P.units;
        sa.k = (int)k;
        sa.tau = tau;
        e = launch_select(1, sa, (int)nq, s);
        if (e != hipSuccess) return hip_fail(e, "threshold select launch");
        a.tau = tau;
      }
      mark(2);
    } else {
      mark(1);
      mark(2);
    }
    a.lv = lv;
    a.li = li;
    a.lcount = cnt;
    a.nlists = (int)P.nlists;
    e = P.topk ? launch_scan_topk(P.cfg, a, (int)(P.groups * P.chunks), s)
        : P.sin ? launch_scan_in(P.cfg, a, (int)P.sin_grid, s)
                : launch_scan(P.cfg, kAppend, a, (int)(P.groups * P.chunks), s);
    if (e != hipSuccess) return hip_fail(e, "scan launch");
    mark(3);
  }
  SelectArgs fa{};
  fa.lv = lv;
  fa.li = li;
  fa.lcount = cnt;
  fa.nlists = (int)P.nlists;
  fa.cap = (int)P.cap;
  fa.k = (int)k;
  fa.out_v = out_v;
  fa.out_i = out_i;
  fa.ids64 = (flags & CVS_FLAG_IDS_INT64) ? 1 : 0;
  e = launch_select(0, fa, (int)nq, s);
  if (e != hipSuccess) return hip_fail(e, "select launch");
  mark(4);
  return CVS_OK;
}

}  // namespace

extern "C" {

int cvs_fused_topk(const void* q, const void* x, int64_t nq, int64_t n, int64_t d, int64_t k,
                   int64_t bq, int64_t chunks, int flags, void* workspace, int64_t workspace_bytes,
                   float* out_v, void* out_i, int64_t* plan_out, int device, void* stream) {
  return run_fused(q, x, nq, n, d, k, bq, chunks, flags, workspace, workspace_bytes, out_v, out_i,
                   plan_out, device, stream, nullptr);
}

int cvs_fused_topk_timed(const void* q, const void* x, int64_t nq, int64_t n, int64_t d, int64_t k,
                         int64_t bq, int64_t chunks, int flags, void* workspace,
                         int64_t workspace_bytes, float* out_v, void* out_i, int64_t* plan_out,
                         int device, void* stream, float* stage_ms) {
  if (stage_ms == nullptr) return fail(CVS_ERR_INVALID, "stage_ms must not be null");
  for (int i = 0; i < 4; ++i) stage_ms[i] = 0.f;
  DeviceGuard guard(device);
  if (guard.err != hipSuccess) return hip_fail(guard.err, "hipSetDevice");
  hipEvent_t ev[5] = {};
  for (int i = 0; i < 5; ++i) {
    hipError_t e = hipEventCreate(&ev[i]);
    if (e != hipSuccess) {
      for (int j = 0; j < i; ++j) (void)hipEventDestroy(ev[j]);
      return hip_fail(e, "hipEventCreate");
    }
  }
  int rc = run_fused(q, x, nq, n, d, k, bq, chunks, flags, workspace, workspace_bytes, out_v, out_i,
                     plan_out, device, stream, nq > 0 ? ev : nullptr);
  if (rc == CVS_OK && nq > 0) {
    hipError_t e = hipEventSynchronize(ev[4]);
    if (e != hipSuccess) rc = hip_fail(e, "hipEventSynchronize");
    for (int i = 0; rc == CVS_OK && i < 4; ++i) {
      e = hipEventElapsedTime(&stage_ms[i], ev[i], ev[i + 1]);
      if (e != hipSuccess) rc = hip_fail(e, "hipEventElapsedTime");
    }
  }
  for (int i = 0; i < 5; ++i) (void)hipEventDestroy(ev[i]);
  return rc;
}

}  // extern "C"

namespace {

// Workspace of cvs_fused_topk_noalloc: one array per GPU the library runs on,
// held until the process ends.  Its name is a host-side stand-in; host code
// uses only the device address hipGetSymbolAddress returns for the current
// device (g_scratch_ptr), taken once per device on the entry point's first call.
constexpr int64_t kScratchBytes = CVS_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

void* g_scratch_ptr[kMaxDevices] = {};
std::once_flag g_scratch_once[kMaxDevices];
hipError_t g_scratch_err[kMaxDevices] = {};

// Device address of `scratch` on `device` (the caller has made it current).
int scratch_for(int device, void** out) {
  std::call_once(g_scratch_once[device], [device] {
    void* p = nullptr;
    g_scratch_err[device] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (g_scratch_err[device] == hipSuccess) g_scratch_ptr[device] = p;
  });
  if (g_scratch_err[device] != hipSuccess) return hip_fail(g_scratch_err[device], "hipGetSymbolAddress(scratch)");
  *out = g_scratch_ptr[device];
  return CVS_OK;
}

}  // namespace

extern "C" {

int cvs_fused_topk_noalloc(const void* q, const void* x, int64_t nq, int64_t n, int64_t d, int64_t k,
                           int flags, float* out_v, void* out_i, int64_t* plan_out, int device, void* stream) {
  DevInfo di;
  int rc = dev_info(device, &di);
  if (rc != CVS_OK) return rc;
  if (!di.gfx950) return fail(CVS_ERR_INVALID, "libcvs_hip targets gfx950 (MI355X); device %d is %s", device, di.arch);
  rc = check_inputs(q, x, nq, n, d);
  if (rc != CVS_OK) return rc;
  Plan P;
  rc = make_plan(nq, n, d, k, 0, 0, flags, di.cus, &P);
  if (rc != CVS_OK) return rc;
  if (P.ws_bytes > kScratchBytes)
    return fail(CVS_ERR_INVALID,
                "the allocation-free search needs %lld bytes of workspace for these sizes, more than its "
                "%lld-byte scratch: use cvs_fused_topk with a workspace",
                (long long)P.ws_bytes, (long long)kScratchBytes);
  void* ws = nullptr;
  {
    DeviceGuard guard(device);
    if (guard.err != hipSuccess) return hip_fail(guard.err, "hipSetDevice");
    rc = scratch_for(device, &ws);
    if (rc != CVS_OK) return rc;
  }
  // The fused path needs no zeroed workspace (every list count and threshold is
  // written before it is read), so nothing is cleared here.
  return run_fused(q, x, nq, n, d, k, 0, 0, flags, ws, kScratchBytes, out_v, out_i, plan_out, device, stream,
                   nullptr);
}

int cvs_fused_topk_marked(const void* q, const void* x, int64_t nq, int64_t n, int64_t d, int64_t k,
                          int64_t bq, int64_t chunks, int flags, void* workspace,
                          int64_t workspace_bytes, float* out_v, void* out_i, int64_t* plan_out,
                          int device, void* stream, void* const* marks) {
  if (marks == nullptr) return fail(CVS_ERR_INVALID, "marks must not be null");
  hipEvent_t ev[5];
  for (int i = 0; i < 5; ++i) {
    if (marks[i] == nullptr) return fail(CVS_ERR_INVALID, "marks[%d] is null", i);
    ev[i] = reinterpret_cast<hipEvent_t>(marks[i]);
  }
  return run_fused(q, x, nq, n, d, k, bq, chunks, flags, workspace, workspace_bytes, out_v, out_i,
                   plan_out, device, stream, nq > 0 ? ev : nullptr);
}

int cvs_scores(const void* q, const void* x, int64_t nq, int64_t n, int64_t d, void* out, int out_fp32,
               int device, void* stream) {
  DevInfo di;
  int rc = dev_info(device, &di);
  if (rc != CVS_OK) return rc;
  if (!di.gfx950) return fail(CVS_ERR_INVALID, "libcvs_hip targets gfx950 (MI355X); device %d is %s", device, di.arch);
  rc = check_inputs(q, x, nq, n, d);
  if (rc != CVS_OK) return rc;
  if (nq == 0 || n == 0) return CVS_OK;
  if (out == nullptr) return fail(CVS_ERR_INVALID, "output pointer must not be null");
  // Same query blocks and chunking as the fused plan: one workgroup per CU,
  // chunks a multiple of the 8 XCDs when several query groups share them.
  ScanCfg cfg;
  int64_t bq = nq <= 16 ? 16 : nq <= 32 ? 32 : nq <= 64 ? 64 : (nq <= 128 || d != 384) ? 128 : 256;
  while (!cfg_for(bq, d, &cfg)) bq >>= 1;
  const int64_t groups = ceil_div(nq, bq);
  const int64_t ntiles = ceil_div(n, cfg.tile_rows());
  const int64_t max_chunks = std::min<int64_t>(ntiles, 65535);
  int64_t c = std::max<int64_t>(1, ceil_div(di.cus, groups));
  c = std::min<int64_t>({c, std::max<int64_t>(1, ntiles / 2), max_chunks});
  int64_t tpc;
  int xcd_pair = 0;
  if (groups > 1 && c >= 8) {
    c = std::min<int64_t>(align_up(c, 8), (max_chunks / 8) * 8);
    tpc = ceil_div(ntiles, c);
    xcd_pair = 1;
  } else {
    tpc = ceil_div(ntiles, c);
    c = ceil_div(ntiles, tpc);
  }
  if (groups * c > INT_MAX) return fail(CVS_ERR_INVALID, "too many queries");

  DeviceGuard guard(device);
  if (guard.err != hipSuccess) return hip_fail(guard.err, "hipSetDevice");
  ScanArgs a{};
  a.q = static_cast<const _Float16*>(q);
  a.x = static_cast<const _Float16*>(x);
  a.n = n;
  a.nq = (int)nq;
  a.d = (int)d;
  a.groups = (int)groups;
  a.nchunks = (int)c;
  a.ntiles = ntiles;
  a.tpc = tpc;
  a.xcd_pair = xcd_pair;
  a.out = out;
  hipError_t e = launch_scan(cfg, out_fp32 ? kStoreF32 : kStoreF16, a, (int)(groups * c),
                             reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "score kernel launch");
  return CVS_OK;
}

namespace {

// Chunks per row for cvs_topk_rows: enough workgroups to keep ~4 per CU busy,
// chunks of at least max(4096, 2k) columns, at most kSelectMaxLists of them.
int64_t rowtopk_chunks(int64_t nq, int64_t n, int64_t k, int cus) {
  const int64_t want = ceil_div(4 * (int64_t)cus, std::max<int64_t>(nq, 1));
  const int64_t most = std::max<int64_t>(1, n / std::max<int64_t>(4096, 2 * k));
  int64_t c = std::max<int64_t>(1, std::min<int64_t>({want, most, (int64_t)kSelectMaxLists}));
  const int64_t len = ceil_div(n, c);
  return ceil_div(n, len);
}

int check_topk_rows(int64_t nq, int64_t n, int64_t k) {
  if (k < 1 || k > kSelectMaxK) return fail(CVS_ERR_INVALID, "topk_rows supports 1 <= k <= %d", kSelectMaxK);
  if (k > n) return fail(CVS_ERR_INVALID, "k must not exceed the row length");
  if (n >= INT_MAX) return fail(CVS_ERR_INVALID, "rows must have fewer than 2^31 columns");
  if (nq < 0 || nq >= INT_MAX) return fail(CVS_ERR_INVALID, "too many rows");
  return CVS_OK;
}

}  // namespace

int cvs_topk_rows_plan(int64_t nq, int64_t n, int64_t k, int device, int64_t* workspace_bytes) {
  DevInfo di;
  int rc = dev_info(device, &di);
  if (rc != CVS_OK) return rc;
  rc = check_topk_rows(nq, n, k);
  if (rc != CVS_OK) return rc;
  const int64_t c = rowtopk_chunks(nq, n, k, di.cus);
  if (nq * c >= INT_MAX) return fail(CVS_ERR_INVALID, "too many rows");
  if (workspace_bytes) *workspace_bytes = c > 1 ? align_up(nq * c * k * 4, 256) * 2 : 0;
  return CVS_OK;
}

int cvs_topk_rows(const float* scores, int64_t nq, int64_t n, int64_t k, int flags, void* workspace,
                  int64_t workspace_bytes, float* out_v, void* out_i, int device, void* stream) {
  DevInfo di;
  int rc = dev_info(device, &di);
  if (rc != CVS_OK) return rc;
  if (!di.gfx950) return fail(CVS_ERR_INVALID, "libcvs_hip targets gfx950 (MI355X); device %d is %s", device, di.arch);
  rc = check_topk_rows(nq, n, k);
  if (rc != CVS_OK) return rc;
  if (nq == 0) return CVS_OK;
  if (scores == nullptr || out_v == nullptr || out_i == nullptr) return fail(CVS_ERR_INVALID, "pointers must not be null");
  if (reinterpret_cast<uintptr_t>(scores) % 4 != 0) return fail(CVS_ERR_INVALID, "scores must be 4-byte aligned");
  const int64_t c = rowtopk_chunks(nq, n, k, di.cus);
  if (nq * c >= INT_MAX) return fail(CVS_ERR_INVALID, "too many rows");
  const int64_t part = align_up(nq * c * k * 4, 256);
  if (c > 1) {
    if (workspace == nullptr || workspace_bytes < 2 * part)
      return fail(CVS_ERR_INVALID, "workspace too small: need %lld bytes, got %lld", (long long)(2 * part),
                  (long long)workspace_bytes);
    if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0) return fail(CVS_ERR_INVALID, "workspace must be 256-byte aligned");
  }
  DeviceGuard guard(device);
  if (guard.err != hipSuccess) return hip_fail(guard.err, "hipSetDevice");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int ids64 = (flags & CVS_FLAG_IDS_INT64) ? 1 : 0;
  RowTopkArgs r{};
  r.scores = scores;
  r.n = n;
  r.len = ceil_div(n, c);
  r.chunks = (int)c;
  r.k = (int)k;
  if (c == 1) {  // one chunk per row: the first stage is the answer
    r.out_v = out_v;
    r.out_i = out_i;
    r.ids64 = ids64;
    hipError_t e = launch_rowtopk(r, (int)nq, s);
    return e == hipSuccess ? CVS_OK : hip_fail(e, "row top-k launch");
  }
  char* ws = static_cast<char*>(workspace);
  r.out_v = reinterpret_cast<float*>(ws);
  r.out_i = ws + part;
  r.ids64 = 0;
  hipError_t e = launch_rowtopk(r, (int)(nq * c), s);
  if (e != hipSuccess) return hip_fail(e, "row top-k launch");
  SelectArgs sa{};  // second stage: merge the c sorted chunk lists of each row
  sa.lv = r.out_v;
  sa.li = reinterpret_cast<const int*>(r.out_i);
  sa.nlists = (int)c;
  sa.cap = (int)k;
  sa.k = (int)k;
  sa.out_v = out_v;
  sa.out_i = out_i;
  sa.ids64 = ids64;
  e = launch_select(0, sa, (int)nq, s);
  if (e != hipSuccess) return hip_fail(e, "select launch");
  return CVS_OK;
}

int cvs_prep_rows(const void* src, void* dst, int64_t n, int64_t d, int64_t src_stride, int64_t dst_width,
                  int normalize, int device, void* stream) {
  DevInfo di;
  int rc = dev_info(device, &di);
  if (rc != CVS_OK) return rc;
  if (!di.gfx950) return fail(CVS_ERR_INVALID, "libcvs_hip targets gfx950 (MI355X); device %d is %s", device, di.arch);
  if (d < 1 || d >= INT_MAX) return fail(CVS_ERR_INVALID, "row width %lld must be in [1, 2^31)", (long long)d);
  if (dst_width < d || dst_width >= INT_MAX)
    return fail(CVS_ERR_INVALID, "destination width %lld must be in [d, 2^31)", (long long)dst_width);
  if (src_stride < d) return fail(CVS_ERR_INVALID, "source row stride must be >= d");
  if (n < 0) return fail(CVS_ERR_INVALID, "row count must be >= 0");
  if (n == 0) return CVS_OK;
  if (src == nullptr || dst == nullptr) return fail(CVS_ERR_INVALID, "row pointers must not be null");
  if (reinterpret_cast<uintptr_t>(src) % 2 != 0 || reinterpret_cast<uintptr_t>(dst) % 2 != 0)
    return fail(CVS_ERR_INVALID, "rows must be fp16-aligned");
  if (src == dst && src_stride != dst_width)
    return fail(CVS_ERR_INVALID, "in-place preparation needs src_stride == dst_width");
  DeviceGuard guard(device);
  if (guard.err != hipSuccess) return hip_fail(guard.err, "hipSetDevice");
  PrepArgs a{};
  a.src = static_cast<const _Float16*>(src);
  a.dst = static_cast<_Float16*>(dst);
  a.n = n;
  a.src_stride = src_stride;
  a.d = (int)d;
  a.dst_width = (int)dst_width;
  a.normalize = normalize ? 1 : 0;
  hipError_t e = launch_prep(a, reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "row preparation launch");
  return CVS_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// int8 pre-filter (no counterpart in the reference): an int8 companion of the
// corpus is scanned instead of the fp16 rows, rows whose score upper bound
// reaches the sampled threshold are kept, and their exact fp16 scores are
// recomputed by the select kernel.  Results equal cvs_fused_topk's.

namespace {

constexpr int64_t kQ8SampleDiv = 8;
// Widest fp16 row the int8 companion covers (int8 rows of 384, 768 or 1536
// bytes; wider corpora are searched by the fp16 scan).
constexpr int64_t kQ8MaxWidth = 1536;

// From this batch size on, the select rescores the candidates itself (one
// workgroup per query, the k of largest bound first, then only those that can
// still enter); below it, a rescoring kernel over (query, list group) pairs
// keeps more CUs busy.  Wider rows cost more per rescored candidate, so the
// select's savings win earlier there (measured at 1M rows: from batch 128 at
// d = 768, batch 160-192 at d = 384).
int64_t q8_two_phase_batch(int64_t d) { return d > 384 ? 128 : 160; }

// int8 row bytes for a row of d fp16 elements: one of the widths the int8
// scan is instantiated for.
int64_t q8_row_bytes(int64_t d) { return d <= 384 ? 384 : d <= 768 ? 768 : 1536; }

// Companion layout: int8 rows [rows, dq] | block meta [nblk] float4 | max row
// norm (16 bytes) | row order perm [rows] int32 (companion row -> corpus row).
struct Q8Layout {
  int64_t dq = 0, rows = 0, nblk = 0, off_meta = 0, off_xmax = 0, off_perm = 0, bytes = 0;
};

Q8Layout q8_layout(int64_t n, int64_t d) {
  Q8Layout L;
  L.dq = q8_row_bytes(d);
  L.nblk = ceil_div(n, 64);
  L.rows = L.nblk * 64;
  L.off_meta = align_up(L.rows * L.dq, 256);
  L.off_xmax = L.off_meta + L.nblk * 16;
  L.off_perm = align_up(L.off_xmax + 16, 256);
  L.bytes = L.off_perm + L.rows * 4;
  return L;
}

struct Q8Plan {
  Plan sample;  // fp16 plan: only its sampling pre-pass (scan or GEMV) is used
  bool gemv = false;  // batch 1: int8 GEMV instead of the int8 scan
  int64_t gemv_grid = 0, rows_per_wave = 0;
  ScanCfg cfg{};
  int64_t dq = 0, bq = 0, groups = 1, chunks = 1, ntiles = 0, tpc = 0, nlists = 0, cap = 0;
  int xcd_pair = 0;
  // int8 sampling pass (scan mode kMaxQ8) over about 1/kQ8SampleDiv of the
  // int8 tiles, instead of the fp16 one (`sample`) for batches
  bool s8 = false;
  int64_t s8_tiles = 0, s8_nsample = 0, s8_spt = 1, s8_units = 0;
  int s8_agg = 0;
  // the lean 384-byte-row int8 scan (q8scan384_kernel), and whether it
  // samples and takes the thresholds itself (tau_in_scan: in_spt tiles per
  // workgroup, in_units units per query) instead of the sampling pass and
  // the threshold launch
  bool lean = false, tau_in_scan = false;
  int64_t in_spt = 0, in_units = 0;
  int64_t off_lv = 0, off_li = 0, off_cnt = 0, off_tau = 0, off_tauw = 0, off_umax = 0, off_uarg = 0, off_qq = 0,
          off_qm = 0, off_qf = 0, ws_bytes = 0;
};

int make_q8_plan(int64_t nq, int64_t n, int64_t d, int64_t k, int flags, int cus, Q8Plan* out) {
  if (d > kQ8MaxWidth)
    return fail(CVS_ERR_INVALID, "the int8 pre-filter supports widths up to %lld, not %lld", (long long)kQ8MaxWidth,
                (long long)d);
  Q8Plan P;
  int rc = make_plan(nq, n, d, k, 0, 0, flags, cus, &P.sample, kQ8SampleDiv, false);
  if (rc != CVS_OK) return rc;
  P.dq = q8_row_bytes(d);
  const int ks = (int)(P.dq / 32);
  P.gemv = (nq == 1 && !(flags & CVS_FLAG_NO_GEMV));
  if (P.gemv) {  // per-wave row ranges as the fp16 GEMV path
    int64_t waves = (int64_t)cus * 16;
    waves = std::max<int64_t>(1, std::min<int64_t>({waves, kSelectMaxLists, ceil_div(n, 16)}));
    P.gemv_grid = ceil_div(waves, 4);
    waves = P.gemv_grid * 4;
    P.rows_per_wave = align_up(ceil_div(n, waves), 16);
    P.bq = 1;
    P.chunks = waves;
    P.nlists = waves;
    P.ntiles = waves;
    P.tpc = 1;
    P.cfg = {32, 1, 1, 1, ks};  // unused (tile/row mapping below uses rows_per_wave)
  } else if (nq <= 32 || (nq <= 64 && ks == 48)) {
    P.cfg = {32, 1, 1, 1, ks};
  } else if (nq <= 64) {
    P.cfg = {32, 1, 2, 1, ks};
  } else if (nq <= 128 || ks == 48) {
    P.cfg = {32, 4, 1, 2, ks};
  } else {
    P.cfg = {32, 8, 1, 2, ks};
  }
  if (!scan_cfg_available(P.cfg, kAppendQ8)) return fail(CVS_ERR_INVALID, "internal: no int8 scan for width %lld", (long long)d);
  if (!P.gemv) {
    P.bq = P.cfg.bq();
    P.groups = ceil_div(std::max<int64_t>(nq, 1), P.bq);
    P.ntiles = ceil_div(n, P.cfg.tile_rows());
    const int64_t rs = P.cfg.rs();
    const int64_t max_chunks = std::min<int64_t>({P.ntiles, 65535, kSelectMaxLists / rs});
    int64_t c = std::max<int64_t>(1, ceil_div(cus, P.groups));
    c = std::min<int64_t>(c, std::max<int64_t>(1, P.ntiles / 2));
    c = std::min<int64_t>(c, max_chunks);
    if (P.groups > 1 && c >= 8) {
      c = std::min<int64_t>(align_up(c, 8), (max_chunks / 8) * 8);
      P.tpc = ceil_div(P.ntiles, c);
    } else {
      P.tpc = ceil_div(P.ntiles, c);
      c = ceil_div(P.ntiles, P.tpc);
    }
    P.chunks = c;
    P.xcd_pair = (P.groups > 1 && c % 8 == 0) ? 1 : 0;
    P.nlists = c * rs;
    // The int8 sampling pass: the fp16 pass's tile count and unit layout on
    // the int8 tiles (half the bytes, the int8 MFMA), with each unit's row
    // kept so that the threshold select can rescore the rows of the largest
    // maxima exactly.  A workgroup sampling several tiles keeps one unit per
    // (row split, lane group) over all of them and writes it once at the end
    // (per-tile units for k = 100 at 1M x 768 cost 7 us more in the scattered
    // stores and in the threshold select than the looser threshold costs
    // later).  At most 16 * 256 units per query (the threshold kernel's limit).
    const int64_t upt = P.cfg.units_per_tile();
    int64_t s = std::min<int64_t>(16384 / kQ8SampleDiv, std::max<int64_t>(P.ntiles / kQ8SampleDiv, ceil_div(8 * k, upt)));
    s = std::min<int64_t>(s, (flags & CVS_FLAG_FORCE_PREPASS) ? P.ntiles : P.ntiles / 4);
    P.s8 = !(flags & CVS_FLAG_NO_PREPASS) &&
           (((flags & CVS_FLAG_FORCE_PREPASS) && s >= 1) || (s >= 4 && s * upt >= 2 * k));
    if (P.s8) {
      P.s8_tiles = s;
      const int64_t wgs = std::max<int64_t>(1, std::min<int64_t>({s, cus / P.groups, (16 * 256) / upt}));
      P.s8_spt = std::max<int64_t>(1, s / wgs);
      P.s8_nsample = wgs;
      P.s8_agg = P.s8_spt > 1 ? 1 : 0;
      P.s8_units = wgs * (P.s8_agg ? 1 : P.s8_spt) * upt;
    }
  }
  if (P.gemv && P.sample.prepass && P.sample.units <= 16 * 256) {
    // batch 1: the fp16 GEMV sample's blocks and units, over the int8 companion
    P.s8 = true;
    P.s8_nsample = P.sample.nsample;
    P.s8_units = P.sample.units;
  }
  P.cap = std::max<int64_t>(128, pow2_at_least(k + 64));
  if (P.groups * P.chunks > INT_MAX) return fail(CVS_ERR_INVALID, "too many queries");
  if (!P.gemv) {
    const ScanCfg c384{32, 8, 1, 2, 12};
    P.lean = P.cfg.ms == c384.ms && P.cfg.qs == c384.qs && P.cfg.qb == c384.qb && P.cfg.rb == c384.rb &&
             P.cfg.ksmax == c384.ksmax && P.dq == 384 && P.nlists == P.chunks;
    // Sampling and thresholds in the scan: every workgroup samples the first
    // in_spt tiles of its chunk (about as many tiles in all as the sampling
    // pass would), workgroup b computes query b's threshold from all of
    // them (the grid extends past the chunks to one workgroup per query), and
    // every workgroup waits for those of its queries, so the whole grid must
    // be resident at once (one 8-wave workgroup per CU).  Two units per
    // chunk and query, at least 2k of them (unless sampling is forced).
    P.tau_in_scan = P.lean && P.s8 && !(flags & CVS_FLAG_TAU_LAUNCH) && P.groups == 1 &&
                    std::max<int64_t>(P.chunks, nq) <= cus && 2 * P.chunks <= 2 * 256 &&
                    (P.chunks >= k || (flags & CVS_FLAG_FORCE_PREPASS)) && d <= 512 && k <= 256;
    if (P.tau_in_scan) {
      P.in_spt = std::max<int64_t>(1, std::min<int64_t>(P.tpc, ceil_div(P.s8_tiles, P.chunks)));
      P.in_units = 2 * P.chunks;
    }
  }
  const int64_t nqq = std::max<int64_t>(nq, 1);
  const int64_t lists = nqq * P.nlists;
  int64_t off = 0;
  P.off_lv = off;
  off = align_up(off + lists * P.cap * 4, 256);
  P.off_li = off;
  off = align_up(off + lists * P.cap * 4, 256);
  P.off_cnt = off;
  off = align_up(off + lists * 4, 256);
  P.off_tau = off;
  off = align_up(off + nqq * 4, 256);
  P.off_tauw = off;  // threshold words, then unit words (zeroed together)
  if (P.tau_in_scan) off = align_up(off + nqq * (1 + P.in_units) * 8, 256);
  P.off_umax = off;
  if (P.s8 && !P.tau_in_scan) {
    off = align_up(off + nqq * P.s8_units * 4, 256);
    P.off_uarg = off;
    off = align_up(off + nqq * P.s8_units * 4, 256);
  } else if (P.sample.prepass) {
    off = align_up(off + nqq * P.sample.units * 4, 256);
  }
  P.off_qq = off;
  off = align_up(off + nqq * P.dq, 256);
  P.off_qm = off;
  off = align_up(off + nqq * 16, 256);
  P.off_qf = off;  // the int8 queries again, in the scans' fragment order (whole 32-query blocks)
  off = align_up(off + align_up(nqq, 32) * P.dq, 256);
  P.ws_bytes = off;
  *out = P;
  return CVS_OK;
}

int run_q8(const void* q, const void* x, const void* xq, int64_t xq_bytes, int64_t nq, int64_t n, int64_t d,
           int64_t k, int flags, void* workspace, int64_t workspace_bytes, float* out_v, void* out_i,
           int64_t* plan_out, int device, void* stream, hipEvent_t* marks) {
  DevInfo di;
  int rc = dev_info(device, &di);
  if (rc != CVS_OK) return rc;
  if (!di.gfx950) return fail(CVS_ERR_INVALID, "libcvs_hip targets gfx950 (MI355X); device %d is %s", device, di.arch);
  rc = check_inputs(q, x, nq, n, d);
  if (rc != CVS_OK) return rc;
  Q8Plan P;
  rc = make_q8_plan(nq, n, d, k, flags, di.cus, &P);
  if (rc != CVS_OK) return rc;
  if (plan_out) {
    plan_out[0] = P.bq;
    plan_out[1] = P.chunks;
  }
  if (nq == 0) return CVS_OK;
  const Q8Layout L = q8_layout(n, d);
  if (xq == nullptr || reinterpret_cast<uintptr_t>(xq) % 256 != 0)
    return fail(CVS_ERR_INVALID, "int8 corpus must be 256-byte aligned");
  if (xq_bytes < L.bytes)
    return fail(CVS_ERR_INVALID, "int8 corpus too small: need %lld bytes, got %lld", (long long)L.bytes, (long long)xq_bytes);
  if (out_v == nullptr || out_i == nullptr) return fail(CVS_ERR_INVALID, "output pointers must not be null");
  if (workspace == nullptr || workspace_bytes < P.ws_bytes)
    return fail(CVS_ERR_INVALID, "workspace too small: need %lld bytes, got %lld", (long long)P.ws_bytes,
                (long long)workspace_bytes);
  if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0) return fail(CVS_ERR_INVALID, "workspace must be 256-byte aligned");

  DeviceGuard guard(device);
  if (guard.err != hipSuccess) return hip_fail(guard.err, "hipSetDevice");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  auto mark = [&](int i) {
    if (marks) (void)hipEventRecord(marks[i], s);
  };
  mark(0);
  char* ws = static_cast<char*>(workspace);
  float* lv = reinterpret_cast<float*>(ws + P.off_lv);
  int* li = reinterpret_cast<int*>(ws + P.off_li);
  int* cnt = reinterpret_cast<int*>(ws + P.off_cnt);
  float* tau = reinterpret_cast<float*>(ws + P.off_tau);
  unsigned long long* tauw = reinterpret_cast<unsigned long long*>(ws + P.off_tauw);
  float* umax = reinterpret_cast<float*>(ws + P.off_umax);
  signed char* qq = reinterpret_cast<signed char*>(ws + P.off_qq);
  float4* qm = reinterpret_cast<float4*>(ws + P.off_qm);
  signed char* qf = reinterpret_cast<signed char*>(ws + P.off_qf);
  const _Float16* qh = static_cast<const _Float16*>(q);
  const _Float16* xh = static_cast<const _Float16*>(x);
  const Plan& S = P.sample;
  const bool fp16_sample = !P.s8 && S.prepass;
  const float4* bmeta = reinterpret_cast<const float4*>(static_cast<const char*>(xq) + L.off_meta);
  const int* perm = reinterpret_cast<const int*>(static_cast<const char*>(xq) + L.off_perm);
  const float gamma = (float)(3 * d + 8) / 16777216.0f;
  hipError_t e;

  if (!fp16_sample) {  // otherwise the threshold select quantises the queries on the way
    // (and, for sampling in the scan, clears its threshold and unit words)
    Q8QueryArgs qa{qh, nq, (int)d, (int)P.dq, qq, qm, qf, tauw, P.tau_in_scan ? nq * (1 + P.in_units) : 0};
    e = launch_q8_queries(qa, s);
    if (e != hipSuccess) return hip_fail(e, "query quantisation launch");
  }
  if (P.s8 && P.gemv) {  // the int8 GEMV sampling pass; the threshold as below
    GemvArgs pg{};
    pg.q = reinterpret_cast<const _Float16*>(qq);
    pg.x = static_cast<const _Float16*>(xq);
    pg.n = n;
    pg.d = (int)P.dq;  // int8 row bytes
    pg.k = (int)k;
    pg.mode = kMaxQ8;
    pg.umax = umax;
    pg.uarg = reinterpret_cast<int*>(ws + P.off_uarg);
    pg.nsample = (int)P.s8_nsample;
    pg.upb = S.upb;
    pg.units = (int)P.s8_units;
    pg.qmeta = qm;
    pg.bmeta = bmeta;
    pg.gamma = gamma;
    e = launch_gemv(pg, (int)ceil_div(P.s8_nsample, 4), s);
    if (e != hipSuccess) return hip_fail(e, "int8 gemv sample pass launch");
    SelectArgs ta{};
    ta.lv = umax;
    ta.li = pg.uarg;
    ta.nlists = 1;
    ta.cap = (int)P.s8_units;
    ta.k = (int)k;
    ta.tau = tau;
    ta.q = qh;
    ta.x = xh;
    ta.n = n;
    ta.d = (int)d;
    ta.perm = perm;
    mark(1);
    e = launch_select(5, ta, (int)nq, s);
    if (e != hipSuccess) return hip_fail(e, "threshold select launch");
    mark(2);
  } else if (P.tau_in_scan) {  // sampling and thresholds inside the int8 scan
    mark(1);
    mark(2);
  } else if (P.s8) {  // int8 sampling pass; the threshold from rescoring its best units' rows
    ScanArgs pa{};
    pa.q = reinterpret_cast<const _Float16*>(qq);  // int8 rows in 2-byte units
    pa.qf = qf;
    pa.x = static_cast<const _Float16*>(xq);
    pa.n = n;
    pa.nq = (int)nq;
    pa.d = (int)(P.dq / 2);
    pa.groups = (int)P.groups;
    pa.nchunks = (int)P.chunks;
    pa.ntiles = P.ntiles;
    pa.tpc = P.tpc;
    pa.k = (int)k;
    pa.cap = (int)P.cap;
    pa.umax = umax;
    pa.uarg = reinterpret_cast<int*>(ws + P.off_uarg);
    pa.nsample = (int)P.s8_nsample;
    pa.spt = (int)P.s8_spt;
    pa.agg = P.s8_agg;
    pa.xcd_pair = (P.groups > 1 && P.s8_nsample % 8 == 0) ? 1 : 0;
    pa.units = (int)P.s8_units;
    pa.qmeta = qm;
    pa.bmeta = bmeta;
    pa.gamma = gamma;
    pa.perm = P.s8_agg ? perm : nullptr;  // units' rows as corpus rows (mapped in the pass's tail)
    e = launch_scan(P.cfg, kMaxQ8, pa, (int)(P.groups * P.s8_nsample), s);
    if (e != hipSuccess) return hip_fail(e, "int8 sample pass launch");
    mark(1);
    {
      SelectArgs ta{};
      ta.lv = umax;
      ta.li = pa.uarg;
      ta.nlists = 1;
      ta.cap = (int)P.s8_units;
      ta.k = (int)k;
      ta.tau = tau;
      ta.q = qh;
      ta.x = xh;
      ta.n = n;
      ta.d = (int)d;
      ta.perm = P.s8_agg ? nullptr : perm;
      e = launch_select(5, ta, (int)nq, s);
      if (e != hipSuccess) return hip_fail(e, "threshold select launch");
    }
    mark(2);
  } else if (fp16_sample) {  // exact fp16 sampling pre-pass and threshold, as in cvs_fused_topk
    if (S.gemv) {
      GemvArgs pg{};
      pg.q = qh;
      pg.x = xh;
      pg.n = n;
      pg.d = (int)d;
      pg.rows_per_wave = S.rows_per_wave;
      pg.k = (int)k;
      pg.cap = (int)S.cap;
      pg.mode = kMax;
      pg.umax = umax;
      pg.nsample = (int)S.nsample;
      pg.upb = S.upb;
      pg.units = (int)S.units;
      e = launch_gemv(pg, (int)ceil_div(S.nsample, 4), s);
    } else {
      ScanArgs pa{};
      pa.q = qh;
      pa.x = xh;
      pa.n = n;
      pa.nq = (int)nq;
      pa.d = (int)d;
      pa.groups = (int)S.groups;
      pa.nchunks = (int)S.chunks;
      pa.ntiles = S.ntiles;
      pa.tpc = S.tpc;
      pa.k = (int)k;
      pa.cap = (int)S.cap;
      pa.umax = umax;
      pa.nsample = (int)S.nsample;
      pa.spt = (int)S.spt;
      pa.agg = S.agg;
      // two query groups of one sampled chunk on one XCD: its rows come from HBM once
      pa.xcd_pair = (S.groups > 1 && S.nsample % 8 == 0) ? 1 : 0;
      pa.units = (int)S.units;
      pa.qq_out = qq;  // the sampling scan quantises the queries on the way
      pa.qf_out = qf;
      pa.qmeta_out = qm;
      pa.dq = (int)P.dq;
      e = launch_scan(S.cfg, kMax, pa, (int)(S.groups * S.nsample), s);
    }
    if (e != hipSuccess) return hip_fail(e, "sample pass launch");
    SelectArgs sa{};
    sa.lv = umax;
    sa.nlists = 1;
    sa.cap = (int)S.units;
    sa.k = (int)k;
    sa.tau = tau;
    sa.q = qh;
    sa.d = (int)d;
    sa.qq_out = S.gemv ? qq : nullptr;  // (after a GEMV sampling pass the threshold select quantises)
    sa.qf_out = S.gemv ? qf : nullptr;
    sa.qmeta_out = qm;
    sa.dq = (int)P.dq;
    mark(1);
    e = launch_select(1, sa, (int)nq, s);
    if (e != hipSuccess) return hip_fail(e, "threshold select launch");
    mark(2);
  } else {
    mark(1);
    mark(2);
  }
  const bool have_tau = P.s8 || S.prepass;
  if (P.gemv) {
    GemvArgs g{};
    g.q = reinterpret_cast<const _Float16*>(qq);
    g.x = static_cast<const _Float16*>(xq);
    g.n = n;
    g.d = (int)P.dq;  // int8 row bytes
    g.rows_per_wave = P.rows_per_wave;
    g.tau = have_tau ? tau : nullptr;
    g.lv = lv;
    g.li = li;
    g.lcount = cnt;
    g.nlists = (int)P.nlists;
    g.cap = (int)P.cap;
    g.k = (int)k;
    g.mode = kAppendQ8;
    g.qmeta = qm;
    g.bmeta = bmeta;
    g.gamma = gamma;
    e = launch_gemv(g, (int)P.gemv_grid, s);
    if (e != hipSuccess) return hip_fail(e, "int8 gemv launch");
  } else {
    ScanArgs a{};
    a.q = reinterpret_cast<const _Float16*>(qq);  // int8 rows in 2-byte units
    a.qf = qf;
    a.x = static_cast<const _Float16*>(xq);
    a.n = n;
    a.nq = (int)nq;
    a.d = (int)(P.dq / 2);
    a.groups = (int)P.groups;
    a.nchunks = (int)P.chunks;
    a.ntiles = P.ntiles;
    a.tpc = P.tpc;
    a.xcd_pair = P.xcd_pair;
    a.tau = have_tau ? tau : nullptr;
    a.lv = lv;
    a.li = li;
    a.lcount = cnt;
    a.nlists = (int)P.nlists;
    a.cap = (int)P.cap;
    a.k = (int)k;
    a.qmeta = qm;
    a.bmeta = bmeta;
    a.gamma = gamma;
    if (P.tau_in_scan) {
      a.tau = nullptr;
      a.tauw = tauw;
      a.tau_out = tau;
      a.su_w = tauw + nq;
      a.no_wait = (flags & CVS_FLAG_TAU_NOWAIT) ? 1 : 0;
      a.su_units = (int)P.in_units;
      a.spt = (int)P.in_spt;
      a.qh = qh;
      a.xh = xh;
      a.dh = (int)d;
      a.perm = perm;  // units hold companion rows
    }
    const bool lean = P.lean && q8scan384_fits(a);
    if (P.tau_in_scan && !lean) return fail(CVS_ERR_INVALID, "internal: in-scan thresholds without the 384-byte int8 scan");
    e = lean ? launch_q8scan384(a, (int)(P.tau_in_scan ? std::max<int64_t>(P.chunks, nq) : P.groups * P.chunks), s)
             : launch_scan(P.cfg, kAppendQ8, a, (int)(P.groups * P.chunks), s);
    if (e != hipSuccess) return hip_fail(e, "int8 scan launch");
  }
  mark(3);
  SelectArgs fa{};
  fa.lv = lv;
  fa.li = li;
  fa.lcount = cnt;
  fa.nlists = (int)P.nlists;
  fa.cap = (int)P.cap;
  fa.k = (int)k;
  fa.out_v = out_v;
  fa.out_i = out_i;
  fa.ids64 = (flags & CVS_FLAG_IDS_INT64) ? 1 : 0;
  fa.q = qh;
  fa.x = xh;
  fa.n = n;
  fa.d = (int)d;
  fa.ntiles = P.ntiles;
  fa.tpc = P.tpc;
  fa.perm = perm;
  if (P.gemv) {  // list L = rows [L * rows_per_wave, (L + 1) * rows_per_wave)
    fa.tile_rows = (int)P.rows_per_wave;
    fa.wave_rows = (int)P.rows_per_wave;
    fa.rsplits = 1;
  } else {
    fa.tile_rows = P.cfg.tile_rows();
    fa.wave_rows = P.cfg.wave_rows();
    fa.rsplits = P.cfg.rs();
  }
  if (nq < q8_two_phase_batch(d)) {
    // rescoring spread over about 4 workgroups per CU, (query, group of lists)
    // each; the select then sees exact scores
    fa.exact = 1;
    fa.tau_in = have_tau ? tau : nullptr;
    fa.qmeta = qm;
    fa.xmax = reinterpret_cast<const float*>(static_cast<const char*>(xq) + L.off_xmax);
    fa.gamma = (float)d / 16777216.0f;
    fa.lpb = 256;
    while (fa.lpb > 8 && nq * ceil_div(P.nlists, fa.lpb) < 4 * (int64_t)di.cus) fa.lpb /= 2;
    e = launch_rescore(fa, (int)nq, s);
    if (e != hipSuccess) return hip_fail(e, "rescore launch");
  }
  e = launch_select(2, fa, (int)nq, s);
  if (e != hipSuccess) return hip_fail(e, "rescore select launch");
  mark(4);
  return CVS_OK;
}

}  // namespace

extern "C" {

int cvs_q8_corpus_bytes(int64_t n, int64_t d, int64_t* bytes) {
  if (bytes == nullptr) return fail(CVS_ERR_INVALID, "bytes must not be null");
  if (d <= 0 || d % 64 != 0) return fail(CVS_ERR_INVALID, "width must be a multiple of 64 (zero-pad it)");
  if (d > kQ8MaxWidth)
    return fail(CVS_ERR_INVALID, "the int8 pre-filter supports widths up to %lld, not %lld", (long long)kQ8MaxWidth,
                (long long)d);
  if (n < 1 || n >= INT_MAX) return fail(CVS_ERR_INVALID, "corpus must have between 1 and 2^31-1 rows");
  *bytes = q8_layout(n, d).bytes;
  return CVS_OK;
}

int cvs_q8_build(const void* x, int64_t n, int64_t d, void* xq, int64_t xq_bytes, int device, void* stream) {
  DevInfo di;
  int rc = dev_info(device, &di);
  if (rc != CVS_OK) return rc;
  if (!di.gfx950) return fail(CVS_ERR_INVALID, "libcvs_hip targets gfx950 (MI355X); device %d is %s", device, di.arch);
  int64_t need = 0;
  rc = cvs_q8_corpus_bytes(n, d, &need);
  if (rc != CVS_OK) return rc;
  if (x == nullptr || reinterpret_cast<uintptr_t>(x) % 16 != 0) return fail(CVS_ERR_INVALID, "corpus must be 16-byte aligned");
  if (xq == nullptr || reinterpret_cast<uintptr_t>(xq) % 256 != 0)
    return fail(CVS_ERR_INVALID, "int8 corpus must be 256-byte aligned");
  if (xq_bytes < need)
    return fail(CVS_ERR_INVALID, "int8 corpus too small: need %lld bytes, got %lld", (long long)need, (long long)xq_bytes);
  const Q8Layout L = q8_layout(n, d);
  DeviceGuard guard(device);
  if (guard.err != hipSuccess) return hip_fail(guard.err, "hipSetDevice");
  Q8BuildArgs a{static_cast<const _Float16*>(x), n, (int)d, (int)L.dq, static_cast<signed char*>(xq),
                reinterpret_cast<float4*>(static_cast<char*>(xq) + L.off_meta),
                reinterpret_cast<float*>(static_cast<char*>(xq) + L.off_xmax),
                reinterpret_cast<int*>(static_cast<char*>(xq) + L.off_perm)};
  hipError_t e = launch_q8_build(a, reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "int8 corpus build launch");
  return CVS_OK;
}

int cvs_q8_plan(int64_t nq, int64_t n, int64_t d, int64_t k, int flags, int device, int64_t* plan_out,
                int64_t* workspace_bytes) {
  DevInfo di;
  int rc = dev_info(device, &di);
  if (rc != CVS_OK) return rc;
  if (d <= 0 || d % 64 != 0) return fail(CVS_ERR_INVALID, "width must be a multiple of 64 (zero-pad it)");
  if (d > kQ8MaxWidth)
    return fail(CVS_ERR_INVALID, "the int8 pre-filter supports widths up to %lld, not %lld", (long long)kQ8MaxWidth,
                (long long)d);
  Q8Plan P;
  rc = make_q8_plan(nq, n, d, k, flags, di.cus, &P);
  if (rc != CVS_OK) return rc;
  if (plan_out) {
    plan_out[0] = P.bq;
    plan_out[1] = P.chunks;
  }
  if (workspace_bytes) *workspace_bytes = P.ws_bytes;
  return CVS_OK;
}

int cvs_q8_topk(const void* q, const void* x, const void* xq, int64_t xq_bytes, int64_t nq, int64_t n, int64_t d,
                int64_t k, int flags, void* workspace, int64_t workspace_bytes, float* out_v, void* out_i,
                int64_t* plan_out, int device, void* stream) {
  return run_q8(q, x, xq, xq_bytes, nq, n, d, k, flags, workspace, workspace_bytes, out_v, out_i, plan_out, device,
                stream, nullptr);
}

int cvs_q8_topk_marked(const void* q, const void* x, const void* xq, int64_t xq_bytes, int64_t nq, int64_t n,
                       int64_t d, int64_t k, int flags, void* workspace, int64_t workspace_bytes, float* out_v,
                       void* out_i, int64_t* plan_out, int device, void* stream, void* const* marks) {
  if (marks == nullptr) return fail(CVS_ERR_INVALID, "marks must not be null");
  hipEvent_t ev[5];
  for (int i = 0; i < 5; ++i) {
    if (marks[i] == nullptr) return fail(CVS_ERR_INVALID, "marks[%d] is null", i);
    ev[i] = reinterpret_cast<hipEvent_t>(marks[i]);
  }
  return run_q8(q, x, xq, xq_bytes, nq, n, d, k, flags, workspace, workspace_bytes, out_v, out_i, plan_out, device,
                stream, nq > 0 ? ev : nullptr);
}

}  // extern "C"
