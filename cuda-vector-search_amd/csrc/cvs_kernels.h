// Host-visible kernel argument blocks and launchers (internal to libcvs_hip.so).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cvs {

// What the scan kernel does with each score tile.
enum ScanMode : int {
  kAppend = 0,    // filter against a threshold, append survivors to per-wave candidate lists
  kMax = 1,       // sample pass: per-(query, unit) maxima over disjoint row sets
  kStoreF32 = 2,  // write the full score matrix (fp32)
  kStoreF16 = 3,  // write the full score matrix (fp16)
  kAppendQ8 = 4,  // int8 pre-filter: int8 rows x int8 queries, append rows whose score
                  // upper bound reaches the threshold (no compaction; full lists overflow)
  kMaxQ8 = 5,     // int8 sample pass: per-(query, unit) largest approximate score
                  // A = s_q s_b sum(q~ x~) over disjoint row sets, and its row
  kTopK = 6,      // no threshold: each lane keeps the k <= 16 best of its own scores of
                  // each query in registers (a running top-k) and appends them at the end
  kAppendIn = 7,  // kAppend with its own sampling: each workgroup publishes the maxima of
                  // its first tile as sampling units, threshold workgroups take each
                  // query's threshold from them, and every workgroup filters with it
};

// One tile of corpus rows is scored against a group of queries by one
// 256-thread workgroup.  Queries are split across the 4 waves (QS ways) and the
// tile's rows across the rest (RS = 4/QS ways).  Queries stay in VGPRs for the
// whole launch; the corpus streams through LDS in 64-column stages.
struct ScanArgs {
  const _Float16* q;  // [nq, d] fp16, row-major, d % 64 == 0
  const _Float16* x;  // [n, d]  fp16, row-major
  int64_t n;
  int nq;
  int d;
  int groups;         // query groups (gridwise); group g owns queries [g*bq, (g+1)*bq)
  int nchunks;        // corpus chunks per query group
  int64_t ntiles;     // ceil(n / tile_rows)
  int64_t tpc;        // tiles per chunk
  int xcd_pair;       // 1: map workgroups so a chunk's query groups share an XCD
  // kAppend
  const float* tau;   // [nq] initial thresholds, or null for -inf
  // kAppend, small batches: when not null (and tau null), each query's initial
  // threshold is the k-th largest of its units_in <= 64 sampling maxima
  // umax_in[q * units_in ..], found by the scan itself
  const float* umax_in;
  int units_in;
  float* lv;          // [nq, nlists, cap] candidate scores
  int* li;            // [nq, nlists, cap] candidate row ids
  int* lcount;        // [nq, nlists]
  int nlists;         // nchunks * RS
  int cap;            // list capacity (power of two, >= k + rows per wave per tile)
  int k;
  // kMax
  float* umax;        // [nq, units]
  int* uarg;          // kMaxQ8: [nq, units] the (companion) row of each unit's maximum; with agg == 1
                      // and perm (below) not null, its corpus row perm[row]
  int nsample;        // sampling workgroups per query group
  int spt;            // consecutive tiles sampled by each of them
  int agg;            // 1: one unit per (workgroup, row split, lane group) over all its tiles;
                      // 2: one unit per workgroup (units = nsample)
  int units;          // units per query = nsample * (agg ? 1 : spt) * units_per_tile
  signed char* qq_out;  // kMax: when not null, also quantise the queries for the int8 pre-filter:
  float4* qmeta_out;    //   qq_out[nq, dq] int8 rows and qmeta_out[nq] (see cvs_q8_row.h),
  signed char* qf_out;  //   and the same bytes in fragment order into qf_out (q8_frag_offset)
  int dq;
  // kStore*
  void* out;          // [nq, n]
  // kAppendQ8 (q, x are int8 rows viewed as 2-byte units: d = row bytes / 2)
  const float4* qmeta;  // [nq] (s_q, |q^|_2 up, |e_q|_2 up, 0): query scale and residual norms
  const signed char* qf;  // the int8 queries in fragment order (q8_frag_offset): what the MFMAs load
  const float4* bmeta;  // [ceil(n/64)] (s_b, max |f_r|_2 up, max |x_r|_2 up, 0) per 64-row block
  float gamma;          // relative slack for fp32 rounding of the scores: (3d + 8) * 2^-24
  // Sampling and thresholds inside the lean int8 scan (cvs_tau_group.h): when
  // tauw is not null (tau null), each scanning workgroup first samples the
  // first spt tiles of its chunk into su_w [nq, su_units] (one unit word per
  // (query, row half), su_units = 2 * nchunks), then computes a threshold
  // per query from those units by exact rescoring against the fp16 query
  // rows qh and corpus xh (dh halfs per row; perm: companion -> corpus row),
  // publishes it in tauw[q] and tau_out[q], and scans.  tauw and su_w are
  // zeroed by the query quantisation that runs before the scan.
  // The fp16 scan in mode kAppendIn uses tauw, tau_out (may be null), su_w and
  // su_units (= nchunks * row splits, or nchunks * lane groups without row
  // splits: the maxima of each workgroup's first tile, (1 << 32) |
  // float_order(max)) the same way, with the thresholds taken by the grid's
  // extra workgroups; launch_scan_in_prep clears them first, and writes qfh.
  unsigned long long* tauw;
  float* tau_out;
  unsigned long long* su_w;
  int su_units;
  const _Float16* qh;
  const _Float16* xh;
  int dh;
  int no_wait;  // tests only (CVS_FLAG_TAU_NOWAIT): the waits above give up at once
  const int* perm;
  // kAppendIn: the fp16 queries in fragment order (q8_frag_offset with d / 16
  // k-steps of 16 halfs): the MFMAs' B operands, 1 KiB of contiguous memory per
  // wave and k-step
  const _Float16* qfh;
};

// Batch-1 GEMV: one query, rows split across waves, 8 lanes per row.
struct GemvArgs {
  const _Float16* q;  // [1, d]
  const _Float16* x;  // [n, d]
  int64_t n;
  int d;
  int64_t rows_per_wave;
  const float* tau;   // [1] or null
  float* lv;
  int* li;
  int* lcount;        // [nlists]
  int nlists;         // total waves
  int cap;
  int k;
  float* umax;        // kMax: [units], upb per sampled 64-row block
  int* uarg;          // kMaxQ8: [units] the (companion) row of each unit's maximum
  int nsample;        // kMax: sampled 64-row blocks (one per wave)
  int upb;            // kMax: units per block, 8 (rows mod 8) or 1 (the block)
  int units;
  int mode;           // kAppend, kMax, kAppendQ8 or kMaxQ8 (the largest approximate score, int8)
  // kAppendQ8: q and x are int8 rows of d bytes (d = 384, 768 or 1536); the
  // filter uses the score upper bound as the scan's kAppendQ8 does
  const float4* qmeta;  // [1]
  const float4* bmeta;  // [ceil(n/64)]
  float gamma;
};

// Row top-k, first stage: one workgroup per (row, chunk of `len` columns).
struct RowTopkArgs {
  const float* scores;  // [rows, n] fp32
  int64_t n;
  int64_t len;          // columns per chunk
  int chunks;           // chunks per row (ceil(n / len))
  int k;
  float* out_v;         // [rows * chunks, k]
  void* out_i;          // [rows * chunks, k] int32 column ids (int64 when ids64)
  int ids64;
};

// Row preparation: dst[r, :d] = src[r, :d] (scaled to unit L2 norm when
// normalize), dst[r, d:width] = 0.
struct PrepArgs {
  const _Float16* src;
  _Float16* dst;
  int64_t n;
  int64_t src_stride;  // elements between source rows (>= d)
  int d;
  int dst_width;       // elements per destination row (>= d)
  int normalize;
};

// Exact selection over candidate lists: one workgroup per query.
struct SelectArgs {
  const float* lv;     // [nq, nlists, cap]
  const int* li;       // [nq, nlists, cap] or null (id = flat position)
  const int* lcount;   // [nq, nlists] or null (every list holds `cap` entries)
  int nlists;
  int cap;
  int k;
  float* out_v;        // [nq, k] (final mode)
  void* out_i;         // [nq, k] int32, or int64 when ids64 (final mode)
  int ids64;
  float* tau;          // [nq]    (threshold mode: score of the k-th best)
  // rescore mode: lv holds each candidate's score upper bound; exact fp16
  // scores are recomputed here.  A list whose count exceeds cap overflowed in the scan and
  // stands for every row of its range, all of which are rescored.
  const _Float16* q;   // [nq, d]
  const _Float16* x;   // [n, d]
  int64_t n;
  int d;
  int64_t ntiles, tpc; // the scan's tiles and tiles per chunk
  int tile_rows, wave_rows, rsplits;  // list L = chunk * rsplits + r
  int exact;           // 1: rescore_kernel has already replaced the bounds by exact scores
  int lpb;             // rescore kernel: lists per workgroup
  // rescore kernel: candidates whose exact score is below the sampled
  // threshold by more than the fp32 rounding slack are dropped
  const float* tau_in;    // [nq] sampled thresholds, or null (keep everything)
  const float4* qmeta;    // [nq] (s_q, |q^|, |e|, 0)
  const float* xmax;      // max |x_r|_2 over the corpus (rounded up)
  float gamma;            // d * 2^-24 (one rounding per accumulated term)
  // threshold mode, int8 pre-filter: also quantise query row q (q, d above)
  // into qq_out[q * dq ..] and qmeta_out[q] (when qq_out is not null), and
  // in fragment order into qf_out (q8_frag_offset; when qf_out is not null)
  signed char* qq_out;
  float4* qmeta_out;
  signed char* qf_out;
  int dq;
  // rescore mode: list entries and list ranges are rows of the int8 companion,
  // whose row r is corpus row perm[r] (null: the identity)
  const int* perm;
};

// int8 companion of an fp16 corpus: rows ordered by their largest magnitude
// and quantised per 64-row block.
struct Q8BuildArgs {
  const _Float16* x;   // [n, d]
  int64_t n;
  int d;
  int dq;              // int8 row bytes (>= d, multiple of 128); columns d..dq are zero
  signed char* xq;     // [ceil(n/64)*64, dq]
  float4* bmeta;       // [ceil(n/64)]
  float* xmax;         // max over blocks of max|x_r|_2
  int* perm;           // [ceil(n/64)*64]: companion row r holds corpus row perm[r] (r < n; perm[r] = r past n)
};

// int8 queries: per-query scale and residual norms.
struct Q8QueryArgs {
  const _Float16* q;   // [nq, d]
  int64_t nq;
  int d;
  int dq;
  signed char* qq;     // [nq, dq]
  float4* qmeta;       // [nq]
  signed char* qf;     // when not null: the same bytes in fragment order (q8_frag_offset), 32 * ceil(nq / 32) * dq bytes
  unsigned long long* zero;  // words [0, nzero) set to 0 (the lean int8 scan's unit and threshold words)
  int64_t nzero;
};

// Scan configurations: MFMA shape ms (16 or 32), queries per wave 16*... = ms*qb,
// tile rows = rs*rb*ms, widest row = ksmax * (ms == 16 ? 32 : 16); ksmax = 0:
// rows of any width (queries staged through LDS instead of held in registers).
// Row splits of a scan configuration (waves = qs * rs): 4 waves, one per SIMD,
// except 8 (two per SIMD) for qs = 8.
constexpr int scan_row_splits(int qs) { return qs >= 4 ? 1 : 4 / qs; }
constexpr int scan_waves(int qs) { return qs * scan_row_splits(qs); }

struct ScanCfg {
  int ms, qs, qb, rb, ksmax;
  int bq() const { return qs * ms * qb; }
  int rs() const { return scan_row_splits(qs); }
  int tile_rows() const { return rs() * rb * ms; }
  int wave_rows() const { return rb * ms; }
  int dmax() const { return ksmax * (ms == 16 ? 32 : 16); }  // 0: no limit
  int units_per_tile() const { return rs() * (64 / ms); }
};

// Returns hipErrorInvalidValue when no kernel is instantiated for (cfg, mode).
hipError_t launch_scan(const ScanCfg& cfg, int mode, const ScanArgs& a, int grid, hipStream_t s);
// Mode kTopK: instantiated for cfg {32, 1, 1, 1, 24} only (batches <= 32, width <= 384).
bool scan_topk_available(const ScanCfg& cfg, int64_t d, int64_t k);
hipError_t launch_scan_topk(const ScanCfg& cfg, const ScanArgs& a, int grid, hipStream_t s);
// Mode kAppendIn: instantiated for full-width (d = 384) configs {32, 1, 1, 1, 24},
// {32, 1, 2, 1, 24}, {32, 4, 1, 2, 24} and {32, 8, 1, 2, 24}, one query group.  The grid
// is nchunks scanning workgroups and then ceil(nq / scan_waves(qs)) threshold workgroups
// (one query per wave), all resident together.
bool scan_in_available(const ScanCfg& cfg, int64_t d);
hipError_t launch_scan_in(const ScanCfg& cfg, const ScanArgs& a, int grid, hipStream_t s);
// Before a kAppendIn scan: sets nwords 64-bit words to zero (the unit and
// threshold words it waits on) and writes the queries q [nq, d] (d = 384) in
// fragment order into qfh (ceil(nq / 32) * 32 * d halfs).
hipError_t launch_scan_in_prep(const _Float16* q, int nq, int d, _Float16* qfh, unsigned long long* words, int64_t nwords,
                               hipStream_t s);
// int8 scan of 384-byte rows at 256 queries per workgroup (cfg {32, 8, 1, 2, 12}):
// the same lists as launch_scan(cfg, kAppendQ8, ...), from a leaner kernel.
bool q8scan384_fits(const ScanArgs& a);
hipError_t launch_q8scan384(const ScanArgs& a, int grid, hipStream_t s);
hipError_t launch_gemv(const GemvArgs& a, int grid, hipStream_t s);  // any d % 64 == 0 (int8: 384/768/1536 bytes)
// mode 0 final, 1 threshold, 2 rescore, 5 threshold from an int8 sampling pass
// (lv / li: each unit's approximate maximum and its companion row, cap units)
hipError_t launch_select(int mode, const SelectArgs& a, int nq, hipStream_t s);
hipError_t launch_rescore(const SelectArgs& a, int nq, hipStream_t s);
hipError_t launch_prep(const PrepArgs& a, hipStream_t s);
hipError_t launch_rowtopk(const RowTopkArgs& a, int blocks, hipStream_t s);
hipError_t launch_q8_build(const Q8BuildArgs& a, hipStream_t s);
hipError_t launch_q8_queries(const Q8QueryArgs& a, hipStream_t s);

bool scan_cfg_available(const ScanCfg& cfg, int mode);

constexpr int kSelectMaxLists = 8192;
constexpr int kMaxCap = 512;  // largest candidate-list capacity (k <= 256)
constexpr int kSelectMaxK = 1024;  // largest k of the select kernel (row top-k of a score matrix)

}  // namespace cvs
