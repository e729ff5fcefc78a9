/*
 * C ABI of libcvs_hip.so, the gfx950 (MI355X) exact top-k search engine.
 *
 * This is the drop-in boundary for the hot path of cuda-vector-search.  The
 * reference exposes two functions through a pybind11 extension
 * (cuda_vector_search/csrc/kernels.cu:586-592) that its Python layer calls
 * through _ext.load() (cuda_vector_search/_ext.py:24-47):
 *
 *     scores(q, x, out_fp32=True)                 kernels.cu:472-497
 *     fused_topk(q, x, k, bq=0, chunks=0)         kernels.cu:501-582
 *
 * Here the same two operations are plain C functions over raw device
 * pointers, so any FFI (ctypes, cffi, cgo, JNI) can bind them.  No torch types
 * appear in the signatures.  Conventions shared by every entry point:
 *
 *   - q is [nq, d] and x is [n, d], fp16 (IEEE binary16), row-major,
 *     contiguous, 16-byte aligned, on `device`; d is any multiple of 64 (the
 *     caller zero-pads, as index.py:27-32 does), as in the reference's
 *     check_matrix (kernels.cu:451-458).  Rows up to 1536 wide run kernels that
 *     hold the queries in registers; wider rows stage them through LDS.  The
 *     int8 pre-filter (cvs_q8_*) covers d <= 1536.
 *   - `stream` is a hipStream_t (NULL = the default stream).  Work is enqueued
 *     asynchronously on it; no entry point synchronises or allocates device
 *     memory.  Results are valid once the stream reaches them.
 *   - The return value is CVS_OK (0) or an error code; cvs_last_error() then
 *     returns a message for the calling thread (the reference raises
 *     RuntimeError with the same wording via TORCH_CHECK, kernels.cu:451-470,
 *     509-518).
 *   - Entry points are thread-safe and re-entrant (no global mutable state
 *     other than an init-once cache of device properties).
 */
#ifndef CVS_H_
#define CVS_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CVS_VERSION 100 /* 0.1.0; the Python package's __version__ mirrors it */

#define CVS_OK 0
#define CVS_ERR_INVALID 1 /* bad argument: the reference's TORCH_CHECK failures */
#define CVS_ERR_HIP 2     /* HIP runtime / launch error */

/* fused_topk flags (0 = the default plan).  Test and tuning knobs. */
#define CVS_FLAG_NO_PREPASS 1    /* skip the sampling pre-pass (threshold starts at -inf) */
#define CVS_FLAG_FORCE_PREPASS 2 /* run the pre-pass whenever it is well defined */
#define CVS_FLAG_NO_GEMV 4       /* batch 1 uses the MFMA scan instead of the GEMV path */
#define CVS_FLAG_IDS_INT64 8     /* out_i is int64 (the dtype Index.search returns, index.py:126) */
#define CVS_FLAG_TAU_LAUNCH 16   /* a sampling pass and a threshold launch of their own, not the scan's
                                    own sampling and thresholds (the 384-byte int8 scan; the fp16 scan
                                    at width 384 with one query group on a grid that fits the GPU) */
#define CVS_FLAG_REGISTER_TOPK 32 /* fp16 fused path: a running top-k per lane in registers instead of the
                                     sampled threshold (batches 2..32, widths <= 384, k <= 16) */
#define CVS_FLAG_TAU_NOWAIT 64   /* tests only: the scans' cross-workgroup waits for sampling units and
                                    thresholds give up at once (the exact fallback of a GPU shared with
                                    other work, made certain) */

/* Library version (CVS_VERSION). */
int cvs_version(void);

/* Message for the last error on the calling thread ("" if none). */
const char* cvs_last_error(void);

/* 1 if `device` is a gfx950 GPU this library can run on, else 0.
 * Replaces the capability gate of _ext.py:15-21 / kernels.cu:468-469. */
int cvs_device_supported(int device);

/*
 * Full score matrix out[i, r] = sum_j q[i, j] * x[r, j], fp32 accumulation.
 * out is [nq, n], fp32 when out_fp32 != 0, else fp16 (rounded to nearest).
 * Replaces scores() of kernels.cu:472-497 (Index.scores, index.py:133-138, and
 * the "twopass" method, index.py:127-130).
 */
int cvs_scores(const void* q, const void* x, int64_t nq, int64_t n, int64_t d, void* out,
               int out_fp32, int device, void* stream);

/*
 * Plan of cvs_fused_topk for these sizes, without running it.
 * plan_out[0] = query-block size (the reference's bq; 1 for the batch-1 GEMV
 * path), plan_out[1] = corpus chunks (lists per query for the GEMV path);
 * *workspace_bytes = device scratch the call needs.  Replaces the plan
 * heuristic of kernels.cu:499-536.  bq = 0 / chunks = 0 mean "auto"; a forced
 * bq must be 16, 32, 64, 128 or 256 and, as in the reference, satisfy
 * bq * slots(k) <= 256 with slots(k) = 1/2/4/8 for k <= 32/64/128/256; a forced
 * chunks >= 1 is clamped to what the corpus allows.
 */
int cvs_fused_plan(int64_t nq, int64_t n, int64_t d, int64_t k, int64_t bq, int64_t chunks,
                   int flags, int device, int64_t* plan_out, int64_t* workspace_bytes);

/*
 * Exact top-k by inner product: for each query, the k rows with the largest
 * fp32-accumulated score, sorted by score descending and then row id
 * ascending.  out_v is [nq, k] fp32, out_i is [nq, k] int32 (int64 with
 * CVS_FLAG_IDS_INT64).  Requires 1 <= k <= 256 and k <= n.  `workspace`
 * (256-byte aligned) must hold at least
 * the bytes cvs_fused_plan reports for the same arguments; its contents need
 * no initialisation.  plan_out (may be NULL) receives the plan as in
 * cvs_fused_plan.  Replaces fused_topk() of kernels.cu:501-582 (Index.search
 * method "fused", index.py:123-126).
 */
int cvs_fused_topk(const void* q, const void* x, int64_t nq, int64_t n, int64_t d, int64_t k,
                   int64_t bq, int64_t chunks, int flags, void* workspace, int64_t workspace_bytes,
                   float* out_v, void* out_i, int64_t* plan_out, int device, void* stream);

/*
 * Diagnostic twin of cvs_fused_topk (no counterpart in the reference): runs
 * exactly the same launches, records a HIP event on `stream` between them,
 * waits for the last one and writes the elapsed milliseconds of each pipeline
 * stage to stage_ms[0..3]: sampling pre-pass, threshold select, scan (or
 * batch-1 GEMV), final select (0 for a stage the plan skips).  Used by the
 * benchmark to time the dominant kernel on the stream it runs on.  Unlike
 * cvs_fused_topk it blocks until the work is done.
 */
int cvs_fused_topk_timed(const void* q, const void* x, int64_t nq, int64_t n, int64_t d, int64_t k,
                         int64_t bq, int64_t chunks, int flags, void* workspace,
                         int64_t workspace_bytes, float* out_v, void* out_i, int64_t* plan_out,
                         int device, void* stream, float* stage_ms);

/*
 * Non-blocking diagnostic twin of cvs_fused_topk (no counterpart in the
 * reference): runs the same launches and records the caller's five HIP events
 * marks[0..4] (hipEvent_t handles, created by the caller with timing enabled)
 * on `stream` around the four pipeline stages, in the order of
 * cvs_fused_topk_timed.  Returns without waiting, so a benchmark can time many
 * back-to-back calls and read the events afterwards.
 */
int cvs_fused_topk_marked(const void* q, const void* x, int64_t nq, int64_t n, int64_t d, int64_t k,
                          int64_t bq, int64_t chunks, int flags, void* workspace,
                          int64_t workspace_bytes, float* out_v, void* out_i, int64_t* plan_out,
                          int device, void* stream, void* const* marks);

/*
 * Allocation-free cvs_fused_topk (no counterpart in the reference).  For
 * callers that cannot allocate device memory at search time: code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc.  Same
 * arguments, results and errors as cvs_fused_topk with bq = chunks = 0 (the
 * auto plan), but the workspace is a library-owned device array of
 * CVS_NOALLOC_SCRATCH_BYTES per GPU (set up on the first call on a device,
 * held until the process ends); calls whose plan needs more (cvs_fused_plan's
 * workspace_bytes) fail with CVS_ERR_INVALID.  It calls no hipMalloc/hipFree.
 * Every call on one GPU shares that array: calls that overlap in time on one
 * GPU (other streams, other threads) race and must be serialised by the caller.
 * Covers the headline shapes (1M x 384, batch 256, k 10: 67.1 MB).
 */
#define CVS_NOALLOC_SCRATCH_BYTES (96ll << 20)
int cvs_fused_topk_noalloc(const void* q, const void* x, int64_t nq, int64_t n, int64_t d, int64_t k,
                           int flags, float* out_v, void* out_i, int64_t* plan_out, int device, void* stream);

/*
 * Exact top-k of each row of an fp32 matrix scores[nq, n] (row-major): the k
 * largest values of each row with their column indices, sorted by value
 * descending then index ascending (the fused path's order).  1 <= k <= 1024,
 * k <= n.  out_v is [nq, k] fp32, out_i [nq, k] int32 (int64 with
 * CVS_FLAG_IDS_INT64; other flag bits are ignored).  Rows are split into
 * chunks whose k best are merged by the select kernel; `workspace` holds the
 * chunk results (size from cvs_topk_rows_plan).  With cvs_scores this is
 * the exact large-k search that the reference leaves to torch (fp16 matmul +
 * torch.topk, index.py:118 / reference.py:8-15) for k > 256.
 */
int cvs_topk_rows(const float* scores, int64_t nq, int64_t n, int64_t k, int flags, void* workspace,
                  int64_t workspace_bytes, float* out_v, void* out_i, int device, void* stream);

/* Workspace bytes cvs_topk_rows needs for these sizes (0 when each row is
 * handled by one workgroup); 256-byte aligned, no initialisation needed. */
int cvs_topk_rows_plan(int64_t nq, int64_t n, int64_t k, int device, int64_t* workspace_bytes);

/*
 * Row preparation, one pass: dst[r, 0:d] = src[r, 0:d], divided by
 * max(||src[r, 0:d]||_2, 1e-12) (fp32 arithmetic, rounded once to fp16) when
 * normalize != 0, and dst[r, d:dst_width] = 0.  Rows are fp16; src rows are
 * src_stride elements apart, dst rows dst_width apart (d <= dst_width < 2^31).
 * src == dst (in place) is allowed when src_stride == dst_width; other
 * overlaps are not.  Replaces the torch sequences of index.py:35-41
 * (_normalize_) and index.py:27-32 (_pad_width) used for cosine queries on
 * every search (index.py:89-98) and for the corpus at construction
 * (index.py:56-78).
 */
int cvs_prep_rows(const void* src, void* dst, int64_t n, int64_t d, int64_t src_stride, int64_t dst_width,
                  int normalize, int device, void* stream);

/*
 * int8 pre-filter for the exact search (no counterpart in the reference, whose
 * only corpus format is the fp16 matrix of index.py:56-78; it serves the same
 * calls as cvs_fused_topk, index.py:123-126, with half the corpus bytes
 * scanned).  An int8 companion of the corpus, built once, is scanned with int8
 * MFMAs; every row whose score upper bound (int8 score + a rigorous
 * quantisation-error bound) reaches the sampled threshold is a candidate, and
 * exact fp16 scores are recomputed for the candidates that can still be in the
 * top k (the bound of the rest is below the k-th best exact score found).
 * Results are those of cvs_fused_topk (same order, same ids, fp32-accumulated
 * scores).
 *
 * cvs_q8_corpus_bytes: size of the companion of an [n, d] corpus (int8 rows of
 *   384, 768 or 1536 bytes, the smallest that holds d, plus 16 bytes per
 *   64-row block, 16 bytes for the corpus-wide maximum row norm and 4 bytes
 *   per row for the row order).
 * cvs_q8_build: writes the companion of x (d multiple of 64, <= 1536) into xq
 *   (256-byte aligned, at least cvs_q8_corpus_bytes): the rows in ascending
 *   order of their largest magnitude (stable), so that each 64-row block, which
 *   shares one int8 scale, holds rows of nearly equal range.  Rebuild it
 *   whenever x changes.  The row-order sort's keys, ids and scratch (about 14
 *   bytes per row) are placed in xq's own int8-row region before the rows
 *   are written, so the call allocates nothing.
 * cvs_q8_plan / cvs_q8_topk: as cvs_fused_plan / cvs_fused_topk (1 <= k <= 256,
 *   auto plan only; flags CVS_FLAG_IDS_INT64, and the pre-pass flags for the
 *   sampling pass), with the companion of x as xq.  plan_out[0] is the int8
 *   scan's query block, plan_out[1] its corpus chunks.
 * cvs_q8_topk_marked: as cvs_fused_topk_marked (events around: query
 *   quantisation + sampling pass, threshold select, int8 scan, rescore select;
 *   where the int8 scan samples and takes the thresholds itself, the first
 *   span is the quantisation alone and the second is empty).
 */
int cvs_q8_corpus_bytes(int64_t n, int64_t d, int64_t* bytes);
int cvs_q8_build(const void* x, int64_t n, int64_t d, void* xq, int64_t xq_bytes, int device, void* stream);
int cvs_q8_plan(int64_t nq, int64_t n, int64_t d, int64_t k, int flags, int device, int64_t* plan_out,
                int64_t* workspace_bytes);
int cvs_q8_topk(const void* q, const void* x, const void* xq, int64_t xq_bytes, int64_t nq, int64_t n, int64_t d,
                int64_t k, int flags, void* workspace, int64_t workspace_bytes, float* out_v, void* out_i,
                int64_t* plan_out, int device, void* stream);
int cvs_q8_topk_marked(const void* q, const void* x, const void* xq, int64_t xq_bytes, int64_t nq, int64_t n,
                       int64_t d, int64_t k, int flags, void* workspace, int64_t workspace_bytes, float* out_v,
                       void* out_i, int64_t* plan_out, int device, void* stream, void* const* marks);

#ifdef __cplusplus
}
#endif

#endif /* CVS_H_ */
