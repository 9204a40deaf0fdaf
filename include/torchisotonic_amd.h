/*
 * torchisotonic_amd: batched weighted L2 isotonic regression on AMD MI355X (gfx950).
 *
 * The C ABI of libtorchisotonic_amd.so. Plain pointers and sizes only; every device pointer
 * is memory of the current HIP device, every launch goes on the stream passed in (a
 * hipStream_t, passed as void*), nothing synchronises the host, and the library never
 * allocates device memory: the caller allocates outputs and the workspace whose size the
 * *_workspace calls report. Functions return TI_OK (0) or a TI_E* code; ti_last_error()
 * then holds a message for the calling thread.
 *
 * Layouts. A problem set is [batch, n] row-major and contiguous, dtype float32 or float64;
 * weights, when given, have the same shape and dtype. The block partition ("starts") is a bit
 * array: row b owns ti_starts_words(1, n) 32-bit words starting at word b * that count; bit i
 * of the row (word i / 32, bit i % 32) is set where a block of the fit starts. Element 0 is
 * always a start.
 *
 * Replaces the reference's operator library (reference src/torchisotonic/csrc/ops.cpp:45-51
 * schemas, ops_tiles.cu:8-11 CUDA registrations).
 */
#ifndef TORCHISOTONIC_AMD_H
#define TORCHISOTONIC_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TI_ABI_VERSION 10

/* dtype codes */
#define TI_F32 0
#define TI_F64 1

/* status codes */
#define TI_OK 0
#define TI_EINVAL 1     /* a null pointer, a negative size, an inconsistent argument */
#define TI_EDTYPE 2     /* a dtype code other than TI_F32 / TI_F64 */
#define TI_ESIZE 3      /* n >= 2^31 - 1, or a row count the grid cannot hold */
#define TI_EWORKSPACE 4 /* workspace missing or smaller than *_workspace reported */
#define TI_ELAUNCH 5    /* the HIP runtime rejected a launch */

/* flag bits */
#define TI_INCREASING 1u /* non-decreasing fit (else non-increasing: minus the fit of -y) */
#define TI_EXACT 2u      /* reference's exact= flag; this library is always exact (see ti_fwd) */
#define TI_CLIP_MIN 4u   /* clamp the fit from below at y_min */
#define TI_CLIP_MAX 8u   /* clamp the fit from above at y_max */
/* A hint for rows over one tile (ti_fwd and its variants; ignored elsewhere): the fit is written
   with non-temporal stores, its cache lines leaving for memory as they are written, for a caller
   whose next kernels read other data (a backward): they then do not wait behind its write-back.
   The results are the same with or without it. */
#define TI_STREAM_OUT 16u
/* A test hook (ti_fwd and its variants, float32 rows over 32 elements): the repair that makes
   each final hull convex in its stored float64 values skips its parallel removal passes and
   finishes every row it repairs with its one-pass sequential monotone chain, the form it
   otherwise takes only after a cascade of removals longer than its pass limit. The results are
   the same with or without it. */
#define TI_REPAIR_CHAIN 32u

/* The ABI version this library was built with (TI_ABI_VERSION). */
int ti_abi_version(void);

/* The last error message of the calling thread ("" if none). */
const char* ti_last_error(void);

/* Number of 32-bit words of the starts bit array of a [batch, n] problem set. */
int64_t ti_starts_words(int64_t batch, int64_t n);

/* Bytes of device workspace ti_fwd needs for this problem set (0 when none): rows of more than
 * 32 elements take a vertex store of a slot per element and small arrays, and a batch whose upper
 * merge levels have few parents (fewer than 256 rows of 1e6 elements, say) a second store. */
int ti_fwd_workspace(int64_t batch, int64_t n, int dtype, int weighted, size_t* bytes);

/* Diagnostic: the kernel geometry ti_fwd takes for rows of more than 32 elements - elements per
 * span of its first kernel (one lane builds each span's hull), the merge launches that follow
 * it, and the rows per wave of the first kernel (1: a wave holds spans of one row). Rows of at
 * most 32 elements report 0, 0, 0. No counterpart in the reference: tests use it to show which
 * geometry a case exercises. */
int ti_fwd_geometry(int64_t batch, int64_t n, int weighted, int64_t* span0, int* levels,
                    int* rows_per_wave);

/*
 * The isotonic fit of every row of y, and optionally its block partition.
 * Replaces torchisotonic::isotonic_tiles (reference ops.cpp:47-49, implementation
 * tiles.cuh:1923-1959), with the clamp the reference applies afterwards in Python
 * (reference _api.py:68-69) fused in.
 *
 *   y       [batch, n] input (dtype), no NaN handling needed by the caller: a row holding a
 *           NaN comes back all NaN with starts [1, 0, ...] (reference pava.h:29-38).
 *   w       [batch, n] positive weights, or NULL for weights of one.
 *   out     [batch, n] the fit, clamped to [y_min, y_max] where TI_CLIP_* is set (a clamp
 *           with y_min > y_max gives y_max, as torch.clamp does). May not alias y or w.
 *   starts  ti_starts_words(batch, n) words, or NULL when the partition is not wanted.
 *   bad_weight  one device word, or NULL: when w is given, the kernels set it to a nonzero
 *           value (and never clear it) if some weight is not > 0, NaN included. This fuses
 *           the reference's separate check bool((w > 0).all()) (reference _api.py:60-61)
 *           into the one read of w; the caller zeroes the word first and reads it afterwards.
 *   flags   TI_INCREASING | TI_EXACT | TI_CLIP_MIN | TI_CLIP_MAX, and the hints
 *           TI_STREAM_OUT and TI_REPAIR_CHAIN.
 *   workspace / workspace_bytes: at least ti_fwd_workspace() bytes, 256-byte aligned
 *           (may be NULL when that is 0).
 *   stream  hipStream_t.
 * Sums and hull predicates run in float64 whatever the dtype; float32 fits are rounded once.
 * TI_EXACT is accepted for API parity and changes nothing.
 */
int ti_fwd(const void* y, const void* w, void* out, uint32_t* starts, uint32_t* bad_weight,
           int64_t batch, int64_t n, int dtype, unsigned flags, double y_min, double y_max,
           void* workspace, size_t workspace_bytes, void* stream);

/*
 * ti_fwd, plus weights_read: a hipEvent_t (or NULL) that the call records on the stream as soon
 * as every weight has been read, i.e. once *bad_weight is final. Up to 2^24 elements a kernel of
 * its own reads w first, so the event comes before the fit; beyond, it comes after the first of
 * the fit's several kernels (rows longer than 32 elements), which reads w once for both. Either
 * way a caller that must refuse non-positive weights before it returns (the reference checks
 * them with a synchronous read of w before fitting, reference _api.py:60-61) waits on the event
 * and reads bad_weight while the rest of the fit still runs. No other counterpart in the
 * reference.
 */
int ti_fwd_ev(const void* y, const void* w, void* out, uint32_t* starts, uint32_t* bad_weight,
              int64_t batch, int64_t n, int dtype, unsigned flags, double y_min, double y_max,
              void* workspace, size_t workspace_bytes, void* stream, void* weights_read);

/*
 * ti_fwd without a workspace argument, for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops, harnesses that forbid hipMalloc). No counterpart in
 * the reference. The workspace is a file-scope device array of TI_NOALLOC_SCRATCH_BYTES (64 MiB)
 * that each GPU the library runs on holds until the process ends; the call allocates nothing
 * (no hipMalloc, hipFree or allocating library routine). Problem sets whose workspace
 * (ti_fwd_workspace) exceeds it fail with TI_EWORKSPACE before any launch. Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (other streams, other host threads)
 * race and must be ordered by the caller. A backward that needs the forward's workspace
 * (ti_bwd, rows over 32 elements) cannot use this one's, which the next call overwrites; ti_grad
 * takes the fit and the partition instead. Arguments and results otherwise as ti_fwd.
 */
#define TI_NOALLOC_SCRATCH_BYTES (64u << 20)
int ti_fwd_noalloc(const void* y, const void* w, void* out, uint32_t* starts, uint32_t* bad_weight,
                   int64_t batch, int64_t n, int dtype, unsigned flags, double y_min, double y_max,
                   void* stream);

/* Bytes of device workspace ti_bwd needs for this problem set (0 when none). */
int ti_bwd_workspace(int64_t batch, int64_t n, int dtype, int weighted, size_t* bytes);

/*
 * Gradients of a fit with respect to y and w, given the upstream gradient g and the fit's
 * block partition. Replaces torchisotonic::isotonic_grad (reference ops.cpp:50, implementation
 * grad.cuh:386-413) together with the clamp's backward (torch's, applied by autograd in the
 * reference, _api.py:69).
 *
 * With G, W and F the sum of g, the sum of w (the count when w is NULL) and the fit (unclamped,
 * rounded to dtype) over an element's block, and mask = [y_min <= F <= y_max] for the flags set
 * (torch.clamp's backward: equality passes, a NaN fit passes nothing):
 *   gy_i = w_i * mask * G / W,          gw_i = (y_i - F) * mask * G / W.
 * A row holding a NaN is one block with F = NaN (the reference CPU path's convention).
 *
 *   starts  the partition ti_fwd wrote for the same y, w.
 *   fwd_workspace / fwd_workspace_bytes: the workspace ti_fwd filled for the same call (none
 *           for rows of up to 32 elements, which recompute their blocks' means from y and w as
 *           the forward formed them). Rows longer than 32 elements take their blocks' weights
 *           and fits from the final hulls ti_fwd left there, so F and the mask are the
 *           forward's bit for bit; without it they fail with TI_EWORKSPACE (a caller holding
 *           only the fit and the partition calls ti_grad).
 *   g       [batch, n] upstream gradient.
 *   w       weights or NULL (unweighted).
 *   y       [batch, n] input of the fit; needed when gw is wanted or a TI_CLIP_* flag is set.
 *   gy, gw  outputs, either may be NULL.
 *   flags   the forward's TI_INCREASING and TI_CLIP_* bits.
 *   workspace / workspace_bytes: at least ti_bwd_workspace() bytes, 256-byte aligned.
 */
int ti_bwd(const uint32_t* starts, const void* fwd_workspace, size_t fwd_workspace_bytes,
           const void* g, const void* w, const void* y, void* gy, void* gw, int64_t batch,
           int64_t n, int dtype, unsigned flags, double y_min, double y_max, void* workspace,
           size_t workspace_bytes, void* stream);

/*
 * Keeping less than the forward's workspace for the backward. No counterpart in the reference,
 * whose autograd keeps the partition and calls the stateless gradient (reference
 * _api.py:73-97, grad.cuh:304-413). Here the backward of rows longer than 32 elements reads
 * only the final hulls and the per-tile records of the forward's workspace (ti_bwd), so a caller
 * that holds the workspace from forward to backward (an autograd node) keeps these instead:
 *
 *   1. ti_fwd_ev_hulls: the forward, reporting a bound on the final hulls' vertex counts;
 *   2. ti_keep_bytes, ti_keep: a buffer of that size, and the copy into it, after which the
 *      workspace is free for work the stream orders later;
 *   3. ti_bwd_kept_workspace, ti_bwd_kept: the backward from the kept buffer, with results
 *      identical to ti_bwd's from the workspace.
 *
 * The kept buffer holds each row's final hull in max_vertices slots (float32 data: 12 bytes a
 * slot, 20 weighted; float64: 20 and 36) and 32 bytes a tile of 4096 elements (2048 weighted):
 * about 1.6 MB for one weighted float32 row of 1e8 with a final hull of about a thousand
 * vertices, against 2.0 GB of workspace. A row whose hull has every element as a vertex
 * (monotone data) keeps as much as the workspace, and a caller may then keep the workspace
 * itself.
 */

/*
 * ti_fwd_ev, plus: for rows of more than 32 elements, a bound on the final hulls' vertex counts
 * (at least the largest over the rows, at most n + 1: the vertices a row has two merge levels
 * before the last) is written to *max_vertices (one int64 that the device writes: device memory,
 * or the device pointer of pinned host memory), and hulls_ready (a hipEvent_t, or NULL) is
 * recorded on the stream once it is written. The last merges and the expansion run after it, so
 * a caller waiting on the event sizes and allocates its kept buffer while the fit finishes. For
 * rows of at most 32 elements nothing is written and the event is recorded after the fit.
 */
int ti_fwd_ev_hulls(const void* y, const void* w, void* out, uint32_t* starts, uint32_t* bad_weight,
                    int64_t batch, int64_t n, int dtype, unsigned flags, double y_min, double y_max,
                    void* workspace, size_t workspace_bytes, void* stream, void* weights_read,
                    void* hulls_ready, int64_t* max_vertices);

/*
 * ti_fwd_ev_hulls with no event between the fit's kernels: a kernel of one thread writes
 * mark_value to *weights_mark (a device-visible word of host memory, or NULL) once every weight
 * has been read and *bad_weight is final, and *max_vertices (likewise host memory, or NULL; rows of
 * more than 32 elements only) is written once the bound is known, both with stores that reach host
 * memory directly. A caller that sets both words to values the call will not write polls them
 * instead of waiting on events: an event recorded between two kernels leaves the GPU idle for some
 * microseconds. No counterpart in the reference (its weight check is a synchronous read of w
 * before the fit, reference _api.py:60-61).
 */
int ti_fwd_marked(const void* y, const void* w, void* out, uint32_t* starts, uint32_t* bad_weight,
                  int64_t batch, int64_t n, int dtype, unsigned flags, double y_min, double y_max,
                  void* workspace, size_t workspace_bytes, void* stream, uint32_t* weights_mark,
                  uint32_t mark_value, int64_t* max_vertices);

/* Bytes of the kept buffer for final hulls of at most max_vertices vertices (0 for rows of at
 * most 32 elements, which keep nothing). */
int ti_keep_bytes(int64_t batch, int64_t n, int dtype, int weighted, int64_t max_vertices, size_t* bytes);

/*
 * Copies the final hulls and per-tile records out of the workspace that ti_fwd / ti_fwd_ev_hulls
 * filled (rows of more than 32 elements) into kept (at least ti_keep_bytes() bytes, 256-byte
 * aligned), on the stream. max_vertices: the value ti_fwd_ev_hulls wrote for that forward (one
 * below a row's final hull count cuts that hull short, and the backward's results are then
 * wrong).
 */
int ti_keep(const void* fwd_workspace, size_t fwd_workspace_bytes, void* kept, size_t kept_bytes,
            int64_t batch, int64_t n, int dtype, int weighted, int64_t max_vertices, void* stream);

/* Bytes of device workspace ti_bwd_kept needs (0 when none). */
int ti_bwd_kept_workspace(int64_t batch, int64_t n, int dtype, int weighted, int64_t max_vertices,
                          size_t* bytes);

/* ti_bwd, from the buffer ti_keep filled (kept, kept_bytes, and the forward's max_vertices) in
 * place of the forward's workspace; the other arguments and the results as ti_bwd's. */
int ti_bwd_kept(const uint32_t* starts, const void* kept, size_t kept_bytes, int64_t max_vertices,
                const void* g, const void* w, const void* y, void* gy, void* gw, int64_t batch,
                int64_t n, int dtype, unsigned flags, double y_min, double y_max, void* workspace,
                size_t workspace_bytes, void* stream);

/*
 * The fit of ragged rows, packed end to end: row r is y[offsets[r], offsets[r + 1]) (offsets:
 * nrows + 1 non-decreasing device int64 values). Rows of 1 to max_len elements (max_len <= 32)
 * are fitted in one launch (one thread per row, no padding pass); a longer row is not fitted
 * (its elements of out are not written) and gets its first start bit only, and an empty row
 * nothing, so the caller fits longer rows by other calls (ti_fwd on each). No counterpart in
 * the reference, whose callers pad ragged rows or lay them end to end (reference README.md:
 * 100-103, examples/ctr_calibration/README.md:25-27).
 *   starts  flat bits of the packed array: bit e (word e / 32, bit e % 32) set where a block
 *           starts, OR-ed into the caller's zeroed array of (offsets[nrows] + 31) / 32 words;
 *           or NULL. ti_grad over the packed array as one row (batch 1) takes these bits.
 *   other arguments as ti_fwd (flags, clamp, bad_weight for the fitted rows' weights).
 */
int ti_fwd_ragged(const void* y, const void* w, void* out, uint32_t* starts, uint32_t* bad_weight,
                  const int64_t* offsets, int64_t nrows, int64_t total, int64_t max_len, int dtype,
                  unsigned flags, double y_min, double y_max, void* stream);

/* The backward of ti_fwd_ragged's rows of at most max_len (<= 32) elements: gy = w * mask * G / W
 * and gw = (y - fit) * mask * G / W over each block of each row, the blocks read from the
 * forward's flat start bits (`starts`), the block's fit recomputed from y and w as the forward
 * formed it, and mask the forward's clamp (flags, y_min, y_max as given to ti_fwd_ragged): the
 * short-row backward's arithmetic (reference grad.cuh:200-290) for rows of their own lengths.
 * One thread per row, a workgroup's rows staged through LDS. Rows longer than max_len are not
 * written (their backward is ti_bwd or ti_grad over their own forward). gy or gw may be null
 * (not wanted); gw needs w and y, the clamp needs y. No reference counterpart: the reference has
 * no ragged rows. */
int ti_bwd_ragged(const uint32_t* starts, const void* g, const void* w, const void* y, void* gy, void* gw,
                  const int64_t* offsets, int64_t nrows, int64_t total, int64_t max_len, int dtype,
                  unsigned flags, double y_min, double y_max, void* stream);

/*
 * The plan of a ragged set, one pass over its offsets (device int64, nrows + 1 values), into
 * TI_RAGGED_PLAN_WORDS device words the caller has zeroed: plan[0] bit 0 set if offsets[0] != 0,
 * bit 1 if offsets[nrows] != total, bit 2 if a row has a negative length (offsets decrease);
 * plan[1] the longest row of at most 32 elements (the max_len ti_fwd_ragged takes), plan[2] the
 * number of longer rows, plan[3] the longest row; plan[4 + b] the number of rows of length
 * bucket b (lengths in (2^(b-1), 2^b], b >= 6) and plan[68 + b] the longest of them. keys
 * (device, one byte a row, or NULL): each row's bucket, 0 for a row of at most 32 elements; a
 * stable sort of them puts the longer rows in bucket order. The host reads the plan back to
 * validate the offsets and size the launches. No counterpart in the reference (see
 * ti_fwd_ragged).
 */
#define TI_RAGGED_PLAN_WORDS 132
int ti_ragged_plan(const int64_t* offsets, int64_t nrows, int64_t total, int64_t* plan, uint8_t* keys, void* stream);

/* The descriptors (first element, length) of rows order[0..n) of a ragged set, into rows (2 n
 * device int64), for ti_ragged_extreme / _pack / _unpack; order's entries are clamped into
 * [0, nrows). No counterpart in the reference (see ti_fwd_ragged). */
int ti_ragged_rows(const int64_t* offsets, int64_t nrows, const int64_t* order, int64_t n, int64_t* rows,
                   void* stream);

/*
 * Ragged rows longer than 32 elements, a length bucket at a time: the k rows described by `rows`
 * (device int64 pairs: first element in the packed array of `total` elements, length) as one
 * dense row-major [k, L] block (L at least every length), which ti_fwd and ti_bwd take as a
 * batch. No counterpart in the reference, whose callers pad ragged rows themselves with tail
 * values that never pool into the data (reference README.md:100-103); these apply that rule.
 * Every kernel clamps a row to the packed array and to L, so no access leaves the buffers.
 *
 * ti_ragged_extreme: each row's largest value (increasing != 0) or smallest (else), NaN skipped,
 *   as an order-preserving key into keys[r] (k device words the caller has zeroed), for the pad.
 * ti_ragged_pack: dst[r][j] = src[first_r + j] for j < len_r, else the row's pad: m + max(1, |m|)
 *   beyond its extreme m (with keys), or `pad` (keys NULL: 0 for a gradient's block; for float32
 *   values, the largest finite float32, negated for a decreasing fit, which needs no extreme);
 *   wdst likewise from w with weight 1 past the row (w and wdst both given or both NULL).
 * ti_ragged_unpack: dst[first_r + j] = src[r][j] for j < len_r (dst2 from src2 likewise, both
 *   given or both NULL). For a gradient block (gy, gw) give starts, the forward's packed starts of
 *   the block, and w, the packed weights (NULL: unweighted): a row whose last block reached into
 *   its pad (a NaN row, or one whose extreme is the dtype's largest finite value or infinite, which
 *   no pad exceeds) has that block's gradients scaled by (W + P) / W, W its own weight over the
 *   block and P the pad elements in it (up to the next start bit), so that the pad's weight
 *   leaves the block's mean gradient. starts NULL: no such scaling (a fit block).
 */
int ti_ragged_extreme(const void* y, int64_t total, const int64_t* rows, int64_t k, int64_t L, int dtype,
                      int increasing, uint64_t* keys, void* stream);
int ti_ragged_pack(const void* src, const void* w, int64_t total, const int64_t* rows, const uint64_t* keys,
                   double pad, int64_t k, int64_t L, int dtype, int increasing, void* dst, void* wdst, void* stream);
int ti_ragged_unpack(const void* src, const void* src2, const int64_t* rows, int64_t k, int64_t L, int dtype,
                     void* dst, void* dst2, int64_t total, const uint32_t* starts, const void* w, void* stream);

/*
 * ti_fwd and ti_bwd for the k rows of a length bucket read and written in place in the packed
 * arrays (`total` elements; rows as for ti_ragged_pack), without a block: row r is taken as the
 * r-th row of a [k, L] block (L > 32, at least every length) whose elements past the row's
 * length are `pad` with weight 1 (g = 0 in the backward), made in registers and never read;
 * y, w, out, g, gy and gw are the packed arrays, and only the rows' own elements are written.
 * starts, the workspaces and the flags are those of ti_fwd / ti_bwd for batch = k and n = L (the
 * starts in the block's layout). Float32 only (TI_EDTYPE otherwise: ti_ragged_pack serves
 * float64). The pad must lie beyond every value of its row, as for ti_ragged_pack: the largest
 * finite float32, negated for a decreasing fit.
 * ti_bwd_rows also applies ti_ragged_unpack's correction to rows whose pad joined their last
 * block. The packed arrays must stay below 0x7FFF0000 bytes (one buffer resource addresses
 * them; TI_ESIZE otherwise: ti_ragged_pack serves larger ones). No counterpart in the reference
 * (see ti_ragged_pack).
 */
int ti_fwd_rows(const void* y, const void* w, void* out, uint32_t* starts, uint32_t* bad_weight, const int64_t* rows,
                int64_t k, int64_t L, int64_t total, double pad, int dtype, unsigned flags, double y_min,
                double y_max, void* workspace, size_t workspace_bytes, void* stream);
int ti_bwd_rows(const uint32_t* starts, const void* fwd_workspace, size_t fwd_workspace_bytes, const void* g,
                const void* w, const void* y, void* gy, void* gw, const int64_t* rows, int64_t k, int64_t L,
                int64_t total, int dtype, unsigned flags, double y_min, double y_max, void* workspace,
                size_t workspace_bytes, void* stream);

/* Bytes of device workspace ti_grad needs for this problem set (0 when batch * n <= 2048). */
int ti_grad_workspace(int64_t batch, int64_t n, int dtype, size_t* bytes);

/*
 * The reference's stateless gradient operator, torchisotonic::isotonic_grad(out, starts, g, w, y)
 * (reference ops.cpp:50, implementation grad.cuh:304-413), for rows of any length: with G and W
 * the sums of g and of w (the element count when w is NULL) over an element's block,
 *   gy_i = w_i * G / W,          gw_i = (y_i - out_i) * G / W.
 * No clamp: in the reference the clamp's backward is torch's, outside this operator.
 *
 *   out     [batch, n] the fit (unclamped), read only when y is given.
 *   starts  the partition (ti_starts_words(batch, n) words, as ti_fwd writes it; element 0 of
 *           every row counts as a start whatever its bit).
 *   g       [batch, n] upstream gradient.
 *   w       weights or NULL.
 *   y       [batch, n] the data, or NULL: given (with w only, as in the reference), gw is
 *           written; else gw is not touched and may be NULL.
 *   gy, gw  outputs.
 *   workspace / workspace_bytes: at least ti_grad_workspace() bytes, 256-byte aligned.
 * Block sums are float64 within 8 elements and double-double beyond.
 */
int ti_grad(const void* out, const uint32_t* starts, const void* g, const void* w, const void* y,
            void* gy, void* gw, int64_t batch, int64_t n, int dtype, void* workspace,
            size_t workspace_bytes, void* stream);

/*
 * The calibration step after a fit: out[i] = the piecewise-linear interpolation at x[i] of the
 * m knots (xp, fp), xp sorted ascending, constant beyond the ends (np.interp's semantics). With
 * j the first knot at or above x[i] (searchsorted, left) clamped to [1, m - 1]:
 *   t = clamp((x - xp[j-1]) / max(xp[j] - xp[j-1], 1e-300), 0, 1),
 *   out = fp[j-1] + t * (fp[j] - fp[j-1]),
 * each operation rounded once, so equal to the reference's tensor formula bit for bit
 * (reference examples/ctr_calibration/calibrate.py:163-168, the predict step of its isotonic
 * calibration). One kernel; x, xp, fp, out of one dtype; NaN x gives NaN.
 */
int ti_interp(const void* x, const void* xp, const void* fp, void* out, int64_t n, int64_t m,
              int dtype, void* stream);

/* The knot index: ti_interp's output bit for bit with each query's search narrowed from all m
 * knots (~log2 m dependent reads, most of them misses) to one bucket of about four. Buckets of
 * equal width cover [xp[0], xp[m-1]] (B = ceil(m / 4)); first[b] is the first knot whose bucket
 * is b or later, so the first knot at or above x lies between first[b] and first[b+1] for x's
 * bucket b (bucket() is monotone). Knots whose ends are not finite, or all equal, give an index
 * under which every query searches all knots. Same semantics as ti_interp (reference
 * examples/ctr_calibration/calibrate.py:163-168); an index depends on xp only, so one built
 * after a fit serves every later call with those knots.
 *
 * ti_interp_index_bytes: the index's size for m knots (m < 2^32).
 * ti_interp_index: build it from xp (m knots, ascending) into `index` (256-byte aligned).
 * ti_interp_indexed: ti_interp through an index built from the same xp. An index built from
 *   another knot count or dtype is not used (every query searches all m knots, as ti_interp);
 *   one of other knots of the same count and dtype gives wrong values but reads nothing outside
 *   x, xp, fp and the index's index_bytes. */
int ti_interp_index_bytes(int64_t m, int dtype, size_t* bytes);
int ti_interp_index(const void* xp, int64_t m, int dtype, void* index, size_t index_bytes,
                    void* stream);
int ti_interp_indexed(const void* x, const void* xp, const void* fp, const void* index,
                      size_t index_bytes, void* out, int64_t n, int64_t m, int dtype, void* stream);

/* Test hook: the starts bit array of a [batch, n] set as bytes (0/1), row-major - the
 * reference's bool starts tensor (reference tests/test_cuda.py:176 reads it). */
int ti_starts_to_bool(const uint32_t* starts, uint8_t* out, int64_t batch, int64_t n,
                      void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TORCHISOTONIC_AMD_H */
