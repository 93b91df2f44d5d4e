/*
 * fmx.h - C ABI of libflashmaxsim, the MI355X (gfx950) MaxSim scoring library.
 *
 * The reference (roipony/flash-maxsim 0.1.0) exposes this path only as a
 * Python API over Triton launches; each entry point below is the native
 * boundary under one of its Python functions, which keep their signatures,
 * asserts and casts in the flash_maxsim_amd package.
 *
 * Conventions (all entry points):
 *  - Every tensor pointer is a device pointer owned by the caller. The library
 *    allocates no device memory; scratch space is a caller-provided workspace
 *    whose size the matching *_workspace_bytes() function returns (0 means none
 *    needed). The backward creates one stream and two events per device on
 *    first use (see fmx_bwd_batched).
 *  - Strides are in elements of the tensor's type. The innermost (d) stride is
 *    1. Row strides of Q and D must be multiples of 8 elements, doc strides of
 *    D multiples of 8, and Q, D 16-byte aligned; d itself may be anything
 *    from 1 to FMX_MAX_D (elements past d in a row are never used).
 *  - `stream` is a hipStream_t (NULL = the default stream). Work is enqueued
 *    asynchronously; nothing synchronises the host.
 *  - Return value: FMX_OK, or a negative FMX_ERR_* code with a message
 *    available from fmx_last_error() on the calling thread.
 *  - Doc lengths are clamped to [0, Ld]; a doc with no valid token scores
 *    -inf (every similarity is masked), and its argmax entries are 0.
 */
#ifndef FMX_H_
#define FMX_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FMX_OK 0
#define FMX_ERR_INVALID (-1)      /* bad shape, stride, alignment or pointer */
#define FMX_ERR_UNSUPPORTED (-2)  /* valid but outside what the kernels cover */
#define FMX_ERR_WORKSPACE (-3)    /* workspace missing or too small */
#define FMX_ERR_HIP (-4)          /* a HIP runtime call failed */

#define FMX_DTYPE_F16 0
#define FMX_DTYPE_BF16 1
#define FMX_DTYPE_F32 2 /* fmx_quantize_int8 sources only */

/* Widest d. Up to 4096 the forward kernels hold each query slice in
 * registers; wider rows (which the reference reaches by padding d to a power
 * of two, flash_maxsim/flash_maxsim.py:8-9) compute similarities into the
 * workspace in chunks of docs and reduce them in a second kernel. */
#define FMX_MAX_D 65536
#define FMX_MAX_TOPK 8192
#define FMX_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20) /* per GPU, see fmx_fwd_noalloc */

/* Library version string ("0.1.0+mi355x"). */
const char* fmx_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* fmx_last_error(void);

/*
 * MaxSim forward: scores[qi, b] = sum_{q < Lq} max_{j < len} <Q[qi, q], D[row, j]>
 * with row = b if shared_docs else qi*B + b, and len = lengths[row] (Ld if
 * lengths is NULL). fp16/bf16 inputs, fp32 accumulation and output.
 *
 *   Q        [Nq, Lq, d]   dtype, strides (q_stride_n, q_stride_l, 1)
 *   D        [B', Ld, d]   dtype, strides (d_stride_b, d_stride_l, 1); B' = B or Nq*B
 *   lengths  [B']          int32, or NULL
 *   scores   [Nq, B]       fp32, strides (s_stride_n, s_stride_b)
 *   argmax   [Nq*B, Lq]    int32, or NULL; row qi*B + b holds, per query token,
 *                          the first doc token reaching the max
 *
 * Replaces flash_maxsim/flash_maxsim.py:195-208 (_launch_fwd) and the kernel
 * it launches, _maxsim_fwd_kernel (flash_maxsim.py:80-146); called by the
 * Python flash_maxsim (flash_maxsim.py:221-230), flash_maxsim_batched
 * (:233-250) and flash_maxsim_train's forward (:254-263).
 */
int fmx_fwd(int dtype, const void* Q, int64_t q_stride_n, int64_t q_stride_l, const void* D,
            int64_t d_stride_b, int64_t d_stride_l, const int32_t* lengths, float* scores,
            int64_t s_stride_n, int64_t s_stride_b, int32_t* argmax, int64_t Nq, int64_t B,
            int64_t Lq, int64_t Ld, int64_t d, int shared_docs, void* workspace,
            size_t workspace_bytes, void* stream);

size_t fmx_fwd_workspace_bytes(int64_t Nq, int64_t B, int64_t Lq, int64_t Ld, int64_t d);

/*
 * fmx_fwd for callers that cannot allocate: code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc. No counterpart in the
 * reference. Same arguments, results and errors as fmx_fwd without the
 * workspace: the partial sums fmx_fwd keeps in its workspace (queries that
 * take several passes, queries straddling row blocks) and, for d > 4096, its
 * chunks of similarities (as many (query, doc) items per chunk as fit, each
 * Lq x (Ld rounded up to 16) x 4 bytes) go to a static device array of
 * FMX_NOALLOC_SCRATCH_BYTES on each GPU, held until the process
 * ends. A call whose chosen kernels need more scratch than that fails with
 * FMX_ERR_UNSUPPORTED before any launch; fmx_fwd_workspace_bytes bounds that
 * need over every kernel route the sizes allow, so a call can succeed where
 * that bound exceeds the limit, never the other way round. The call
 * allocates nothing (no hipMalloc, no allocating library routine). The
 * first call on a GPU that needs scratch looks up that GPU's copy of the
 * array (hipGetSymbolAddress), so make that call outside stream capture;
 * later calls may be captured into a HIP graph and replayed. Every call on
 * one GPU shares that GPU's array: calls that overlap on one GPU (other
 * streams, other threads) race, and must be ordered by the caller. Nothing in
 * the array needs to start at zero.
 */
int fmx_fwd_noalloc(int dtype, const void* Q, int64_t q_stride_n, int64_t q_stride_l, const void* D,
                    int64_t d_stride_b, int64_t d_stride_l, const int32_t* lengths, float* scores,
                    int64_t s_stride_n, int64_t s_stride_b, int32_t* argmax, int64_t Nq, int64_t B,
                    int64_t Lq, int64_t Ld, int64_t d, int shared_docs, void* stream);

/*
 * Fused uint8-dequant MaxSim forward: doc token j of doc b is
 * code * scales[b, j] + mins[b, j] (per-token affine, fp16 scale and min).
 * Queries of more than 64 tokens at d <= 128, and of more than 64 tokens over
 * docs of up to 128 tokens at d <= 256, round each dequantised value to fp16
 * before the dot product, as the reference's kernel does
 * (flash_maxsim_quant.py:89); the others apply the affine map to the fp32
 * dot product. The two differ by under 1e-3 per score at a few hundred query
 * tokens.
 *
 *   Q        [Lq, d]   fp16, row stride q_stride_l
 *   D        [B, Ld, d] uint8 codes, strides (d_stride_b, d_stride_l, 1)
 *   scales   [B, Ld]   fp16, strides (sm_stride_b, 1), 2-byte aligned
 *   mins     [B, Ld]   fp16, strides (sm_stride_b, 1), 2-byte aligned
 *   lengths  [B]       int32, or NULL
 *   scores   [B]       fp32, contiguous
 *
 * Scale and min rows are read in aligned 4-byte words, so a read may touch
 * the 2 bytes before a doc's first value or after its last (the same word,
 * never another page); their contents do not matter.
 *
 * Replaces flash_maxsim/flash_maxsim_quant.py:135-141 (the launch in
 * flash_maxsim_int8) and _maxsim_int8_kernel (flash_maxsim_quant.py:40-98).
 */
int fmx_fwd_int8(const void* Q, int64_t q_stride_l, const uint8_t* D, int64_t d_stride_b,
                 int64_t d_stride_l, const void* scales, const void* mins, int64_t sm_stride_b,
                 const int32_t* lengths, float* scores, int64_t B, int64_t Lq, int64_t Ld, int64_t d,
                 void* workspace, size_t workspace_bytes, void* stream);

size_t fmx_fwd_int8_workspace_bytes(int64_t B, int64_t Lq, int64_t Ld, int64_t d);

/*
 * Sparse MaxSim forward: doc b is scored with its own K query tokens,
 * scores[b] = sum_{k < K} max_{j < len} <Q[indices[b, k]], D[b, j]>.
 * An index outside [0, Lq) selects a zero query token.
 *
 *   Q        [Lq, d]   dtype, row stride q_stride_l
 *   D        [B, Ld, d] dtype, strides (d_stride_b, d_stride_l, 1)
 *   indices  [B, K]    int32, strides (idx_stride_b, idx_stride_k)
 *   lengths  [B]       int32, or NULL
 *   scores   [B]       fp32, contiguous
 *
 * Replaces flash_maxsim/flash_maxsim_sparse.py:131-139 (the launch in
 * flash_maxsim_sparse) and _sparse_maxsim_kernel (flash_maxsim_sparse.py:28-91).
 */
int fmx_fwd_sparse(int dtype, const void* Q, int64_t q_stride_l, int64_t Lq, const void* D,
                   int64_t d_stride_b, int64_t d_stride_l, const int32_t* indices, int64_t idx_stride_b,
                   int64_t idx_stride_k, int64_t K, const int32_t* lengths, float* scores, int64_t B,
                   int64_t Ld, int64_t d, void* workspace, size_t workspace_bytes, void* stream);

size_t fmx_fwd_sparse_workspace_bytes(int64_t B, int64_t K, int64_t Ld, int64_t d);

/*
 * Per-token uint8 quantisation (the encoder of fmx_fwd_int8's doc format):
 * for every token row x (d values, widened to fp32)
 *   lo = min x, step = max((max x - lo) / 255, 1e-8),
 *   code = clamp(round_half_even((x - lo) / step), 0, 255),
 *   scale = fp16(step), min = fp16(lo)   (round to nearest even)
 * with IEEE fp32 operations in that order: bit-identical to the reference's
 * torch formula.
 *
 *   src      [B, Ld, d]  src_dtype (F16, BF16 or F32), strides (s_stride_b, s_stride_l, 1)
 * Padded output (tok_group NULL), the reference layout; lengths is ignored:
 *   codes    [B, Ld, d]  uint8, token (b, j) at row b*Ld + j, row stride c_stride_l
 *   scales   [B, Ld]     fp16, strides (sm_stride_b, 1); mins likewise
 * Packed output (tok_group non-NULL): doc b's first len_b = lengths[b] tokens
 * (clamped to [0, Ld]; NULL lengths = Ld) go to rows 4*tok_group[b] + j of
 *   codes    [T, d]      uint8, row stride c_stride_l
 *   scales   [T]         fp16; mins likewise (sm_stride_b unused)
 * and rows len_b .. 4*ceil(len_b/4)-1 of the doc's group are zeroed. The caller
 * lays groups out without overlap (e.g. tok_group = exclusive prefix sum of
 * ceil(len_b / 4)) and passes T = tok_rows; rows outside [0, T) are not written.
 *
 * Replaces flash_maxsim/flash_maxsim_quant.py:11-28 (quantize_int8, torch ops
 * there); the packed layout is an extension (no counterpart in the reference).
 */
int fmx_quantize_int8(int src_dtype, const void* src, int64_t s_stride_b, int64_t s_stride_l, int64_t B, int64_t Ld,
                      int64_t d, const int32_t* lengths, const int64_t* tok_group, int64_t tok_rows, uint8_t* codes,
                      int64_t c_stride_l, void* scales, void* mins, int64_t sm_stride_b, void* stream);

/*
 * Packed-doc forwards (no counterpart in the reference, whose docs are always
 * padded [B, Ld, d]): the T token rows of all docs are stored back to back,
 * doc b in rows 4*tok_group[b] .. 4*tok_group[b] + lengths[b] - 1, so padding
 * costs neither storage nor reads. tok_group and lengths (int32, clamped to
 * [0, Ld_max]) are required; reads are clamped to the T = tok_rows rows of D.
 * Scores equal fmx_fwd / fmx_fwd_int8 (Nq = 1) on the padded equivalent.
 *
 * doc_ids (int32 [B], may be NULL): the docs may be laid out in another order
 * than they are numbered. Entry b of tok_group and lengths then describes the
 * b-th doc in that order (its slot) and doc_ids[b] is the doc's number: its
 * score goes to scores[doc_ids[b]]. doc_ids must be a permutation of 0..B-1;
 * an entry outside [0, B) is skipped (that score is not written). NULL: slot b
 * is doc b. Laying docs out longest first and passing that order here scans
 * variable-length docs faster (concurrent workgroups then stream docs of
 * similar length side by side).
 *
 *   Q        [Lq, d]   dtype (fp16 for int8), row stride q_stride_l
 *   D/codes  [T, d]    dtype / uint8, row stride d_stride_l / c_stride_l
 *   scales   [T]       fp16 (int8 only); mins likewise
 *   scores   [B]       fp32, contiguous
 */
int fmx_fwd_packed(int dtype, const void* Q, int64_t q_stride_l, int64_t Lq, const void* D, int64_t d_stride_l,
                   int64_t tok_rows, const int64_t* tok_group, const int32_t* lengths, const int32_t* doc_ids,
                   float* scores, int64_t B, int64_t Ld_max, int64_t d, void* workspace, size_t workspace_bytes,
                   void* stream);

size_t fmx_fwd_packed_workspace_bytes(int64_t B, int64_t Lq, int64_t Ld_max, int64_t d);

int fmx_fwd_int8_packed(const void* Q, int64_t q_stride_l, int64_t Lq, const uint8_t* codes, int64_t c_stride_l,
                        const void* scales, const void* mins, int64_t tok_rows, const int64_t* tok_group,
                        const int32_t* lengths, const int32_t* doc_ids, float* scores, int64_t B, int64_t Ld_max,
                        int64_t d, void* workspace, size_t workspace_bytes, void* stream);

size_t fmx_fwd_int8_packed_workspace_bytes(int64_t B, int64_t Lq, int64_t Ld_max, int64_t d);

/*
 * Top-k of score rows: for each row r < Nq of scores [Nq, B] (row stride
 * s_stride_n), the k best (score, doc index) pairs, best first, into values
 * [Nq, k] (fp32) and indices [Nq, k] (int64), row stride o_stride_n. Order:
 * score descending, NaN before every number, equal scores by smaller index.
 * 1 <= k <= min(B, FMX_MAX_TOPK); B < 2^32; Nq <= 65535.
 *
 * The values and the ranking are those of torch.topk(scores, k) (sorted), with
 * ties resolved to the smaller index. No counterpart in the reference library:
 * its callers rank flash_maxsim's scores themselves (torch topk / argsort);
 * this is that step on the GPU, run after the scoring kernel on the same stream.
 */
int fmx_topk(const float* scores, int64_t s_stride_n, int64_t Nq, int64_t B, int64_t k, float* values,
             int64_t* indices, int64_t o_stride_n, void* workspace, size_t workspace_bytes, void* stream);

size_t fmx_topk_workspace_bytes(int64_t Nq, int64_t B, int64_t k);

/*
 * Single-query scoring and top-k in one call: scores[b] as fmx_fwd (Nq = 1,
 * shared docs, contiguous scores [B]), then values [k] / indices [k] as
 * fmx_topk over them, back to back on the stream. Workspace:
 * fmx_fwd_topk_workspace_bytes bytes, 256-byte aligned (or NULL when that is
 * 0).
 *
 * No counterpart in the reference: its callers rank flash_maxsim's scores
 * themselves (torch topk / argsort: benchmarks/bench.py:36,
 * examples/demo.py:127-128, tests/test_flash_maxsim.py:87-88).
 */
int fmx_fwd_topk(int dtype, const void* Q, int64_t q_stride_l, const void* D, int64_t d_stride_b,
                 int64_t d_stride_l, const int32_t* lengths, int64_t B, int64_t Lq, int64_t Ld, int64_t d,
                 int64_t k, float* scores, float* values, int64_t* indices, void* workspace,
                 size_t workspace_bytes, void* stream);

size_t fmx_fwd_topk_workspace_bytes(int64_t B, int64_t Lq, int64_t Ld, int64_t d, int64_t k);

/*
 * Argmax backward of the single-query forward (argmax from fmx_fwd, Nq = 1):
 *   dQ[q, :]    = sum_b grad[b] * D[b, argmax[b, q], :]
 *   dD[b, j, :] = grad[b] * sum_{q : argmax[b, q] = j} Q[q, :]
 * dQ ([Lq, d]) and dD ([B, Ld, d]) are written contiguous in `dtype`, each
 * skipped when NULL. dD is fully written (zeros where no token picked a row).
 * Streams as fmx_bwd_batched.
 *
 * Replaces flash_maxsim/flash_maxsim.py:265-286 (_FlashMaxSimFn.backward) and
 * its kernels _maxsim_bwd_dQ_kernel (:153-168) and _maxsim_bwd_dD_kernel
 * (:171-188).
 */
int fmx_bwd(int dtype, const void* Q, int64_t q_stride_l, const void* D, int64_t d_stride_b,
            int64_t d_stride_l, const int32_t* argmax, const float* grad_scores, void* dQ, void* dD,
            int64_t B, int64_t Lq, int64_t Ld, int64_t d, void* workspace, size_t workspace_bytes,
            void* stream);

/*
 * Workspace of fmx_bwd: the dD row index (B*Ld uint32 + B*Lq uint16, when dD
 * is written) followed by the dQ partial sums (fp32, when dQ is written). The
 * returned size covers both; a call writing only one of them may pass just
 * that part.
 */
size_t fmx_bwd_workspace_bytes(int64_t B, int64_t Lq, int64_t Ld, int64_t d);

/*
 * Argmax backward of the batched forward (argmax from fmx_fwd with Nq >= 1,
 * shared docs), with doc lengths:
 *   dQ[qi, q, :] = sum_b g[qi, b] * D[b, argmax[qi*B + b, q], :]
 *   dD[b, j, :]  = sum_{(qi, q) : argmax[qi*B + b, q] = j} g[qi, b] * Q[qi, q, :]
 * where g = grad_scores [Nq, B] with strides (g_stride_n, g_stride_b), either
 * of which may be 0 (an expanded gradient, such as that of scores.sum(), is
 * read in place). Docs with lengths[b] <= 0 (score -inf) take no part, as in
 * autograd through the masked naive MaxSim; lengths may be NULL (= Ld).
 * dQ [Nq, Lq, d] and dD [B, Ld, d] are written contiguous in `dtype`, each
 * skipped when NULL; dD rows no token picked are zeros, picked rows are the
 * fp32 sum in (qi, q) order (deterministic). dD needs Ld < 2^19 (any Nq*Lq).
 *
 * Streams: all work is ordered on `stream`. When both dQ and dD are asked for
 * and dD holds 2^24 bytes or more, the dQ kernels run on a second stream of
 * the library's (one per device, created on first use, default priority),
 * forked from and joined back to `stream` with events, so work enqueued on
 * `stream` after the call sees both outputs. Under stream capture everything
 * stays on `stream`. Calls from several host threads are safe; their dQ
 * kernels share the second stream.
 *
 * Generalises fmx_bwd (which is its Nq = 1, lengths = NULL case; reference
 * flash_maxsim/flash_maxsim.py:265-286) to the batched and variable-length
 * training the reference's flash_maxsim_train does not offer (:289-291).
 */
int fmx_bwd_batched(int dtype, const void* Q, int64_t q_stride_n, int64_t q_stride_l, const void* D,
                    int64_t d_stride_b, int64_t d_stride_l, const int32_t* lengths, const int32_t* argmax,
                    const float* grad_scores, int64_t g_stride_n, int64_t g_stride_b, void* dQ, void* dD,
                    int64_t Nq, int64_t B, int64_t Lq, int64_t Ld, int64_t d, void* workspace,
                    size_t workspace_bytes, void* stream);

/* Workspace of fmx_bwd_batched: as fmx_bwd_workspace_bytes with Nq*Lq entries per doc. */
size_t fmx_bwd_batched_workspace_bytes(int64_t Nq, int64_t B, int64_t Lq, int64_t Ld, int64_t d);

#ifdef __cplusplus
}
#endif

#endif /* FMX_H_ */
