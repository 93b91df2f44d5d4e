// Host-visible kernel launchers of the flash_maxsim MI355X library. The C ABI
// in fmx_api.cpp validates arguments and picks a launcher; each launcher picks
// the template instance for the shape and enqueues it on the caller's stream.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fmx {

// One forward call: Nq queries of Lq tokens scored against docs of Ld tokens
// with d-wide embeddings. Strides are in elements of the operand's type.
struct FwdArgs {
  const void* Q;              // [Nq, Lq, d] fp16/bf16, row stride sq_l, query stride sq_n
  const void* D;              // [B' , Ld, d] fp16/bf16/uint8, strides sd_b, sd_l
  const int32_t* lengths;     // [B'] valid tokens per doc row, or null (= Ld)
  float* scores;              // [Nq, B] fp32, strides ss_n, ss_b
  int32_t* argmax;            // [Nq*B, Lq] int32, or null
  const uint16_t* scales;     // uint8 docs: fp16 bits [B', Ld], doc stride sm_b, token stride 1
  const uint16_t* mins;       // uint8 docs: fp16 bits, same layout as scales
  float* partial;             // workspace: per-pass partial sums [passes, Nq*B]
  const int32_t* qidx;        // sparse scoring: [B, Lq] rows of Q per doc, or null
  int64_t si_b, si_k;         // qidx strides
  int64_t sq_n, sq_l;
  int64_t sd_b, sd_l;
  int64_t ss_n, ss_b;
  int64_t sm_b;
  int Nq, B, Lq, Ld, d;
  int Lq_rows;                // rows of Q (= Lq unless qidx gathers from a longer Q)
  const int64_t* tok_group;   // packed docs: doc row r starts at token row 4*tok_group[r]
                              // (then sd_b and sm_b are unused), or null
  int64_t tok_rows;           // packed docs: token rows in D (reads are clamped to them)
  const int32_t* doc_ids;     // packed docs laid out in another order than numbered: the
                              // score column of doc row b is doc_ids[b] (ids outside [0, B)
                              // are not written), or null (= b)
  int shared_docs;            // doc row of (query qi, doc b) is b, else qi*B + b
  int vec;                    // uint8 docs, bit 0: 16-byte aligned code rows and scales/mins
                              // readable 4 tokens per 8-byte load; bit 1: 16-byte aligned
                              // code rows (compile-time paths)
};

// Backward of the forward with saved argmax (Nq queries, shared docs).
struct BwdArgs {
  const void* Q;              // [Nq, Lq, d], strides sq_n, sq_l
  const void* D;              // [B, Ld, d], strides sd_b, sd_l
  const int32_t* lengths;     // [B] or null: docs of length <= 0 get and give no gradient
  const int32_t* argmax;      // [Nq*B, Lq], row qi*B + b
  const float* grad;          // [Nq, B], strides g_n, g_b (either may be 0)
  void* dQ;                   // [Nq, Lq, d] contiguous, or null
  void* dD;                   // [B, Ld, d] contiguous, or null
  float* ws;                  // dQ partial sums [nchunk, Nq*Lq, d]
  int64_t sq_n, sq_l, sd_b, sd_l, g_n, g_b;
  int Nq, B, Lq, Ld, d;
  int nchunk;                 // doc chunks of the dQ gather
  int sort_n;                 // dD: entries of one index chunk padded to a power of two
  int dd_chunks;              // dD: index chunks of kDdChunk (query, token) entries per doc
  uint32_t* dd_rows;          // dD index [dd_chunks, B, Ld]: first sorted entry | count << 16, or ~0
  uint16_t* dd_ent;           // dD index [B, Nq*Lq]: each chunk's entries sorted by row (chunk-local)
  int dd_slab;                // rows per dD writer workgroup
};

// Shape class handled by the streaming kernel (query tile in VGPRs, docs read
// straight from HBM into VGPRs): d <= 256.
bool stream_fwd_supported(int d);
int stream_fwd_ks(int d);             // 32-wide k-steps held per fragment row
int stream_fwd_nqb(int Lq, int d);     // 16-token query blocks per pass (fp16/bf16 and uint8 docs)
int stream_fwd_passes(int Lq, int d);  // > 1: partial sums in FwdArgs::partial
hipError_t launch_stream_fwd(int kind, const FwdArgs& a, bool with_argmax, hipStream_t s);

// Split-d kernel: the eight waves of a workgroup each own a slice of d and
// reduce partial similarities through LDS before the max. 256 < d <= 4096.
bool splitd_fwd_supported(int d);
int splitd_fwd_ksw(int d);            // k-steps per wave
int splitd_fwd_nqb(int Lq, int d);    // 16-token query blocks per pass
int splitd_fwd_passes(int Lq, int d); // > 1: partial sums in FwdArgs::partial
hipError_t launch_splitd_fwd(int kind, const FwdArgs& a, bool with_argmax, hipStream_t s);

// Wide kernels, d > 4096: the similarities of a chunk of (query, doc) items go
// to a workspace S [items, Lq, Ld rounded up to 16] (fp32), then a reduction
// takes each query token's max (and argmax) and the sum. The workspace holds
// ws_bytes / wide_item_bytes(Lq, Ld) items per chunk (at least one).
constexpr int kSplitMaxD = 4096;
constexpr size_t kWideChunkBytes = (size_t)64 << 20;  // preferred S chunk
size_t wide_item_bytes(int64_t Lq, int64_t Ld);
size_t wide_fwd_workspace_bytes(int64_t items, int64_t Lq, int64_t Ld);
hipError_t launch_wide_fwd(int kind, const FwdArgs& a, bool with_argmax, float* ws, size_t ws_bytes, hipStream_t s);

// Tiled kernel (MFMA-bound regime): persistent 8- or 4-wave workgroups keep a
// block of query rows in VGPRs and stream shared docs through LDS. d <= 256.
// fp16/bf16 docs, and uint8 docs (dequantised to fp16 on their way to LDS;
// single queries, no argmax).
struct TiledPlan {
  int ks;              // 32-wide k-steps (4: d <= 128, 8: d <= 256)
  int nw;              // waves per workgroup (8, or 4 with three workgroups per CU)
  int nb;              // 16-row query blocks per wave
  int rows_per_block;  // nw * 16 * nb
  int nRB;             // row blocks over the Nq*Lq flattened query rows
  int G;               // doc groups (workgroups per row block)
  int xcd_map;         // XCD-aware blockIdx mapping (G % 8 == 0)
  int grid;            // workgroups launched
  int straddle;        // some query spans two row blocks: partial sums + second pass
};
bool tiled_fwd_applicable(int64_t Nq, int64_t Lq, int64_t Ld, int d);  // fmx_fwd's choice
bool tiled_fwd_possible(int64_t Nq, int64_t Lq, int d);                 // for some Ld (workspace bounds)
bool tiled_u8_applicable(int64_t Lq, int64_t Ld, int d);                 // fmx_fwd_int8's choice (single query)
TiledPlan tiled_fwd_plan(int64_t Nq, int64_t B, int64_t Lq, int d, int cus);
size_t tiled_fwd_workspace_bytes(const TiledPlan& p, int64_t Nq, int64_t B);
hipError_t launch_tiled_fwd(int kind, const FwdArgs& a, const TiledPlan& p, bool with_argmax, hipStream_t s);

// Per-token uint8 quantisation (the encoder of the uint8 doc format).
struct QuantArgs {
  const void* src;            // [B, Ld, d] fp16 / bf16 / fp32, strides s_stride_b, s_stride_l
  int64_t s_stride_b, s_stride_l;
  int64_t B, Ld, d;
  int esz;                    // bytes per source element
  const int32_t* lengths;     // [B] valid tokens per doc (packed output), or null (= Ld)
  const int64_t* tok_group;   // packed output: doc b starts at row 4*tok_group[b]; null = padded
  int64_t tok_rows;           // packed output: rows of codes/scales/mins (rows outside are skipped)
  uint8_t* codes;             // padded [B, Ld, d] (row b*Ld + j) or packed [T, d]; row stride c_stride_l
  int64_t c_stride_l;
  void* scales;               // fp16 bits: padded [B, Ld] (doc stride sm_stride_b) or packed [T]
  void* mins;
  int64_t sm_stride_b;
  int vec;                    // 16-byte source rows and 8-byte code rows: vector loads/stores
};
hipError_t launch_quantize(int src_kind, const QuantArgs& a, hipStream_t s);  // 0 f16, 1 bf16, 2 f32

// Top-k selection over score rows (descending, NaN first, ties to the smaller
// index).
struct TopkArgs {
  const float* scores;        // [Nq, B], row stride s_stride
  int64_t s_stride;
  int64_t Nq, B;
  int k;                      // 1 <= k <= min(B, 8192)
  float* values;              // [Nq, k], row stride o_stride
  int64_t* indices;           // [Nq, k], row stride o_stride
  int64_t o_stride;
  uint64_t* ws;               // topk_ws_keys(Nq, B, k, topk_chunk(k)) keys
};
int topk_chunk(int k);                                            // keys sorted per workgroup
int64_t topk_ws_keys(int64_t Nq, int64_t B, int64_t k, int64_t C);
hipError_t launch_topk(const TopkArgs& a, hipStream_t s);

// dQ / dD of the argmax backward.
constexpr int kDdChunk = 8192;                 // (query, token) entries per dD index chunk
int bwd_dq_chunks(int B, int rows, int d);     // rows = Nq * Lq query tokens
int bwd_sort_n(int64_t entries);               // power of two >= min(Nq * Lq, kDdChunk) (>= 64)
int64_t bwd_dd_chunks(int64_t entries);        // dD index chunks per doc
size_t bwd_dd_lds_bytes(int64_t entries);      // dynamic LDS of the dD index kernel
size_t bwd_dd_index_bytes(int64_t B, int64_t entries, int64_t Ld);  // its workspace
int bwd_dd_slab(int d);                         // rows per dD writer workgroup
hipError_t launch_bwd(int kind, const BwdArgs& a, hipStream_t s);

}  // namespace fmx
