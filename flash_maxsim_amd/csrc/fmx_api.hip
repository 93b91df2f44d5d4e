// C ABI of libflashmaxsim: argument validation, workspace sizing and kernel
// selection. Declarations and the contract live in include/fmx.h.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>
#include <string>

#include "../../include/fmx.h"
#include "fmx_device.h"
#include "fmx_kernels.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int ok() {
  g_err.clear();
  return FMX_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

constexpr int64_t kOffLimit = (int64_t)1 << 31;  // buffer offsets stay below 2^31

// Kernel family and pass count for a forward shape.
struct FwdPlan {
  bool wide;    // d > 4096: similarities through a workspace, then a reduction
  bool splitd;  // 256 < d <= 4096
  int passes;
};

FwdPlan plan_fwd(int64_t Lq, int64_t d) {
  FwdPlan p;
  p.wide = d > fmx::kSplitMaxD;
  p.splitd = !p.wide && d > 256;
  p.passes = p.wide ? 1 : p.splitd ? fmx::splitd_fwd_passes((int)Lq, (int)d) : fmx::stream_fwd_passes((int)Lq, (int)d);
  return p;
}

// Compute units of the current device (cached per device; 256 if unknown).
int device_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

// Whether fmx_fwd takes the tiled (MFMA-bound) kernel for this call.
bool use_tiled(int64_t Nq, int64_t Lq, int64_t Ld, int64_t d, int shared_docs) {
  return (shared_docs || Nq == 1) && fmx::tiled_fwd_applicable(Nq, Lq, Ld, (int)d);
}

// Streaming / split-d kernels: per-pass partial sums when the query needs
// several passes; wide kernels: a chunk of similarity rows.
size_t stream_ws_bytes(int64_t Nq, int64_t B, int64_t Lq, int64_t Ld, int64_t d) {
  if (Lq < 1 || d < 1 || d > FMX_MAX_D || Nq < 1 || B < 1) return 0;
  const FwdPlan p = plan_fwd(Lq, d);
  if (p.wide) return fmx::wide_fwd_workspace_bytes(Nq * B, Lq, Ld);
  return p.passes > 1 ? (size_t)p.passes * (size_t)Nq * (size_t)B * sizeof(float) : 0;
}

// Upper bound over the kernels fmx_fwd may pick for these sizes.
size_t fwd_ws_bytes(int64_t Nq, int64_t B, int64_t Lq, int64_t Ld, int64_t d) {
  size_t n = stream_ws_bytes(Nq, B, Lq, Ld, d);
  if (Nq >= 1 && B >= 1 && Lq >= 1 && fmx::tiled_fwd_possible(Nq, Lq, (int)d)) {
    const fmx::TiledPlan p = fmx::tiled_fwd_plan(Nq, B, Lq, (int)d, device_cus());
    const size_t t = fmx::tiled_fwd_workspace_bytes(p, Nq, B);
    if (t > n) n = t;
  }
  return n;
}

// Checks shared by the forward entry points. esz: bytes per D element.
int check_common(int64_t Nq, int64_t B, int64_t Lq, int64_t Ld, int64_t d, int64_t q_stride_l,
                 int64_t d_stride_b, int64_t d_stride_l, int esz) {
  if (Nq < 1 || B < 0 || Lq < 1 || Ld < 0 || d < 1)
    return fail(FMX_ERR_INVALID, "invalid sizes Nq=%lld B=%lld Lq=%lld Ld=%lld d=%lld", (long long)Nq,
                (long long)B, (long long)Lq, (long long)Ld, (long long)d);
  if (d > FMX_MAX_D) return fail(FMX_ERR_UNSUPPORTED, "d=%lld exceeds FMX_MAX_D=%d", (long long)d, FMX_MAX_D);
  if (q_stride_l < d || (q_stride_l & 7))
    return fail(FMX_ERR_INVALID, "Q row stride %lld must be >= d and a multiple of 8", (long long)q_stride_l);
  if (d_stride_l < d || (d_stride_l & 7))
    return fail(FMX_ERR_INVALID, "D row stride %lld must be >= d and a multiple of 8", (long long)d_stride_l);
  if (d_stride_b & 7) return fail(FMX_ERR_INVALID, "D doc stride %lld must be a multiple of 8", (long long)d_stride_b);
  if (Nq * B >= kOffLimit) return fail(FMX_ERR_UNSUPPORTED, "Nq*B=%lld too large", (long long)(Nq * B));
  if ((Lq + 128) * q_stride_l * 2 >= kOffLimit)
    return fail(FMX_ERR_UNSUPPORTED, "query of %lld x %lld elements exceeds 2 GiB", (long long)Lq,
                (long long)q_stride_l);
  if ((Ld + 16) * d_stride_l * esz >= kOffLimit)
    return fail(FMX_ERR_UNSUPPORTED, "doc of %lld x %lld elements exceeds 2 GiB", (long long)Ld,
                (long long)d_stride_l);
  return FMX_OK;
}

int hip_status(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(FMX_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

}  // namespace

// Scratch of fmx_fwd_noalloc: a static device array, one copy per GPU, held
// until the process ends. Its name is a host-side stand-in, never a device
// address: host code uses only the per-device address hipGetSymbolAddress
// returns (scratch_address).
static __device__ __align__(256) unsigned char scratch[FMX_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch`, looked up on the first call on
// that device (with it current) and kept.
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(FMX_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(FMX_ERR_UNSUPPORTED, "device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(FMX_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return FMX_OK;
}

}  // namespace

extern "C" {

const char* fmx_version(void) { return "0.1.0+mi355x"; }

const char* fmx_last_error(void) { return g_err.c_str(); }

size_t fmx_fwd_workspace_bytes(int64_t Nq, int64_t B, int64_t Lq, int64_t Ld, int64_t d) {
  return fwd_ws_bytes(Nq, B, Lq, Ld, d);
}

size_t fmx_fwd_int8_workspace_bytes(int64_t B, int64_t Lq, int64_t Ld, int64_t d) {
  return fwd_ws_bytes(1, B, Lq, Ld, d);  // every kernel family takes uint8 docs
}

}  // extern "C"

namespace {

// fmx_fwd and fmx_fwd_packed: tok_group non-null selects packed docs.
int fwd_impl(int dtype, const void* Q, int64_t q_stride_n, int64_t q_stride_l, const void* D, int64_t d_stride_b,
             int64_t d_stride_l, const int64_t* tok_group, int64_t tok_rows, const int32_t* lengths, float* scores,
             int64_t s_stride_n, int64_t s_stride_b, int32_t* argmax, int64_t Nq, int64_t B, int64_t Lq, int64_t Ld,
             int64_t d, int shared_docs, void* workspace, size_t workspace_bytes, void* stream,
             bool noalloc = false, const int32_t* doc_ids = nullptr) {
  if (dtype != FMX_DTYPE_F16 && dtype != FMX_DTYPE_BF16) return fail(FMX_ERR_INVALID, "unknown dtype %d", dtype);
  int rc = check_common(Nq, B, Lq, Ld, d, q_stride_l, d_stride_b, d_stride_l, 2);
  if (rc) return rc;
  if (B == 0) return ok();
  if (!Q || !D || !scores) return fail(FMX_ERR_INVALID, "Q, D and scores must be non-null");
  if (!aligned16(Q) || !aligned16(D)) return fail(FMX_ERR_INVALID, "Q and D must be 16-byte aligned");
  if (Nq > 1 && (q_stride_n & 7)) return fail(FMX_ERR_INVALID, "Q query stride must be a multiple of 8");
  const bool tiled = use_tiled(Nq, Lq, Ld, d, shared_docs);
  fmx::TiledPlan tp = {};
  size_t need;
  if (tiled) {
    tp = fmx::tiled_fwd_plan(Nq, B, Lq, (int)d, device_cus());
    need = fmx::tiled_fwd_workspace_bytes(tp, Nq, B);
  } else {
    need = stream_ws_bytes(Nq, B, Lq, Ld, d);
  }
  const bool wide = plan_fwd(Lq, d).wide;
  if (noalloc) {
    // the static scratch array stands in for the workspace; the wide kernels
    // take as many items per chunk as it holds
    if (wide && need > 0) need = fmx::wide_item_bytes(Lq, Ld);
    if (need > FMX_NOALLOC_SCRATCH_BYTES)
      return fail(FMX_ERR_UNSUPPORTED, "scratch of %zu bytes required, FMX_NOALLOC_SCRATCH_BYTES is %zu", need,
                  (size_t)FMX_NOALLOC_SCRATCH_BYTES);
    workspace = nullptr;
    workspace_bytes = 0;
    if (need > 0) {
      rc = scratch_address(&workspace);
      if (rc) return rc;
      workspace_bytes = FMX_NOALLOC_SCRATCH_BYTES;
    }
  }
  if (need > 0 && (!workspace || workspace_bytes < need))
    return fail(FMX_ERR_WORKSPACE, "workspace of %zu bytes required, %zu given", need, workspace_bytes);

  fmx::FwdArgs a = {};
  a.Q = Q;
  a.D = D;
  a.lengths = lengths;
  a.scores = scores;
  a.argmax = argmax;
  a.partial = static_cast<float*>(workspace);
  a.tok_group = tok_group;
  a.tok_rows = tok_rows;
  a.doc_ids = doc_ids;
  a.sq_n = Nq > 1 ? q_stride_n : 0;
  a.sq_l = q_stride_l;
  a.sd_b = d_stride_b;
  a.sd_l = d_stride_l;
  a.ss_n = s_stride_n;
  a.ss_b = s_stride_b;
  a.Nq = (int)Nq;
  a.B = (int)B;
  a.Lq = (int)Lq;
  a.Lq_rows = (int)Lq;
  a.Ld = (int)Ld;
  a.d = (int)d;
  a.shared_docs = shared_docs ? 1 : 0;
  const int kind = dtype == FMX_DTYPE_BF16 ? fmx::KIND_BF16 : fmx::KIND_F16;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (tiled) {
    e = fmx::launch_tiled_fwd(kind, a, tp, argmax != nullptr, s);
  } else if (wide) {
    e = fmx::launch_wide_fwd(kind, a, argmax != nullptr, static_cast<float*>(workspace), workspace_bytes, s);
  } else if (plan_fwd(Lq, d).splitd) {
    e = fmx::launch_splitd_fwd(kind, a, argmax != nullptr, s);
  } else {
    e = fmx::launch_stream_fwd(kind, a, argmax != nullptr, s);
  }
  return hip_status(e, "fmx_fwd launch");
}

// fmx_fwd_int8 and fmx_fwd_int8_packed: tok_group non-null selects packed docs.
int int8_impl(const void* Q, int64_t q_stride_l, const uint8_t* D, int64_t d_stride_b, int64_t d_stride_l,
              const void* scales, const void* mins, int64_t sm_stride_b, const int64_t* tok_group, int64_t tok_rows,
              const int32_t* lengths, float* scores, int64_t B, int64_t Lq, int64_t Ld, int64_t d, void* workspace,
              size_t workspace_bytes, void* stream, const int32_t* doc_ids = nullptr) {
  int rc = check_common(1, B, Lq, Ld, d, q_stride_l, d_stride_b, d_stride_l, 1);
  if (rc) return rc;
  if (B == 0) return ok();
  if (!Q || !D || !scores || !scales || !mins)
    return fail(FMX_ERR_INVALID, "Q, D, scales, mins and scores must be non-null");
  if (!aligned16(Q) || !aligned16(D)) return fail(FMX_ERR_INVALID, "Q and D must be 16-byte aligned");
  if ((reinterpret_cast<uintptr_t>(scales) | reinterpret_cast<uintptr_t>(mins)) & 1u)
    return fail(FMX_ERR_INVALID, "scales and mins must be 2-byte aligned");
  if (!tok_group && sm_stride_b < Ld)
    return fail(FMX_ERR_INVALID, "scale doc stride %lld < Ld", (long long)sm_stride_b);
  const bool tiled = d <= 256 && fmx::tiled_u8_applicable(Lq, Ld, (int)d);
  fmx::TiledPlan tp = {};
  size_t need;
  if (tiled) {
    tp = fmx::tiled_fwd_plan(1, B, Lq, (int)d, device_cus());
    need = fmx::tiled_fwd_workspace_bytes(tp, 1, B);
  } else {
    need = stream_ws_bytes(1, B, Lq, Ld, d);
  }
  if (need > 0 && (!workspace || workspace_bytes < need))
    return fail(FMX_ERR_WORKSPACE, "workspace of %zu bytes required, %zu given", need, workspace_bytes);

  fmx::FwdArgs a = {};
  a.Q = Q;
  a.D = D;
  a.lengths = lengths;
  a.scores = scores;
  a.argmax = nullptr;
  a.scales = static_cast<const uint16_t*>(scales);
  a.mins = static_cast<const uint16_t*>(mins);
  a.partial = static_cast<float*>(workspace);
  a.tok_group = tok_group;
  a.tok_rows = tok_rows;
  a.doc_ids = doc_ids;
  a.sq_n = 0;
  a.sq_l = q_stride_l;
  a.sd_b = d_stride_b;
  a.sd_l = d_stride_l;
  a.ss_n = 0;
  a.ss_b = 1;
  a.sm_b = sm_stride_b;
  a.Nq = 1;
  a.B = (int)B;
  a.Lq = (int)Lq;
  a.Lq_rows = (int)Lq;
  a.Ld = (int)Ld;
  a.d = (int)d;
  a.shared_docs = 1;
  // The vector path reads codes 16 bytes at a time (16-byte aligned rows) and
  // four scales per 8-byte load, which needs 8-byte aligned scale rows and a
  // padded length that never passes the end of a doc's scales: Ld % 4 == 0 for
  // padded docs; packed docs start on 4-token groups, whose rows are the doc's.
  const bool sm8 = ((reinterpret_cast<uintptr_t>(scales) | reinterpret_cast<uintptr_t>(mins)) & 7u) == 0;
  const bool rows16 = (d_stride_l & 15) == 0 && (tok_group || (d_stride_b & 15) == 0);
  a.vec = (rows16 && sm8 && (tok_group || ((sm_stride_b & 3) == 0 && (Ld & 3) == 0))) ? 1 : 0;
  if (rows16 && aligned16(D)) a.vec |= 2;  // without bit 0: 16-byte code loads, per-tile scale loads
  hipStream_t s = static_cast<hipStream_t>(stream);
  const FwdPlan p = plan_fwd(Lq, d);
  const hipError_t e = tiled    ? fmx::launch_tiled_fwd(fmx::KIND_U8, a, tp, false, s)
                       : p.wide ? fmx::launch_wide_fwd(fmx::KIND_U8, a, false, static_cast<float*>(workspace),
                                                       workspace_bytes, s)
                       : p.splitd ? fmx::launch_splitd_fwd(fmx::KIND_U8, a, false, s)
                                  : fmx::launch_stream_fwd(fmx::KIND_U8, a, false, s);
  return hip_status(e, "fmx_fwd_int8 launch");
}

int check_packed(const int64_t* tok_group, const int32_t* lengths, int64_t tok_rows) {
  if (!tok_group || !lengths) return fail(FMX_ERR_INVALID, "packed docs need tok_group and lengths");
  if (tok_rows < 0) return fail(FMX_ERR_INVALID, "tok_rows=%lld must be >= 0", (long long)tok_rows);
  return FMX_OK;
}

}  // namespace

extern "C" {

int fmx_fwd(int dtype, const void* Q, int64_t q_stride_n, int64_t q_stride_l, const void* D,
            int64_t d_stride_b, int64_t d_stride_l, const int32_t* lengths, float* scores,
            int64_t s_stride_n, int64_t s_stride_b, int32_t* argmax, int64_t Nq, int64_t B,
            int64_t Lq, int64_t Ld, int64_t d, int shared_docs, void* workspace,
            size_t workspace_bytes, void* stream) {
  return fwd_impl(dtype, Q, q_stride_n, q_stride_l, D, d_stride_b, d_stride_l, nullptr, 0, lengths, scores,
                  s_stride_n, s_stride_b, argmax, Nq, B, Lq, Ld, d, shared_docs, workspace, workspace_bytes, stream);
}

int fmx_fwd_int8(const void* Q, int64_t q_stride_l, const uint8_t* D, int64_t d_stride_b,
                 int64_t d_stride_l, const void* scales, const void* mins, int64_t sm_stride_b,
                 const int32_t* lengths, float* scores, int64_t B, int64_t Lq, int64_t Ld, int64_t d,
                 void* workspace, size_t workspace_bytes, void* stream) {
  return int8_impl(Q, q_stride_l, D, d_stride_b, d_stride_l, scales, mins, sm_stride_b, nullptr, 0, lengths, scores,
                   B, Lq, Ld, d, workspace, workspace_bytes, stream);
}

int fmx_fwd_noalloc(int dtype, const void* Q, int64_t q_stride_n, int64_t q_stride_l, const void* D,
                    int64_t d_stride_b, int64_t d_stride_l, const int32_t* lengths, float* scores,
                    int64_t s_stride_n, int64_t s_stride_b, int32_t* argmax, int64_t Nq, int64_t B,
                    int64_t Lq, int64_t Ld, int64_t d, int shared_docs, void* stream) {
  return fwd_impl(dtype, Q, q_stride_n, q_stride_l, D, d_stride_b, d_stride_l, nullptr, 0, lengths, scores,
                  s_stride_n, s_stride_b, argmax, Nq, B, Lq, Ld, d, shared_docs, nullptr, 0, stream, true);
}

}  // extern "C"

namespace {

// fmx_fwd_topk's workspace: fmx_fwd's, then fmx_topk's (256-byte aligned).
size_t topk_fwd_part(int64_t B, int64_t Lq, int64_t Ld, int64_t d) {
  return (fwd_ws_bytes(1, B, Lq, Ld, d) + 255) & ~(size_t)255;
}

}  // namespace

extern "C" {

size_t fmx_fwd_topk_workspace_bytes(int64_t B, int64_t Lq, int64_t Ld, int64_t d, int64_t k) {
  // the scoring part is needed for any k (k = 0 still scores the docs)
  if (B < 1 || Lq < 1 || d < 1 || d > FMX_MAX_D || k < 0) return 0;
  return topk_fwd_part(B, Lq, Ld, d) + fmx_topk_workspace_bytes(1, B, k);
}

int fmx_fwd_topk(int dtype, const void* Q, int64_t q_stride_l, const void* D, int64_t d_stride_b,
                 int64_t d_stride_l, const int32_t* lengths, int64_t B, int64_t Lq, int64_t Ld, int64_t d,
                 int64_t k, float* scores, float* values, int64_t* indices, void* workspace,
                 size_t workspace_bytes, void* stream) {
  if (k < 0 || B < 0) return fail(FMX_ERR_INVALID, "invalid sizes B=%lld k=%lld", (long long)B, (long long)k);
  if (k > B) return fail(FMX_ERR_INVALID, "k=%lld exceeds the %lld scores", (long long)k, (long long)B);
  if (k > FMX_MAX_TOPK) return fail(FMX_ERR_UNSUPPORTED, "k=%lld exceeds FMX_MAX_TOPK=%d", (long long)k, FMX_MAX_TOPK);
  int rc = check_common(1, B, Lq, Ld, d, q_stride_l, d_stride_b, d_stride_l, 2);
  if (rc) return rc;
  if (k > 0 && (!values || !indices)) return fail(FMX_ERR_INVALID, "values and indices must be non-null");
  const size_t need = fmx_fwd_topk_workspace_bytes(B, Lq, Ld, d, k);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return fail(FMX_ERR_WORKSPACE, "workspace of %zu bytes required, %zu given", need, workspace_bytes);
  if (reinterpret_cast<uintptr_t>(workspace) & 255u) return fail(FMX_ERR_INVALID, "workspace must be 256-byte aligned");
  char* w = static_cast<char*>(workspace);
  const size_t fws = B > 0 ? topk_fwd_part(B, Lq, Ld, d) : 0;
  rc = fmx_fwd(dtype, Q, 0, q_stride_l, D, d_stride_b, d_stride_l, lengths, scores, 0, 1, nullptr, 1, B, Lq, Ld, d, 1,
               fws ? w : nullptr, fws, stream);
  if (rc || B == 0 || k == 0) return rc;
  const size_t tws = fmx_topk_workspace_bytes(1, B, k);
  return fmx_topk(scores, B, 1, B, k, values, indices, k, tws ? w + fws : nullptr, tws, stream);
}

size_t fmx_fwd_packed_workspace_bytes(int64_t B, int64_t Lq, int64_t Ld_max, int64_t d) {
  return fwd_ws_bytes(1, B, Lq, Ld_max, d);
}

int fmx_fwd_packed(int dtype, const void* Q, int64_t q_stride_l, int64_t Lq, const void* D, int64_t d_stride_l,
                   int64_t tok_rows, const int64_t* tok_group, const int32_t* lengths, const int32_t* doc_ids,
                   float* scores, int64_t B, int64_t Ld_max, int64_t d, void* workspace, size_t workspace_bytes,
                   void* stream) {
  if (B > 0) {
    const int rc = check_packed(tok_group, lengths, tok_rows);
    if (rc) return rc;
  }
  return fwd_impl(dtype, Q, 0, q_stride_l, D, 0, d_stride_l, tok_group, tok_rows, lengths, scores, 0, 1, nullptr,
                  1, B, Lq, Ld_max, d, 1, workspace, workspace_bytes, stream, false, doc_ids);
}

size_t fmx_fwd_int8_packed_workspace_bytes(int64_t B, int64_t Lq, int64_t Ld_max, int64_t d) {
  return fwd_ws_bytes(1, B, Lq, Ld_max, d);
}

int fmx_fwd_int8_packed(const void* Q, int64_t q_stride_l, int64_t Lq, const uint8_t* codes, int64_t c_stride_l,
                        const void* scales, const void* mins, int64_t tok_rows, const int64_t* tok_group,
                        const int32_t* lengths, const int32_t* doc_ids, float* scores, int64_t B, int64_t Ld_max,
                        int64_t d, void* workspace, size_t workspace_bytes, void* stream) {
  if (B > 0) {
    const int rc = check_packed(tok_group, lengths, tok_rows);
    if (rc) return rc;
  }
  return int8_impl(Q, q_stride_l, codes, 0, c_stride_l, scales, mins, 0, tok_group, tok_rows, lengths, scores, B,
                   Lq, Ld_max, d, workspace, workspace_bytes, stream, doc_ids);
}

int fmx_quantize_int8(int src_dtype, const void* src, int64_t s_stride_b, int64_t s_stride_l, int64_t B, int64_t Ld,
                      int64_t d, const int32_t* lengths, const int64_t* tok_group, int64_t tok_rows, uint8_t* codes,
                      int64_t c_stride_l, void* scales, void* mins, int64_t sm_stride_b, void* stream) {
  int esz;
  switch (src_dtype) {
    case FMX_DTYPE_F16: esz = 2; break;
    case FMX_DTYPE_BF16: esz = 2; break;
    case FMX_DTYPE_F32: esz = 4; break;
    default: return fail(FMX_ERR_INVALID, "unknown source dtype %d", src_dtype);
  }
  if (B < 0 || Ld < 0 || d < 1 || d > FMX_MAX_D)
    return fail(FMX_ERR_INVALID, "invalid sizes B=%lld Ld=%lld d=%lld", (long long)B, (long long)Ld, (long long)d);
  if (s_stride_l < d || c_stride_l < d || s_stride_b < 0)
    return fail(FMX_ERR_INVALID, "row strides must be >= d");
  if (!tok_group && (sm_stride_b < Ld)) return fail(FMX_ERR_INVALID, "scale doc stride < Ld");
  if (tok_group && tok_rows < 0) return fail(FMX_ERR_INVALID, "tok_rows=%lld must be >= 0", (long long)tok_rows);
  if (B == 0 || Ld == 0) return ok();
  if (!src || !codes || !scales || !mins) return fail(FMX_ERR_INVALID, "src, codes, scales and mins must be non-null");
  if ((reinterpret_cast<uintptr_t>(scales) | reinterpret_cast<uintptr_t>(mins)) & 1u)
    return fail(FMX_ERR_INVALID, "scales and mins must be 2-byte aligned");
  if (reinterpret_cast<uintptr_t>(src) % esz) return fail(FMX_ERR_INVALID, "src must be aligned to its element");
  fmx::QuantArgs a = {};
  a.src = src;
  a.s_stride_b = s_stride_b;
  a.s_stride_l = s_stride_l;
  a.B = B;
  a.Ld = Ld;
  a.d = d;
  a.esz = esz;
  a.lengths = lengths;
  a.tok_group = tok_group;
  a.tok_rows = tok_rows;
  a.codes = codes;
  a.c_stride_l = c_stride_l;
  a.scales = scales;
  a.mins = mins;
  a.sm_stride_b = sm_stride_b;
  a.vec = (aligned16(src) && ((s_stride_b * esz) & 15) == 0 && ((s_stride_l * esz) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(codes) & 7u) == 0 && (c_stride_l & 7) == 0)
              ? 1
              : 0;
  const int kind = src_dtype == FMX_DTYPE_F32 ? 2 : (src_dtype == FMX_DTYPE_BF16 ? 1 : 0);
  return hip_status(fmx::launch_quantize(kind, a, static_cast<hipStream_t>(stream)), "fmx_quantize_int8 launch");
}

size_t fmx_topk_workspace_bytes(int64_t Nq, int64_t B, int64_t k) {
  if (Nq < 1 || B < 1 || k < 1 || k > FMX_MAX_TOPK) return 0;
  return (size_t)fmx::topk_ws_keys(Nq, B, k, fmx::topk_chunk((int)k)) * sizeof(uint64_t);
}

int fmx_topk(const float* scores, int64_t s_stride_n, int64_t Nq, int64_t B, int64_t k, float* values,
             int64_t* indices, int64_t o_stride_n, void* workspace, size_t workspace_bytes, void* stream) {
  if (Nq < 0 || B < 0 || k < 0) return fail(FMX_ERR_INVALID, "invalid sizes Nq=%lld B=%lld k=%lld", (long long)Nq,
                                            (long long)B, (long long)k);
  if (k > B) return fail(FMX_ERR_INVALID, "k=%lld exceeds the %lld scores per row", (long long)k, (long long)B);
  if (k > FMX_MAX_TOPK) return fail(FMX_ERR_UNSUPPORTED, "k=%lld exceeds FMX_MAX_TOPK=%d", (long long)k, FMX_MAX_TOPK);
  if (B >= ((int64_t)1 << 32)) return fail(FMX_ERR_UNSUPPORTED, "B=%lld too large", (long long)B);
  if (Nq > 65535) return fail(FMX_ERR_UNSUPPORTED, "Nq=%lld exceeds 65535 rows", (long long)Nq);
  if (Nq == 0 || k == 0) return ok();
  if (!scores || !values || !indices) return fail(FMX_ERR_INVALID, "scores, values and indices must be non-null");
  if (s_stride_n < B && Nq > 1) return fail(FMX_ERR_INVALID, "score row stride %lld < B", (long long)s_stride_n);
  if (o_stride_n < k && Nq > 1) return fail(FMX_ERR_INVALID, "output row stride %lld < k", (long long)o_stride_n);
  const size_t need = fmx_topk_workspace_bytes(Nq, B, k);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return fail(FMX_ERR_WORKSPACE, "workspace of %zu bytes required, %zu given", need, workspace_bytes);
  if (reinterpret_cast<uintptr_t>(workspace) & 7u) return fail(FMX_ERR_INVALID, "workspace must be 8-byte aligned");
  fmx::TopkArgs a = {};
  a.scores = scores;
  a.s_stride = s_stride_n;
  a.Nq = Nq;
  a.B = B;
  a.k = (int)k;
  a.values = values;
  a.indices = indices;
  a.o_stride = o_stride_n;
  a.ws = static_cast<uint64_t*>(workspace);
  return hip_status(fmx::launch_topk(a, static_cast<hipStream_t>(stream)), "fmx_topk launch");
}

size_t fmx_fwd_sparse_workspace_bytes(int64_t B, int64_t K, int64_t Ld, int64_t d) {
  return stream_ws_bytes(1, B, K, Ld, d);
}

int fmx_fwd_sparse(int dtype, const void* Q, int64_t q_stride_l, int64_t Lq, const void* D,
                   int64_t d_stride_b, int64_t d_stride_l, const int32_t* indices, int64_t idx_stride_b,
                   int64_t idx_stride_k, int64_t K, const int32_t* lengths, float* scores, int64_t B,
                   int64_t Ld, int64_t d, void* workspace, size_t workspace_bytes, void* stream) {
  if (dtype != FMX_DTYPE_F16 && dtype != FMX_DTYPE_BF16) return fail(FMX_ERR_INVALID, "unknown dtype %d", dtype);
  if (Lq < 1) return fail(FMX_ERR_INVALID, "Lq=%lld must be >= 1", (long long)Lq);
  int rc = check_common(1, B, K > Lq ? K : Lq, Ld, d, q_stride_l, d_stride_b, d_stride_l, 2);
  if (rc) return rc;
  if (K < 1) return fail(FMX_ERR_INVALID, "K=%lld must be >= 1", (long long)K);
  if (B == 0) return ok();
  if (!Q || !D || !scores || !indices) return fail(FMX_ERR_INVALID, "Q, D, indices and scores must be non-null");
  if (!aligned16(Q) || !aligned16(D)) return fail(FMX_ERR_INVALID, "Q and D must be 16-byte aligned");
  const size_t need = stream_ws_bytes(1, B, K, Ld, d);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return fail(FMX_ERR_WORKSPACE, "workspace of %zu bytes required, %zu given", need, workspace_bytes);

  fmx::FwdArgs a = {};
  a.Q = Q;
  a.D = D;
  a.lengths = lengths;
  a.scores = scores;
  a.argmax = nullptr;
  a.partial = static_cast<float*>(workspace);
  a.qidx = indices;
  a.si_b = idx_stride_b;
  a.si_k = idx_stride_k;
  a.sq_n = 0;
  a.sq_l = q_stride_l;
  a.sd_b = d_stride_b;
  a.sd_l = d_stride_l;
  a.ss_n = 0;
  a.ss_b = 1;
  a.Nq = 1;
  a.B = (int)B;
  a.Lq = (int)K;
  a.Lq_rows = (int)Lq;
  a.Ld = (int)Ld;
  a.d = (int)d;
  a.shared_docs = 1;
  const int kind = dtype == FMX_DTYPE_BF16 ? fmx::KIND_BF16 : fmx::KIND_F16;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const FwdPlan p = plan_fwd(K, d);
  const hipError_t e = p.wide     ? fmx::launch_wide_fwd(kind, a, false, static_cast<float*>(workspace), workspace_bytes, s)
                       : p.splitd ? fmx::launch_splitd_fwd(kind, a, false, s)
                                  : fmx::launch_stream_fwd(kind, a, false, s);
  return hip_status(e, "fmx_fwd_sparse launch");
}

// Backward workspace: the dD index (when dD is written) at offset 0, then the
// dQ partial sums (when dQ is written).
static size_t bwd_dd_ws(int64_t Nq, int64_t B, int64_t Lq, int64_t Ld) {
  return fmx::bwd_dd_index_bytes(B, Nq * Lq, Ld);
}
static size_t bwd_dq_ws(int64_t Nq, int64_t B, int64_t Lq, int64_t d) {
  const int64_t rows = Nq * Lq;
  return (size_t)fmx::bwd_dq_chunks((int)B, (int)rows, (int)d) * (size_t)rows * (size_t)d * sizeof(float);
}

size_t fmx_bwd_batched_workspace_bytes(int64_t Nq, int64_t B, int64_t Lq, int64_t Ld, int64_t d) {
  if (Nq < 1 || B < 0 || Lq < 1 || Ld < 0 || d < 1 || Nq * Lq > INT32_MAX) return 0;
  return bwd_dd_ws(Nq, B, Lq, Ld) + bwd_dq_ws(Nq, B, Lq, d);
}

size_t fmx_bwd_workspace_bytes(int64_t B, int64_t Lq, int64_t Ld, int64_t d) {
  return fmx_bwd_batched_workspace_bytes(1, B, Lq, Ld, d);
}

int fmx_bwd_batched(int dtype, const void* Q, int64_t q_stride_n, int64_t q_stride_l, const void* D,
                    int64_t d_stride_b, int64_t d_stride_l, const int32_t* lengths, const int32_t* argmax,
                    const float* grad_scores, int64_t g_stride_n, int64_t g_stride_b, void* dQ, void* dD,
                    int64_t Nq, int64_t B, int64_t Lq, int64_t Ld, int64_t d, void* workspace,
                    size_t workspace_bytes, void* stream) {
  if (dtype != FMX_DTYPE_F16 && dtype != FMX_DTYPE_BF16) return fail(FMX_ERR_INVALID, "unknown dtype %d", dtype);
  int rc = check_common(Nq, B, Lq, Ld, d, q_stride_l, d_stride_b, d_stride_l, 2);
  if (rc) return rc;
  if (Ld < 1) return fail(FMX_ERR_INVALID, "backward needs Ld >= 1");
  if (g_stride_n < 0 || g_stride_b < 0) return fail(FMX_ERR_INVALID, "gradient strides must be >= 0");
  if (!dQ && !dD) return ok();
  if (!Q || !D || (B > 0 && (!argmax || !grad_scores))) return fail(FMX_ERR_INVALID, "Q, D, argmax and grad must be non-null");
  if (!aligned16(Q) || !aligned16(D)) return fail(FMX_ERR_INVALID, "Q and D must be 16-byte aligned");
  if ((dQ && !aligned16(dQ)) || (dD && !aligned16(dD))) return fail(FMX_ERR_INVALID, "dQ and dD must be 16-byte aligned");
  if (Nq > 1 && (q_stride_n & 7)) return fail(FMX_ERR_INVALID, "Q query stride must be a multiple of 8");
  if (dD) {
    if (Ld >= (1 << 19))
      return fail(FMX_ERR_UNSUPPORTED, "dD needs Ld < 2^19 (Ld=%lld)", (long long)Ld);
    if (Nq * Lq >= INT32_MAX || fmx::bwd_dd_chunks(Nq * Lq) > 65535)
      return fail(FMX_ERR_UNSUPPORTED, "Nq*Lq=%lld too large", (long long)(Nq * Lq));
  }
  const size_t dd_ws = dD ? bwd_dd_ws(Nq, B, Lq, Ld) : 0;
  const size_t need = dd_ws + (dQ ? bwd_dq_ws(Nq, B, Lq, d) : 0);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return fail(FMX_ERR_WORKSPACE, "workspace of %zu bytes required, %zu given", need, workspace_bytes);

  fmx::BwdArgs a = {};
  a.Q = Q;
  a.D = D;
  a.lengths = lengths;
  a.argmax = argmax;
  a.grad = grad_scores;
  a.dQ = dQ;
  a.dD = dD;
  if (workspace) {
    char* w = static_cast<char*>(workspace);
    a.dd_rows = reinterpret_cast<uint32_t*>(w);
    a.dd_ent = reinterpret_cast<uint16_t*>(w + (size_t)fmx::bwd_dd_chunks(Nq * Lq) * (size_t)B * (size_t)Ld *
                                           sizeof(uint32_t));
    a.ws = reinterpret_cast<float*>(w + dd_ws);
  }
  a.dd_slab = fmx::bwd_dd_slab((int)d);
  a.sq_n = Nq > 1 ? q_stride_n : 0;
  a.sq_l = q_stride_l;
  a.sd_b = d_stride_b;
  a.sd_l = d_stride_l;
  a.g_n = g_stride_n;
  a.g_b = g_stride_b;
  a.Nq = (int)Nq;
  a.B = (int)B;
  a.Lq = (int)Lq;
  a.Ld = (int)Ld;
  a.d = (int)d;
  a.nchunk = fmx::bwd_dq_chunks((int)B, (int)(Nq * Lq), (int)d);
  a.sort_n = fmx::bwd_sort_n(Nq * Lq);
  a.dd_chunks = (int)fmx::bwd_dd_chunks(Nq * Lq);
  const int kind = dtype == FMX_DTYPE_BF16 ? fmx::KIND_BF16 : fmx::KIND_F16;
  return hip_status(fmx::launch_bwd(kind, a, static_cast<hipStream_t>(stream)), "fmx_bwd launch");
}

int fmx_bwd(int dtype, const void* Q, int64_t q_stride_l, const void* D, int64_t d_stride_b,
            int64_t d_stride_l, const int32_t* argmax, const float* grad_scores, void* dQ, void* dD,
            int64_t B, int64_t Lq, int64_t Ld, int64_t d, void* workspace, size_t workspace_bytes,
            void* stream) {
  return fmx_bwd_batched(dtype, Q, 0, q_stride_l, D, d_stride_b, d_stride_l, nullptr, argmax, grad_scores, 0, 1,
                         dQ, dD, 1, B, Lq, Ld, d, workspace, workspace_bytes, stream);
}

}  // extern "C"
