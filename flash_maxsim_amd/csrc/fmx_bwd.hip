// Argmax backward of MaxSim (single or batched queries over shared docs).
//
// Replaces _maxsim_bwd_dQ_kernel and _maxsim_bwd_dD_kernel (reference
// flash_maxsim/flash_maxsim.py:153-188) with the same mathematics, extended to
// Nq queries and doc lengths (a = argmax, g = upstream gradient of scores):
//   dQ[qi, q, :] = sum_b g[qi, b] * D[b, a[qi*B + b, q], :]
//   dD[b, j, :]  = sum_{(qi, q) : a[qi*B + b, q] = j} g[qi, b] * Q[qi, q, :]
// Docs of length 0 (every similarity masked, score -inf) take no part, as in
// autograd through the masked naive MaxSim.
// Differences by design:
//  * dQ is a two-stage gather-reduce: doc chunks accumulate fp32 partials in a
//    caller workspace, then a second kernel adds the chunks in order. The
//    reference runs one program per query token looping over every doc.
//  * dD is written exactly once per element by the doc's workgroup (zeros for
//    rows no query token picked, the fp32 sum for picked rows, in (query,
//    token) order), so there is no torch.zeros_like memset and no fp16
//    atomics; results are bitwise deterministic.
#include "fmx_device.h"
#include "fmx_kernels.h"

namespace fmx {
namespace {

template <bool BF>
struct Elem;
template <>
struct Elem<false> {
  static __device__ __forceinline__ float to_f(uint16_t v) { return (float)__builtin_bit_cast(_Float16, v); }
  static __device__ __forceinline__ uint16_t from_f(float x) {
    return __builtin_bit_cast(uint16_t, (_Float16)x);
  }
};
template <>
struct Elem<true> {
  static __device__ __forceinline__ float to_f(uint16_t v) {
    return __builtin_bit_cast(float, (uint32_t)v << 16);
  }
  static __device__ __forceinline__ uint16_t from_f(float x) {
    return __builtin_bit_cast(uint16_t, (__bf16)x);
  }
};

// Loads elements k0 .. k0+7 (those < d) of a 2-byte row as fp32.
template <bool BF>
__device__ __forceinline__ void load8(const uint16_t* row, int k0, int d, float (&x)[8]) {
  if (k0 + 8 <= d) {
    const uint4 v = *reinterpret_cast<const uint4*>(row + k0);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = Elem<BF>::to_f(w[e] & 0xffffu);
      x[2 * e + 1] = Elem<BF>::to_f(w[e] >> 16);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = (k0 + e < d) ? Elem<BF>::to_f(row[k0 + e]) : 0.f;
  }
}

// Stores elements k0 .. k0+7 (those < d); 16-byte stores need d % 8 == 0 so
// that every row of the contiguous output starts 16-byte aligned. dD is
// written once and read only by the optimiser later: non-temporal stores
// stream it out instead of leaving it dirty in the caches, where its
// write-back would compete with the next forward's reads.
template <bool BF>
__device__ __forceinline__ void store8(uint16_t* row, int k0, int d, const float (&x)[8]) {
  if ((d & 7) == 0) {
    u32x4_t v;
    v[0] = (uint32_t)Elem<BF>::from_f(x[0]) | ((uint32_t)Elem<BF>::from_f(x[1]) << 16);
    v[1] = (uint32_t)Elem<BF>::from_f(x[2]) | ((uint32_t)Elem<BF>::from_f(x[3]) << 16);
    v[2] = (uint32_t)Elem<BF>::from_f(x[4]) | ((uint32_t)Elem<BF>::from_f(x[5]) << 16);
    v[3] = (uint32_t)Elem<BF>::from_f(x[6]) | ((uint32_t)Elem<BF>::from_f(x[7]) << 16);
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(row + k0));
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (k0 + e < d) row[k0 + e] = Elem<BF>::from_f(x[e]);
  }
}

__device__ __forceinline__ int clamp_index(int j, int Ld) { return j < 0 ? 0 : (j >= Ld ? Ld - 1 : j); }

__device__ __forceinline__ int doc_len(const BwdArgs& a, int b) {
  if (!a.lengths) return a.Ld;
  const int l = a.lengths[b];
  return l < 0 ? 0 : (l > a.Ld ? a.Ld : l);
}

// Stage 1 of dQ: one thread per (query token row r = qi*Lq + q, 8-wide k
// chunk), one grid row per chunk of docs; ws[chunk][r][k] = sum over the
// chunk's docs, in order.
template <bool BF>
__device__ __forceinline__ void dq_partial_block(const BwdArgs& a, int bx, int by) {
  const int nkc = (a.d + 7) >> 3;
  const int64_t rows = (int64_t)a.Nq * a.Lq;
  const int64_t tid = (int64_t)bx * 256 + threadIdx.x;
  if (tid >= rows * nkc) return;
  const int64_t r = tid / nkc;
  const int k0 = (int)(tid - r * nkc) * 8;
  const int qi = (int)(r / a.Lq), q = (int)(r - (int64_t)qi * a.Lq);
  const int per = (a.B + a.nchunk - 1) / a.nchunk;
  const int b0 = by * per;
  const int b1 = min(a.B, b0 + per);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const uint16_t* D = static_cast<const uint16_t*>(a.D);
  const int32_t* am = a.argmax + (int64_t)qi * a.B * a.Lq + q;
  const float* g = a.grad + (int64_t)qi * a.g_n;
#pragma unroll 4
  for (int b = b0; b < b1; ++b) {
    if (a.lengths && doc_len(a, b) == 0) continue;
    const int j = clamp_index(am[(int64_t)b * a.Lq], a.Ld);
    const float gb = g[(int64_t)b * a.g_b];
    float x[8];
    load8<BF>(D + (int64_t)b * a.sd_b + (int64_t)j * a.sd_l, k0, a.d, x);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = fmaf(gb, x[e], acc[e]);
  }
  float* out = a.ws + ((int64_t)by * rows + r) * a.d + k0;
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (k0 + e < a.d) out[e] = acc[e];
}

// Stage 2 of dQ: dQ[r][k] = sum over chunks (in order) of ws[chunk][r][k].
template <bool BF>
__global__ void __launch_bounds__(256) bwd_dq_finalize_kernel(BwdArgs a) {
  const int64_t n = (int64_t)a.Nq * a.Lq * a.d;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  float s = 0.f;
#pragma unroll 8
  for (int c = 0; c < a.nchunk; ++c) s += a.ws[(int64_t)c * n + i];  // chunk order: deterministic
  static_cast<uint16_t*>(a.dQ)[i] = Elem<BF>::from_f(s);
}

constexpr int kEntryBits = 13;  // (query, token) entries per doc < 2^13

// dD for one doc per workgroup. LDS: the doc's (query, token) entries as keys
// row << 13 | entry, sorted ascending (bitonic), and a bitmap of picked rows.
// A picked row's entries are then contiguous and in entry order.
template <bool BF>
__device__ __forceinline__ void dd_block(const BwdArgs& a, int b, uint32_t* smem) {
  uint32_t* keys = smem;
  uint32_t* hit = smem + a.sort_n;
  const int nkc = (a.d + 7) >> 3;
  const int NL = a.Nq * a.Lq;
  const bool empty = a.lengths && doc_len(a, b) == 0;
  const int nwords = (a.Ld + 31) >> 5;
  for (int i = threadIdx.x; i < nwords; i += 256) hit[i] = 0u;
  __syncthreads();
  for (int e = threadIdx.x; e < a.sort_n; e += 256) {
    uint32_t key = 0xffffffffu;
    if (e < NL && !empty) {
      const int qi = e / a.Lq, q = e - qi * a.Lq;
      const int j = clamp_index(a.argmax[((int64_t)qi * a.B + b) * a.Lq + q], a.Ld);
      key = ((uint32_t)j << kEntryBits) | (uint32_t)e;
      atomicOr(&hit[j >> 5], 1u << (j & 31));
    }
    keys[e] = key;
  }
  __syncthreads();
  for (int size = 2; size <= a.sort_n; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int p = threadIdx.x; p < a.sort_n / 2; p += 256) {
        const int i = 2 * stride * (p / stride) + (p % stride);
        const int j = i + stride;
        const bool asc = (i & size) == 0;
        const uint32_t x = keys[i], y = keys[j];
        if ((x > y) == asc) {
          keys[i] = y;
          keys[j] = x;
        }
      }
      __syncthreads();
    }
  }

  // Rows are dealt to the four waves; a wave's lanes cover a row's 8-wide
  // k chunks, so each store instruction writes 64 contiguous chunks and all
  // row/chunk arithmetic is 32-bit without divisions.
  uint16_t* out = static_cast<uint16_t*>(a.dD) + (int64_t)b * a.Ld * a.d;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const float zero[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int row = wave; row < a.Ld; row += 4) {
    if ((hit[row >> 5] >> (row & 31)) & 1u) continue;  // uniform over the wave
    uint16_t* orow = out + (int64_t)row * a.d;
    for (int kc = lane; kc < nkc; kc += 64) store8<BF>(orow, kc * 8, a.d, zero);
  }
  if (empty) return;
  const uint16_t* Q = static_cast<const uint16_t*>(a.Q);
  for (int p = wave; p < NL; p += 4) {
    const uint32_t j = keys[p] >> kEntryBits;
    if (p > 0 && (keys[p - 1] >> kEntryBits) == j) continue;  // not the first entry of its row
    // The row's entries keys[p .. p2) in entry order, their query rows
    // weighted by the upstream gradient of (query, doc).
    for (int kc = lane; kc < nkc; kc += 64) {
      const int k0 = kc * 8;
      float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int p2 = p; p2 < NL && (keys[p2] >> kEntryBits) == j; ++p2) {
        const int e = (int)(keys[p2] & ((1u << kEntryBits) - 1));
        const int qi = e / a.Lq, q = e - qi * a.Lq;
        const float g = a.grad[(int64_t)qi * a.g_n + (int64_t)b * a.g_b];
        float x[8];
        load8<BF>(Q + (int64_t)qi * a.sq_n + (int64_t)q * a.sq_l, k0, a.d, x);
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[k] = fmaf(g, x[k], acc[k]);
      }
      store8<BF>(out + (int64_t)j * a.d, k0, a.d, acc);
    }
  }
}

template <bool BF>
__global__ void __launch_bounds__(256) bwd_dq_partial_kernel(BwdArgs a) {
  dq_partial_block<BF>(a, blockIdx.x, blockIdx.y);
}

template <bool BF>
__global__ void __launch_bounds__(256) bwd_dd_kernel(BwdArgs a) {
  extern __shared__ uint32_t smem[];
  dd_block<BF>(a, blockIdx.x, smem);
}

// dQ and dD run as separate launches: interleaving the read-bound dQ blocks
// with the write-bound dD blocks in one grid measured 15 % slower on config 5.
template <bool BF>
hipError_t launch_bwd_t(const BwdArgs& a, hipStream_t s) {
  const int nkc = (a.d + 7) >> 3;
  if (a.dQ) {
    const int64_t threads = (int64_t)a.Nq * a.Lq * nkc;
    hipLaunchKernelGGL(bwd_dq_partial_kernel<BF>, dim3((unsigned)((threads + 255) / 256), a.nchunk), dim3(256),
                       0, s, a);
    const int64_t n = (int64_t)a.Nq * a.Lq * a.d;
    hipLaunchKernelGGL(bwd_dq_finalize_kernel<BF>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a);
  }
  if (a.dD && a.B > 0) {
    const size_t lds = bwd_dd_lds_bytes((int64_t)a.Nq * a.Lq, a.Ld);
    hipLaunchKernelGGL(bwd_dd_kernel<BF>, dim3((unsigned)a.B), dim3(256), lds, s, a);
  }
  return hipGetLastError();
}

}  // namespace

// Doc chunks of the dQ gather: enough (row, k-chunk, doc-chunk) threads to keep
// the GPU's loads in flight (about 2^19), at most 64 chunks, at least 8 docs each.
int bwd_dq_chunks(int B, int rows, int d) {
  if (B <= 0) return 1;
  const int64_t per_chunk = (int64_t)rows * ((d + 7) / 8);
  int64_t n = ((int64_t)1 << 19) / (per_chunk > 0 ? per_chunk : 1);
  const int64_t by_docs = (B + 7) / 8;
  if (n > by_docs) n = by_docs;
  if (n > 64) n = 64;
  if (n < 1) n = 1;
  return (int)n;
}

int bwd_sort_n(int64_t entries) {
  int n = 64;
  while (n < entries) n <<= 1;
  return n;
}

size_t bwd_dd_lds_bytes(int64_t entries, int64_t Ld) {
  return ((size_t)bwd_sort_n(entries) + (size_t)((Ld + 31) / 32)) * sizeof(uint32_t);
}

hipError_t launch_bwd(int kind, const BwdArgs& a, hipStream_t s) {
  switch (kind) {
    case KIND_F16: return launch_bwd_t<false>(a, s);
    case KIND_BF16: return launch_bwd_t<true>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fmx
