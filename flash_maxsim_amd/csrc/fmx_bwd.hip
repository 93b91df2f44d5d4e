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
#include <mutex>

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
// chunk's docs, in order. Docs go in batches of DB: the batch's argmax, upstream
// gradients and lengths are loaded together, then its DB row chunks of D, so a
// thread has DB gathers in flight instead of one (a doc at a time costs two
// dependent memory round trips, and config 5's threads walk 32 docs each).
// Positions past the chunk read its last doc again and, like empty docs, are
// skipped (not multiplied by zero: a row may hold NaN padding); whether a doc
// counts depends on the doc alone, so the skip is uniform over the wave.
template <bool BF, bool FULL>
__device__ __forceinline__ void dq_partial_block(const BwdArgs& a, int bx, int by) {
  constexpr int DB = 8;
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
  for (int bb = b0; bb < b1; bb += DB) {
    int j[DB];
    float gb[DB];
    int bi[DB];
#pragma unroll
    for (int u = 0; u < DB; ++u) {
      bi[u] = bb + u < b1 ? bb + u : b1 - 1;
      j[u] = am[(int64_t)bi[u] * a.Lq];
      gb[u] = g[(int64_t)bi[u] * a.g_b];
    }
    bool live[DB];
#pragma unroll
    for (int u = 0; u < DB; ++u) {
      live[u] = bb + u < b1;
      if (a.lengths) live[u] = live[u] && a.lengths[bi[u]] > 0;
      j[u] = clamp_index(j[u], a.Ld);
    }
    float x[DB][8];
#pragma unroll
    for (int u = 0; u < DB; ++u) {
      const uint16_t* row = D + (int64_t)bi[u] * a.sd_b + (int64_t)j[u] * a.sd_l;
      if constexpr (FULL) {
        const uint4 v = *reinterpret_cast<const uint4*>(row + k0);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x[u][2 * e] = Elem<BF>::to_f(w[e] & 0xffffu);
          x[u][2 * e + 1] = Elem<BF>::to_f(w[e] >> 16);
        }
      } else {
        load8<BF>(row, k0, a.d, x[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < DB; ++u)
      if (live[u])
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = fmaf(gb[u], x[u][e], acc[e]);
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

constexpr int kEntryBits = 13;  // entries of one chunk < 2^13 (kDdChunk)
constexpr uint32_t kNoRow = 0xffffffffu;
constexpr int kDdMaxPasses = 4;  // workgroup row passes per dD writer slab, at most
// dD sizes from which the dQ chain runs on a second stream (launch_bwd_t).
constexpr int64_t kBwdForkBytes = (int64_t)1 << 24;

// dD index, one workgroup per (doc, chunk of kDdChunk consecutive (query,
// token) entries). The chunk's entries e become keys row << 13 | (e - e0) in
// LDS, bitonic-sorted, so each picked row's entries are contiguous and in
// entry order. Written to the workspace:
//   ent[b][e0 + p]     chunk-local entry of sorted position p (uint16)
//   rows[c][b][j]      first sorted position | count << 16 of row j within
//                      chunk c, or kNoRow.
// Chunks hold consecutive entries, so a row's entries taken chunk by chunk
// are in entry order. Docs of length 0 pick no rows.
__device__ __forceinline__ void dd_index_block(const BwdArgs& a, int b, int chunk, uint32_t* keys) {
  const int NL = a.Nq * a.Lq;
  const int e0 = chunk * kDdChunk;
  const int n = NL - e0 < kDdChunk ? NL - e0 : kDdChunk;  // entries of this chunk
  const bool empty = a.lengths && doc_len(a, b) == 0;
  for (int p = threadIdx.x; p < a.sort_n; p += 256) {
    uint32_t key = kNoRow;
    if (p < n && !empty) {
      const int e = e0 + p;
      const int qi = e / a.Lq, q = e - qi * a.Lq;
      const int j = clamp_index(a.argmax[((int64_t)qi * a.B + b) * a.Lq + q], a.Ld);
      key = ((uint32_t)j << kEntryBits) | (uint32_t)p;
    }
    keys[p] = key;
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
  uint16_t* ent = a.dd_ent + (int64_t)b * NL + e0;
  for (int p = threadIdx.x; p < n; p += 256) ent[p] = (uint16_t)(keys[p] & ((1u << kEntryBits) - 1));
  uint32_t* rows = a.dd_rows + ((int64_t)chunk * a.B + b) * a.Ld;
  for (int j = threadIdx.x; j < a.Ld; j += 256) {
    // first sorted position with row >= j (keys of empty slots are kNoRow)
    const uint32_t lo_key = (uint32_t)j << kEntryBits;
    int lo = 0, hi = n;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (keys[mid] < lo_key) lo = mid + 1; else hi = mid;
    }
    uint32_t info = kNoRow;
    if (lo < n && (keys[lo] >> kEntryBits) == (uint32_t)j) {
      int cnt = 1;
      while (lo + cnt < n && (keys[lo + cnt] >> kEntryBits) == (uint32_t)j) ++cnt;
      info = (uint32_t)lo | ((uint32_t)cnt << 16);
    }
    rows[j] = info;
  }
}

// dD writer: rows of [B, Ld, d] in memory order, a slab of consecutive rows
// per workgroup, so the stores stream like a fill of the whole tensor. A row
// no entry picked is zeros; a picked row is the fp32 sum over its entries, in
// entry order, of g[qi, b] * Q[qi, q]. Lanes cover a row's 8-wide k chunks:
// L = min(64, pow2 >= chunks) lanes per row, 64 / L rows per wave pass.
template <bool BF>
__device__ __forceinline__ void dd_write_block(const BwdArgs& a, int slab) {
  const int nkc = (a.d + 7) >> 3;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int lsh = 0;
  while ((1 << lsh) < nkc && lsh < 6) ++lsh;
  const int rpw = 64 >> lsh;               // rows per wave pass
  const int sub = lane >> lsh;             // this lane's row within the pass
  const int kc0 = lane & ((1 << lsh) - 1);
  const int64_t total = (int64_t)a.B * a.Ld;
  const int64_t r0 = (int64_t)slab * a.dd_slab;
  const int64_t r1 = r0 + a.dd_slab < total ? r0 + a.dd_slab : total;
  const int step = 4 * rpw;
  int64_t r = r0 + wave * rpw + sub;
  int b = (int)(r / a.Ld);
  int j = (int)(r - (int64_t)b * a.Ld);
  const int NL = a.Nq * a.Lq;
  const uint16_t* Q = static_cast<const uint16_t*>(a.Q);
  const float zero[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  // The row-index entries of all of this lane's passes (a slab is at most
  // kDdMaxPasses of them) are loaded up front, so their round trips overlap.
  uint32_t infos[kDdMaxPasses];
#pragma unroll
  for (int p = 0; p < kDdMaxPasses; ++p) {
    const int64_t rp = r + (int64_t)p * step;
    infos[p] = rp < r1 ? a.dd_rows[rp] : kNoRow;
  }
#pragma unroll
  for (int p = 0; p < kDdMaxPasses; ++p, r += step) {
    if (r >= r1) break;
    uint16_t* orow = static_cast<uint16_t*>(a.dD) + r * a.d;
    const uint32_t info0 = infos[p];
    if (a.dd_chunks == 1 && info0 == kNoRow) {
      for (int kc = kc0; kc < nkc; kc += 64) store8<BF>(orow, kc * 8, a.d, zero);
    } else {
      for (int kc = kc0; kc < nkc; kc += 64) {
        const int k0 = kc * 8;
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        // the row's entries chunk by chunk: entry order overall
        for (int ch = 0; ch < a.dd_chunks; ++ch) {
          const uint32_t info = ch == 0 ? info0 : a.dd_rows[(int64_t)ch * total + r];
          if (info == kNoRow) continue;
          const int e0 = ch * kDdChunk;
          const uint16_t* ent = a.dd_ent + (int64_t)b * NL + e0 + (info & 0xffffu);
          const int n = (int)(info >> 16);
          for (int i = 0; i < n; ++i) {
            const int e = e0 + ent[i];
            const int qi = e / a.Lq, q = e - qi * a.Lq;
            const float g = a.grad[(int64_t)qi * a.g_n + (int64_t)b * a.g_b];
            float x[8];
            load8<BF>(Q + (int64_t)qi * a.sq_n + (int64_t)q * a.sq_l, k0, a.d, x);
#pragma unroll
            for (int k = 0; k < 8; ++k) acc[k] = fmaf(g, x[k], acc[k]);
          }
        }
        store8<BF>(orow, k0, a.d, acc);
      }
    }
    j += step;
    while (j >= a.Ld) {
      j -= a.Ld;
      ++b;
    }
  }
}

template <bool BF, bool FULL>
__global__ void __launch_bounds__(256) bwd_dq_partial_kernel(BwdArgs a) {
  dq_partial_block<BF, FULL>(a, blockIdx.x, blockIdx.y);
}

__global__ void __launch_bounds__(256) bwd_dd_index_kernel(BwdArgs a) {
  extern __shared__ uint32_t smem[];
  dd_index_block(a, blockIdx.x, blockIdx.y, smem);
}

template <bool BF>
__global__ void __launch_bounds__(256) bwd_dd_write_kernel(BwdArgs a) {
  dd_write_block<BF>(a, blockIdx.x);
}

template <bool BF>
void launch_dq_chain(const BwdArgs& a, hipStream_t s) {
  const int nkc = (a.d + 7) >> 3;
  const int64_t threads = (int64_t)a.Nq * a.Lq * nkc;
  // FULL: every 8-wide chunk lies inside d, so each gather is one 16-byte load
  const dim3 grid((unsigned)((threads + 255) / 256), a.nchunk);
  if ((a.d & 7) == 0 && (a.sd_b & 7) == 0 && (a.sd_l & 7) == 0)
    hipLaunchKernelGGL((bwd_dq_partial_kernel<BF, true>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((bwd_dq_partial_kernel<BF, false>), grid, dim3(256), 0, s, a);
  const int64_t n = (int64_t)a.Nq * a.Lq * a.d;
  hipLaunchKernelGGL(bwd_dq_finalize_kernel<BF>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a);
}

template <bool BF>
void launch_dd_chain(const BwdArgs& a, hipStream_t s) {
  const size_t lds = bwd_dd_lds_bytes((int64_t)a.Nq * a.Lq);
  hipLaunchKernelGGL(bwd_dd_index_kernel, dim3((unsigned)a.B, (unsigned)a.dd_chunks), dim3(256), lds, s, a);
  const int64_t slabs = ((int64_t)a.B * a.Ld + a.dd_slab - 1) / a.dd_slab;
  hipLaunchKernelGGL(bwd_dd_write_kernel<BF>, dim3((unsigned)slabs), dim3(256), 0, s, a);
}

// A second stream per device for the dQ chain, with the two events that fork
// it from and join it to the caller's stream. Created on first use (default
// priority, non-blocking) and kept until the process ends. One mutex orders
// whole fork/launch/join sequences, so concurrent callers never interleave
// their event records.
constexpr int kBwdMaxDevices = 64;
struct BwdSide {
  hipStream_t st = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
std::mutex g_side_mu;
BwdSide g_side[kBwdMaxDevices];

hipError_t bwd_side(BwdSide** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kBwdMaxDevices) return hipErrorInvalidDevice;
  BwdSide& b = g_side[dev];
  if (!b.st) {
    hipStream_t st = nullptr;
    hipEvent_t f = nullptr, j = nullptr;
    if ((e = hipStreamCreateWithFlags(&st, hipStreamNonBlocking)) != hipSuccess) return e;
    if ((e = hipEventCreateWithFlags(&f, hipEventDisableTiming)) != hipSuccess) return e;
    if ((e = hipEventCreateWithFlags(&j, hipEventDisableTiming)) != hipSuccess) return e;
    b.fork = f;
    b.join = j;
    b.st = st;
  }
  *out = &b;
  return hipSuccess;
}

// dQ and dD run as separate launches: interleaving the read-bound dQ blocks
// with the write-bound dD blocks in one grid measured 15 % slower on config 5.
// When both are asked for and dD is large, the dQ chain (gather, sum) runs on
// a second stream beside the dD chain (index, writer): the two share only
// their inputs and write disjoint outputs and workspace regions, and the
// caller's stream waits for both. The small kernels of each chain then
// overlap the other's large one (config 5's step 430 -> 408 us with the
// forward). Under stream capture the chains stay on the caller's stream.
template <bool BF>
hipError_t launch_bwd_t(const BwdArgs& a, hipStream_t s) {
  const bool do_dd = a.dD && a.B > 0;
  const int64_t dd_bytes = (int64_t)a.B * a.Ld * a.d * 2;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (a.dQ && do_dd && dd_bytes >= kBwdForkBytes && hipStreamIsCapturing(s, &cap) == hipSuccess &&
      cap == hipStreamCaptureStatusNone) {
    std::lock_guard<std::mutex> lock(g_side_mu);
    BwdSide* side = nullptr;
    hipError_t e = bwd_side(&side);
    if (e != hipSuccess) return e;
    if ((e = hipEventRecord(side->fork, s)) != hipSuccess) return e;
    if ((e = hipStreamWaitEvent(side->st, side->fork, 0)) != hipSuccess) return e;
    launch_dq_chain<BF>(a, side->st);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if ((e = hipEventRecord(side->join, side->st)) != hipSuccess) return e;
    launch_dd_chain<BF>(a, s);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    return hipStreamWaitEvent(s, side->join, 0);
  }
  if (a.dQ) launch_dq_chain<BF>(a, s);
  if (do_dd) launch_dd_chain<BF>(a, s);
  return hipGetLastError();
}

}  // namespace

// Doc chunks of the dQ gather: about 2^17 (row, k-chunk, doc-chunk) threads,
// at most 64 chunks, at least 8 docs each. Each thread keeps 8 gathers in
// flight, so fewer, longer chunks keep the loads going with less partial-sum
// traffic (config 5, 8 chunks: step 437 us; 16: 439; 32: 444).
int bwd_dq_chunks(int B, int rows, int d) {
  if (B <= 0) return 1;
  const int64_t per_chunk = (int64_t)rows * ((d + 7) / 8);
  int64_t n = ((int64_t)1 << 17) / (per_chunk > 0 ? per_chunk : 1);
  const int64_t by_docs = (B + 7) / 8;
  if (n > by_docs) n = by_docs;
  if (n > 64) n = 64;
  if (n < 1) n = 1;
  return (int)n;
}

// Sort size of one dD index chunk: a power of two >= the chunk's entries.
int bwd_sort_n(int64_t entries) {
  int n = 64;
  while (n < entries && n < kDdChunk) n <<= 1;
  return n;
}

int64_t bwd_dd_chunks(int64_t entries) { return entries > 0 ? (entries + kDdChunk - 1) / kDdChunk : 1; }

size_t bwd_dd_lds_bytes(int64_t entries) { return (size_t)bwd_sort_n(entries) * sizeof(uint32_t); }

// Workspace of the dD index: rows [chunks, B, Ld] uint32, then ent [B, entries] uint16.
size_t bwd_dd_index_bytes(int64_t B, int64_t entries, int64_t Ld) {
  const size_t rows = (size_t)bwd_dd_chunks(entries) * (size_t)B * (size_t)Ld * sizeof(uint32_t);
  return rows + (((size_t)B * (size_t)entries * sizeof(uint16_t) + 255) & ~(size_t)255);
}

// Rows per dD writer workgroup: about 16 KB of output, a whole number of
// the workgroup's row passes (4 waves x 64 / L rows, L lanes per row), at
// most kDdMaxPasses of them.
int bwd_dd_slab(int d) {
  const int nkc = (d + 7) / 8;
  int lsh = 0;
  while ((1 << lsh) < nkc && lsh < 6) ++lsh;
  const int pass = 4 * (64 >> lsh);
  int rows = 16384 / (2 * d);
  if (rows < pass) rows = pass;
  if (rows > kDdMaxPasses * pass) rows = kDdMaxPasses * pass;
  return (rows + pass - 1) / pass * pass;
}

hipError_t launch_bwd(int kind, const BwdArgs& a, hipStream_t s) {
  switch (kind) {
    case KIND_F16: return launch_bwd_t<false>(a, s);
    case KIND_BF16: return launch_bwd_t<true>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fmx
