// MaxSim forward for embeddings wider than the split-d kernel's 4096 (up to
// FMX_MAX_D): the reference pads any d to a power of two and keeps one query
// token's full row per program (flash_maxsim/flash_maxsim.py:8-9, :80-146);
// here a query tile of that width fits neither VGPRs nor LDS, so the forward
// runs in two kernels over chunks of (query, doc) items:
//  * wide_sim_kernel: each wave computes the similarities of 32 doc tokens
//    (two 16-token tiles) against up to 128 query tokens (eight 16-token
//    blocks) over the whole of d on v_mfma_f32_16x16x32 with fp32
//    accumulation, reading doc fragments once from HBM and the workgroup's
//    query rows through LDS four 32-wide k-steps at a time, and stores them
//    to the workspace S[item][query token][doc token];
//  * wide_reduce_kernel: per item, the max over each query token's row of S
//    up to the doc's length (the first index reaching it, with torch.max's NaN
//    rule, when the argmax is requested), summed over query tokens in order.
// uint8 docs are dequantised to fp16 per fragment as the reference's int8
// kernel does (flash_maxsim_quant.py:89) before the MFMA. Sparse scoring
// (query rows gathered per doc), per-query docs and packed docs address their
// rows as the other kernels do (query_row_offset, make_doc_res).
// Bound: HBM for the doc stream at small query counts; the S round trip adds
// 8 x Lq bytes per doc token to the d x 2 (fp16) read (1.6 % at Lq = 32,
// d = 8192).
#include <type_traits>

#include "fmx_kernels.h"
#include "fmx_tile.h"

namespace fmx {
namespace {

constexpr int kWideQB = 8;     // 16-token query blocks per similarity pass, at most
constexpr int kWideTW = 2;     // 16-token doc tiles per wave
constexpr int kWideKC = 4;     // k-steps per staged query chunk
constexpr int kWideQRow = 80;  // LDS bytes per query row and k-step: 64 + 16 spreads a b128 read over all banks

// Item (query qi, doc b) of the call, its doc row and the doc's length.
__device__ __forceinline__ void wide_item(const FwdArgs& a, int item, int& qi, int& b, int64_t& drow, int& len) {
  qi = a.Nq > 1 ? item / a.B : 0;
  b = item - qi * a.B;
  drow = a.shared_docs ? (int64_t)b : (int64_t)item;
  len = a.lengths ? a.lengths[drow] : a.Ld;
  len = len < 0 ? 0 : (len > a.Ld ? a.Ld : len);
}

// blockIdx.x: item of the chunk; blockIdx.y: group of 4 * kWideTW doc tiles;
// blockIdx.z: group of QB query blocks. S rows are ldp floats apart.
// The workgroup's 16 * QB query rows come through LDS kWideKC k-steps at a
// time (each thread loads 16 bytes of up to two rows per k-step), so L2 serves
// each query fragment once per workgroup instead of once per wave; the next
// chunk's query and doc fragments are loaded while this chunk's MFMAs run.
// QB (2, 4 or 8) follows the query: a 32-token query's accumulators and
// staging take a quarter of the 128-row instance's registers and LDS, so more
// waves share a CU.
template <int KIND, int QB>
__global__ void __launch_bounds__(256) wide_sim_kernel(FwdArgs a, float* S, int item0, int ldp) {
  constexpr bool U8 = KIND == KIND_U8;
  constexpr int ESZ = KindInfo<KIND>::esz;
  constexpr int NH = (16 * QB + 63) / 64;  // staged rows per thread and k-step
  __shared__ __attribute__((aligned(16))) unsigned char qs[kWideKC][16 * QB * kWideQRow];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15, g = lane >> 4;
  const int il = blockIdx.x, item = item0 + il;
  int qi, b, len;
  int64_t drow;
  wide_item(a, item, qi, b, drow, len);
  if (blockIdx.y * 4 * kWideTW * 16 >= len) return;  // the whole workgroup: before any barrier
  const int tile0 = (blockIdx.y * 4 + wave) * kWideTW;
  const bool active = tile0 * 16 < len;  // wave-uniform; inactive waves still stage query rows
  const int qb0 = blockIdx.z * QB;
  const int nqb = (a.Lq + 15) / 16 - qb0 < QB ? (a.Lq + 15) / 16 - qb0 : QB;
  const int kp = a.d & ~7;
  const u32x4_t pmask = prefix_mask16(a.d & 7);

  // query staging: thread (r, p) = (tid / 4, tid % 4) loads bytes 16p .. 16p+15 of
  // each k-step of rows r (and r + 64) of the block group
  const rsrc_t rq = make_rsrc((const char*)a.Q + (int64_t)qi * a.sq_n * 2, (uint32_t)(a.Lq_rows * a.sq_l * 2));
  const int sr = tid >> 2, sp = tid & 3;
  uint32_t qoff[NH];
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    const int r = sr + 64 * h;
    qoff[h] = r < 16 * nqb ? query_row_offset(a, b, qb0 * 16 + r) : kOOB;
  }
  u32x4_t vq[NH][kWideKC];
  auto qload = [&](int kc) {
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
      for (int t = 0; t < kWideKC; ++t) {
        const int k = (kc * kWideKC + t) * 32 + 8 * sp;
        vq[h][t] = ld16(rq, k < a.d ? qoff[h] + (uint32_t)(k * 2) : kOOB);
        if (k == kp) vq[h][t] &= pmask;
      }
  };
  auto qstore = [&]() {
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      if (sr + 64 * h < 16 * QB) {  // rows of the block group only
#pragma unroll
        for (int t = 0; t < kWideKC; ++t)
          *reinterpret_cast<u32x4_t*>(&qs[t][(sr + 64 * h) * kWideQRow + 16 * sp]) = vq[h][t];
      }
    }
  };

  // doc rows: each lane loads token tile*16 + c, as in load_tile; rows past
  // the length read zeros and their similarities are never reduced
  const DocRes dr = make_doc_res<KIND, false>(a, drow, len);
  uint32_t drowoff[kWideTW];
  uint16_t sc[kWideTW], mn[kWideTW];
#pragma unroll
  for (int w = 0; w < kWideTW; ++w) {
    const int row = (tile0 + w) * 16 + c;
    drowoff[w] = (uint32_t)row * dr.rowb;
    if constexpr (U8) {
      sc[w] = ld2(dr.s, dr.ss + (uint32_t)row * 2u);
      mn[w] = ld2(dr.m, dr.sm + (uint32_t)row * 2u);
    }
  }
  using Raw = typename std::conditional<U8, u32x2_t, u32x4_t>::type;
  Raw vd[kWideTW][kWideKC];
  auto dload = [&](int kc) {
#pragma unroll
    for (int w = 0; w < kWideTW; ++w)
#pragma unroll
      for (int t = 0; t < kWideKC; ++t) {
        const int k0 = (kc * kWideKC + t) * 32 + 8 * g;
        const uint32_t o = k0 < a.d ? drowoff[w] + (uint32_t)(k0 * ESZ) : kOOB;
        if constexpr (U8) {
          vd[w][t] = ld8(dr.d, active ? o : kOOB);
        } else {
          vd[w][t] = ld16(dr.d, active ? o : kOOB);
          if (k0 == kp) vd[w][t] &= pmask;  // the row's elements past d are not the doc's
        }
      }
  };

  f32x4_t acc[kWideTW][QB];
#pragma unroll
  for (int w = 0; w < kWideTW; ++w)
#pragma unroll
    for (int nb = 0; nb < QB; ++nb) acc[w][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int nkc = (a.d + 32 * kWideKC - 1) / (32 * kWideKC);
  qload(0);
  dload(0);
  for (int kc = 0; kc < nkc; ++kc) {
    __syncthreads();  // the previous chunk's readers are done with qs
    qstore();
    u32x4_t af[kWideTW][kWideKC];
#pragma unroll
    for (int w = 0; w < kWideTW; ++w)
#pragma unroll
      for (int t = 0; t < kWideKC; ++t) {
        if constexpr (U8) {
          af[w][t] = dequant_biased_f16(codes_to_f16_biased(vd[w][t]), sc[w], mn[w]);
        } else {
          af[w][t] = vd[w][t];
        }
      }
    __syncthreads();
    if (kc + 1 < nkc) {
      qload(kc + 1);
      dload(kc + 1);
    }
    if (active) {
#pragma unroll
      for (int t = 0; t < kWideKC; ++t)
#pragma unroll
        for (int nb = 0; nb < QB; ++nb) {
          if (nb < nqb) {  // uniform
            const u32x4_t bq = *reinterpret_cast<const u32x4_t*>(&qs[t][(16 * nb + c) * kWideQRow + 16 * g]);
#pragma unroll
            for (int w = 0; w < kWideTW; ++w)
              acc[w][nb] = mfma16x16x32<KindInfo<KIND>::bf>(af[w][t], bq, acc[w][nb]);
          }
        }
    }
  }
  if (!active) return;

  // result lane (c, g): doc tokens tile*16 + 4g .. +3 of query token 16*qb + c
  float* Si = S + (int64_t)il * a.Lq * ldp;
#pragma unroll
  for (int nb = 0; nb < QB; ++nb) {
    const int q = (qb0 + nb) * 16 + c;
    if (nb < nqb && q < a.Lq) {
#pragma unroll
      for (int w = 0; w < kWideTW; ++w) {
        const int tok = (tile0 + w) * 16 + 4 * g;
        if (tok < len) *reinterpret_cast<f32x4_t*>(Si + (int64_t)q * ldp + tok) = acc[w][nb];
      }
    }
  }
}

// One workgroup per item: wave w reduces query tokens w, w + 4, ... and sums
// its maxima in that order; the four sums are added in wave order.
template <bool ARGMAX>
__global__ void __launch_bounds__(256) wide_reduce_kernel(FwdArgs a, const float* S, int item0, int ldp) {
  __shared__ float part[4];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int il = blockIdx.x, item = item0 + il;
  int qi, b, len;
  int64_t drow;
  wide_item(a, item, qi, b, drow, len);
  const float* Si = S + (int64_t)il * a.Lq * ldp;
  float sum = 0.f;
  for (int q = wave; q < a.Lq; q += 4) {
    const float* row = Si + (int64_t)q * ldp;
    float m = -INFINITY;
    int mi = 0;
    for (int j = lane; j < len; j += 64) {
      if constexpr (ARGMAX) {
        argmax_fold(row[j], j, m, mi);
      } else {
        m = vmax(m, row[j]);
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float om = __shfl_xor(m, off);
      if constexpr (ARGMAX) {
        const int oi = __shfl_xor(mi, off);
        argmax_merge(m, mi, om, oi);
      } else {
        m = vmax(m, om);
      }
    }
    if (ARGMAX && lane == 0) a.argmax[(int64_t)item * a.Lq + q] = mi;
    sum += m;
  }
  if (lane == 0) part[wave] = sum;
  __syncthreads();
  if (threadIdx.x == 0) store_score(a, qi, b, ((part[0] + part[1]) + part[2]) + part[3]);
}

int wide_ldp(int Ld) { return (Ld + 15) & ~15; }

template <int KIND>
hipError_t launch_kind(const FwdArgs& a, bool with_argmax, float* ws, size_t ws_bytes, hipStream_t s) {
  const int64_t items = (int64_t)a.Nq * a.B;
  const int ldp = wide_ldp(a.Ld);
  const size_t per = wide_item_bytes(a.Lq, a.Ld);
  int64_t chunk = per ? (int64_t)(ws_bytes / per) : items;  // Ld = 0: no similarities, only the reduction
  if (chunk < 1) return hipErrorInvalidValue;
  if (chunk > items) chunk = items;
  const int ntile = (a.Ld + 15) / 16;
  const int nqb = (a.Lq + 15) / 16;
  const int qb = nqb <= 2 ? 2 : nqb <= 4 ? 4 : kWideQB;
  const dim3 sgrid(1u, (unsigned)((ntile + 4 * kWideTW - 1) / (4 * kWideTW)), (unsigned)((nqb + qb - 1) / qb));
  for (int64_t i0 = 0; i0 < items; i0 += chunk) {
    const int n = (int)(items - i0 < chunk ? items - i0 : chunk);
    if (ntile > 0) {
      const dim3 grid((unsigned)n, sgrid.y, sgrid.z);
      if (qb == 2) {
        hipLaunchKernelGGL((wide_sim_kernel<KIND, 2>), grid, dim3(256), 0, s, a, ws, (int)i0, ldp);
      } else if (qb == 4) {
        hipLaunchKernelGGL((wide_sim_kernel<KIND, 4>), grid, dim3(256), 0, s, a, ws, (int)i0, ldp);
      } else {
        hipLaunchKernelGGL((wide_sim_kernel<KIND, kWideQB>), grid, dim3(256), 0, s, a, ws, (int)i0, ldp);
      }
    }
    if (with_argmax) {
      hipLaunchKernelGGL(wide_reduce_kernel<true>, dim3((unsigned)n), dim3(256), 0, s, a, ws, (int)i0, ldp);
    } else {
      hipLaunchKernelGGL(wide_reduce_kernel<false>, dim3((unsigned)n), dim3(256), 0, s, a, ws, (int)i0, ldp);
    }
  }
  return hipGetLastError();
}

}  // namespace

size_t wide_item_bytes(int64_t Lq, int64_t Ld) { return (size_t)Lq * (size_t)wide_ldp((int)Ld) * sizeof(float); }

size_t wide_fwd_workspace_bytes(int64_t items, int64_t Lq, int64_t Ld) {
  if (items < 1 || Lq < 1 || Ld < 0) return 0;
  const size_t per = wide_item_bytes(Lq, Ld);
  if (per == 0) return 0;
  int64_t chunk = (int64_t)(kWideChunkBytes / per);
  if (chunk < 1) chunk = 1;
  if (chunk > items) chunk = items;
  return (size_t)chunk * per;
}

hipError_t launch_wide_fwd(int kind, const FwdArgs& a, bool with_argmax, float* ws, size_t ws_bytes, hipStream_t s) {
  if ((int64_t)a.Nq * a.B > 0x7fffffff) return hipErrorInvalidValue;
  switch (kind) {
    case KIND_F16: return launch_kind<KIND_F16>(a, with_argmax, ws, ws_bytes, s);
    case KIND_BF16: return launch_kind<KIND_BF16>(a, with_argmax, ws, ws_bytes, s);
    case KIND_U8: return launch_kind<KIND_U8>(a, false, ws, ws_bytes, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fmx
