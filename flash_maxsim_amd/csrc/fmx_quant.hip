// Per-token uint8 quantisation on the GPU: the encoder of the storage format
// the uint8 forward kernels read.
//
// Computes, for every doc token row x of d values, exactly what the reference
// quantize_int8 (flash_maxsim/flash_maxsim_quant.py:11-28) computes with torch
// ops, in one pass over the input:
//   lo   = min(x), hi = max(x)                        (x widened to fp32)
//   step = max((hi - lo) / 255, 1e-8)                 (fp32, correctly rounded /)
//   code = clamp(round_half_even((x - lo) / step), 0, 255)
//   scale = fp16(step), min = fp16(lo)                (round to nearest even)
// Every operation is a single IEEE fp32 operation in the same order, so codes,
// scales and mins are bit-identical to the torch formula.
//
// Output rows: token (b, j) goes to row b*Ld + j of a padded [B, Ld, d] code
// tensor (the reference layout), or, for the packed layout, to row
// 4*tok_group[b] + j with only the first lengths[b] tokens of each doc stored;
// rows between a doc's length and the next multiple of 4 get zero codes,
// scales and mins.
//
// Mapping: LPR lanes share a token row (LPR = 8-element chunks of d rounded up
// to a power of two, at most 64); each lane handles CPL chunks of 8 elements.
// Row min/max meet through cross-lane shuffles inside the LPR-lane group.
#include "fmx_device.h"
#include "fmx_kernels.h"

namespace fmx {
namespace {

template <int SRC>
__device__ __forceinline__ float src_elem(const void* p, int64_t i) {
  if constexpr (SRC == 0) {
    return (float)static_cast<const _Float16*>(p)[i];
  } else if constexpr (SRC == 1) {
    return bf16_bits_to_float(static_cast<const uint16_t*>(p)[i]);
  } else {
    return static_cast<const float*>(p)[i];
  }
}

// Eight consecutive source elements k0..k0+7 of a row; elements at or past d
// are not read (they come back as 0 and are excluded by the caller).
template <int SRC>
__device__ __forceinline__ void load8(const void* row, int k0, int d, bool vec, float (&x)[8]) {
  if (vec && k0 + 8 <= d) {
    if constexpr (SRC == 2) {
      const f32x4_t a = *reinterpret_cast<const f32x4_t*>(static_cast<const float*>(row) + k0);
      const f32x4_t b = *reinterpret_cast<const f32x4_t*>(static_cast<const float*>(row) + k0 + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[i] = a[i];
        x[4 + i] = b[i];
      }
    } else {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(row) + k0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (SRC == 0) {
          x[2 * i] = half_bits_to_float(v[i] & 0xffffu);
          x[2 * i + 1] = half_bits_to_float(v[i] >> 16);
        } else {
          x[2 * i] = bf16_bits_to_float(v[i] & 0xffffu);
          x[2 * i + 1] = bf16_bits_to_float(v[i] >> 16);
        }
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = k0 + i < d ? src_elem<SRC>(row, k0 + i) : 0.f;
  }
}

template <int SRC, int LPR, int CPL>
__global__ void __launch_bounds__(256) quantize_kernel(QuantArgs a) {
  constexpr int RPB = 256 / LPR;  // token rows per block pass
  const int lane_in_row = threadIdx.x % LPR;
  const int64_t Ld4 = (a.Ld + 3) & ~(int64_t)3;
  const int64_t rows = a.B * Ld4;
  for (int64_t r = (int64_t)blockIdx.x * RPB + threadIdx.x / LPR; r < rows; r += (int64_t)gridDim.x * RPB) {
    const int64_t b = r / Ld4, j = r - b * Ld4;
    int64_t len = a.Ld;
    if (a.lengths) {
      len = a.lengths[b];
      len = len < 0 ? 0 : (len > a.Ld ? a.Ld : len);
    }
    const bool packed = a.tok_group != nullptr;
    // Padded layout: every real token row. Packed: the first len tokens, plus
    // zero rows up to the next multiple of 4.
    if (packed ? j >= ((len + 3) & ~(int64_t)3) : j >= a.Ld) continue;
    const int64_t orow = packed ? 4 * a.tok_group[b] + j : b * a.Ld + j;
    uint8_t* crow = a.codes + orow * a.c_stride_l;
    uint16_t* sp = static_cast<uint16_t*>(a.scales) + (packed ? orow : b * a.sm_stride_b + j);
    uint16_t* mp = static_cast<uint16_t*>(a.mins) + (packed ? orow : b * a.sm_stride_b + j);
    if (packed && j >= len) {
      for (int k = lane_in_row; k < a.d; k += LPR) crow[k] = 0;
      if (lane_in_row == 0) {
        *sp = 0;
        *mp = 0;
      }
      continue;
    }

    const char* srow = static_cast<const char*>(a.src) + (b * a.s_stride_b + j * a.s_stride_l) * a.esz;
    float x[CPL][8];
    float lo = INFINITY, hi = -INFINITY;
#pragma unroll
    for (int cc = 0; cc < CPL; ++cc) {
      const int k0 = (cc * LPR + lane_in_row) * 8;
      load8<SRC>(srow, k0, a.d, a.vec != 0, x[cc]);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (k0 + i < a.d) {  // NaN-propagating, as torch.aminmax
          lo = __builtin_elementwise_minimum(lo, x[cc][i]);
          hi = __builtin_elementwise_maximum(hi, x[cc][i]);
        }
      }
    }
#pragma unroll
    for (int s = LPR / 2; s >= 1; s >>= 1) {
      lo = __builtin_elementwise_minimum(lo, __shfl_xor(lo, s, LPR));
      hi = __builtin_elementwise_maximum(hi, __shfl_xor(hi, s, LPR));
    }
    float step = (hi - lo) / 255.0f;
    if (step < 1e-8f) step = 1e-8f;  // NaN stays NaN, as torch.clamp_min
#pragma unroll
    for (int cc = 0; cc < CPL; ++cc) {
      const int k0 = (cc * LPR + lane_in_row) * 8;
      if (k0 >= a.d) continue;
      uint32_t w[2] = {0u, 0u};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float v = __builtin_rintf((x[cc][i] - lo) / step);
        v = v < 0.f ? 0.f : (v > 255.f ? 255.f : v);
        w[i >> 2] |= ((uint32_t)v & 0xffu) << (8 * (i & 3));
      }
      if (a.vec && k0 + 8 <= a.d) {
        *reinterpret_cast<u32x2_t*>(crow + k0) = u32x2_t{w[0], w[1]};
      } else {
        for (int i = 0; i < 8 && k0 + i < a.d; ++i) crow[k0 + i] = (uint8_t)(w[i >> 2] >> (8 * (i & 3)));
      }
    }
    if (lane_in_row == 0) {
      *sp = __builtin_bit_cast(uint16_t, (_Float16)step);
      *mp = __builtin_bit_cast(uint16_t, (_Float16)lo);
    }
  }
}

template <int SRC, int LPR, int CPL>
hipError_t launch_q(const QuantArgs& a, hipStream_t s) {
  constexpr int RPB = 256 / LPR;
  const int64_t rows = a.B * ((a.Ld + 3) & ~(int64_t)3);
  int64_t blocks = (rows + RPB - 1) / RPB;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL((quantize_kernel<SRC, LPR, CPL>), dim3((unsigned)blocks), dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int SRC>
hipError_t dispatch_q(const QuantArgs& a, hipStream_t s) {
  const int chunks = (int)((a.d + 7) / 8);
  if (chunks <= 1) return launch_q<SRC, 1, 1>(a, s);
  if (chunks <= 2) return launch_q<SRC, 2, 1>(a, s);
  if (chunks <= 4) return launch_q<SRC, 4, 1>(a, s);
  if (chunks <= 8) return launch_q<SRC, 8, 1>(a, s);
  if (chunks <= 16) return launch_q<SRC, 16, 1>(a, s);
  if (chunks <= 32) return launch_q<SRC, 32, 1>(a, s);
  if (chunks <= 64) return launch_q<SRC, 64, 1>(a, s);
  if (chunks <= 128) return launch_q<SRC, 64, 2>(a, s);
  return launch_q<SRC, 64, 4>(a, s);  // d <= 2048
}

}  // namespace

hipError_t launch_quantize(int src_kind, const QuantArgs& a, hipStream_t s) {
  switch (src_kind) {
    case 0: return dispatch_q<0>(a, s);
    case 1: return dispatch_q<1>(a, s);
    case 2: return dispatch_q<2>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fmx
