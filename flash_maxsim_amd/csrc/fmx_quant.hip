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
// scales and mins are bit-identical to the torch formula. The quotient
// (x - lo) / step is the correctly rounded one, computed per element from the
// row's correctly rounded reciprocal by Markstein's correction (see div_rn).
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
// NT: the 16-byte loads are non-temporal, for fp16/bf16 rows of 64 elements
// or more, where every load instruction of a wave covers whole 128-byte lines
// and the source is read once (config 4's docs 389 -> 385 us); the
// non-temporal policy costs where an instruction covers half lines.
template <int SRC, bool NT>
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
      const u32x4_t* p = reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(row) + k0);
      const u32x4_t v = NT ? __builtin_nontemporal_load(p) : *p;
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

// fp16 sources keep their loaded halves packed: the row scan runs on pairs
// and the subtraction x - lo reads each half directly, so no fp32 copy of the
// row is formed (one conversion per element fewer).
// Packed NaN-propagating minimum / maximum of three fp16 pairs (as the fp32
// minimum and maximum: NaN wins, -0 < +0).
__device__ __forceinline__ uint32_t pk_min3(uint32_t a, uint32_t b, uint32_t c) {
  uint32_t r;
  asm("v_pk_minimum3_f16 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ __forceinline__ uint32_t pk_max3(uint32_t a, uint32_t b, uint32_t c) {
  uint32_t r;
  asm("v_pk_maximum3_f16 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
// Minimum (maximum) over the eight halves of w, as fp32: three packed steps
// (the last pairs each half with the other) and one conversion.
__device__ __forceinline__ float min8_f16(const uint32_t (&w)[4]) {
  uint32_t m = pk_min3(w[0], w[1], w[2]);
  m = pk_min3(m, w[3], w[3]);
  uint32_t r;
  asm("v_pk_minimum3_f16 %0, %1, %1, %1 op_sel:[0,1,0] op_sel_hi:[1,0,1]" : "=v"(r) : "v"(m));
  return half_bits_to_float(r & 0xffffu);
}
__device__ __forceinline__ float max8_f16(const uint32_t (&w)[4]) {
  uint32_t m = pk_max3(w[0], w[1], w[2]);
  m = pk_max3(m, w[3], w[3]);
  uint32_t r;
  asm("v_pk_maximum3_f16 %0, %1, %1, %1 op_sel:[0,1,0] op_sel_hi:[1,0,1]" : "=v"(r) : "v"(m));
  return half_bits_to_float(r & 0xffffu);
}
// RN(x - lo) for the fp16 value in half H of w, x widened exactly inside a
// mixed-precision fma (x * 1 + (-lo), one rounding): the same fp32 value as
// converting x and subtracting.
template <int H>
__device__ __forceinline__ float sub_f16(uint32_t w, float nlo) {
  float r;
  if constexpr (H == 0) {
    asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(nlo));
  } else {
    asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(nlo));
  }
  return r;
}
// Eight fp16 elements k0..k0+7 of a row as four packed words; halves at or
// past d repeat element k0 (k0 < d), which leaves the row's min and max as
// they are.
template <bool NT>
__device__ __forceinline__ void load8_f16(const void* row, int k0, int d, bool vec, uint32_t (&w)[4]) {
  const uint16_t* r = static_cast<const uint16_t*>(row);
  if (vec && k0 + 8 <= d) {
    const u32x4_t* p = reinterpret_cast<const u32x4_t*>(r + k0);
    const u32x4_t v = NT ? __builtin_nontemporal_load(p) : *p;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = v[i];
  } else if (k0 < d) {
    const uint32_t first = r[k0];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = k0 + 2 * i < d ? (uint32_t)r[k0 + 2 * i] : first;
      const uint32_t hi = k0 + 2 * i + 1 < d ? (uint32_t)r[k0 + 2 * i + 1] : first;
      w[i] = lo | (hi << 16);
    }
  }
}

// Correctly rounded a / b from y = RN(1 / b). q0 = RN(a * y) can be 2 ulp
// off (y and the product each round by up to 2^-24 relative); one fma
// correction, q1 = RN(q0 + RN(a - b*q0) * y), brings it within 1 ulp, after
// which the remainder a - b*q1 is exact as an fma and RN(q1 + rem * y) is the
// correctly rounded quotient (Markstein's theorem; Handbook of Floating-Point
// Arithmetic, 2nd ed., sec. 4.7), provided nothing under- or overflows. Here
// b >= 1e-8 and a = x - lo is 0 or >= 2^-24 for fp16 sources (a nonzero
// difference of two fp16 values is a multiple of 2^-24); bf16/fp32 sources can
// produce tiny nonzero a, and numerators below 2^-64 (where a remainder could
// leave the normal range) and NaN take the IEEE division (TINY_OK = false).
template <bool TINY_OK>
__device__ __forceinline__ float div_rn(float a, float b, float y) {
  if constexpr (!TINY_OK) {
    if (!(a >= 0x1p-64f) && a != 0.f) return a / b;
  }
  const float q0 = a * y;
  const float q1 = __builtin_fmaf(__builtin_fmaf(-q0, b, a), y, q0);
  const float rem = __builtin_fmaf(-q1, b, a);
  return __builtin_fmaf(rem, y, q1);
}

// Byte `sel` of `into` replaced by q rounded half to even and clamped to
// [0, 255], NaN giving 0: torch's round() then clamp(0, 255) and the uint8
// cast in one v_cvt_pk_u8_f32 (in the default round-to-nearest-even mode, the
// conversion saturates and sends NaN to 0; checked on gfx950 against rint and
// clamp over every half-integer from 0.5 to 256.5 and its two neighbours,
// -4 .. 300 in steps of 1/8, +-inf, +-0 and NaN; the quantiser's bit-exact
// tests cover quotients on and next to half-integers).
__device__ __forceinline__ uint32_t cvt_u8_rne(float q, int sel, uint32_t into) {
  return __builtin_amdgcn_cvt_pk_u8_f32(q, sel, into);
}

template <bool MAX>
__device__ __forceinline__ float mm(float a, float b) {  // NaN-propagating, as torch.aminmax
  return MAX ? __builtin_elementwise_maximum(a, b) : __builtin_elementwise_minimum(a, b);
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

// Min or max over each aligned group of LPR lanes, left in every lane of the
// group: quad permutes (lane ^ 1, lane ^ 2), then the half-row and row mirrors
// pair quads and half-rows; groups wider than a 16-lane row use shuffles.
template <int LPR, bool MAX>
__device__ __forceinline__ float group_reduce(float v) {
  if constexpr (LPR >= 2) v = mm<MAX>(v, dpp<0xB1>(v));   // quad_perm(1, 0, 3, 2)
  if constexpr (LPR >= 4) v = mm<MAX>(v, dpp<0x4E>(v));   // quad_perm(2, 3, 0, 1)
  if constexpr (LPR >= 8) v = mm<MAX>(v, dpp<0x141>(v));  // row_half_mirror
  if constexpr (LPR >= 16) v = mm<MAX>(v, dpp<0x140>(v)); // row_mirror
  if constexpr (LPR >= 32) v = mm<MAX>(v, __shfl_xor(v, 16));
  if constexpr (LPR >= 64) v = mm<MAX>(v, __shfl_xor(v, 32));
  return v;
}

// Each LPR-lane group takes R consecutive token rows per step and issues all
// their loads before reducing any of them, so R rows of source are in flight
// per group instead of one.
template <int SRC, int LPR, int CPL, int R>
__global__ void __launch_bounds__(256) quantize_kernel(QuantArgs a) {
  constexpr int GPB = 256 / LPR;  // lane groups per block
  const int lane_in_row = threadIdx.x % LPR;
  const int64_t Ld4 = (a.Ld + 3) & ~(int64_t)3;
  const bool packed = a.tok_group != nullptr;
  // blockIdx.x: a chunk of GPB * R token rows of one doc; blockIdx.y (strided): docs.
  const int64_t jbase = ((int64_t)blockIdx.x * GPB + threadIdx.x / LPR) * R;
  if (jbase >= Ld4) return;
  for (int64_t b = blockIdx.y; b < a.B; b += gridDim.y) {
    int64_t len = a.Ld;
    if (a.lengths && packed) {  // the padded layout quantises every token
      len = a.lengths[b];
      len = len < 0 ? 0 : (len > a.Ld ? a.Ld : len);
    }
    // Padded layout: every real token row. Packed: the first len tokens, plus
    // zero rows up to the next multiple of 4.
    const int64_t jend = packed ? ((len + 3) & ~(int64_t)3) : a.Ld;
    const int64_t obase = packed ? 4 * a.tok_group[b] : b * a.Ld;
    constexpr bool PK = SRC == 0;  // packed fp16 halves (above)
    float x[PK ? 1 : R][CPL][8];
    uint32_t xh[PK ? R : 1][CPL][4];
#pragma unroll
    for (int k = 0; k < R; ++k) {
      const int64_t j = jbase + k;
      if (j < jend && j < len) {
        const char* src = static_cast<const char*>(a.src) + (b * a.s_stride_b + j * a.s_stride_l) * a.esz;
#pragma unroll
        for (int cc = 0; cc < CPL; ++cc) {
          if constexpr (PK)
            load8_f16<(LPR >= 8)>(src, (cc * LPR + lane_in_row) * 8, a.d, a.vec != 0, xh[k][cc]);
          else
            load8<SRC, (SRC != 2 && LPR >= 8)>(src, (cc * LPR + lane_in_row) * 8, a.d, a.vec != 0, x[k][cc]);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < R; ++k) {
      const int64_t j = jbase + k;
      const int64_t orow = obase + j;
      int mode = j >= jend ? 0 : (j >= len ? 1 : 2);  // none / packed zero row / quantise
      if (packed && (orow < 0 || orow >= a.tok_rows)) mode = 0;  // outside the output: skipped
      uint8_t* crow = a.codes + orow * a.c_stride_l;
      const int64_t smi = packed ? orow : b * a.sm_stride_b + j;
      uint16_t* sp = static_cast<uint16_t*>(a.scales) + smi;
      uint16_t* mp = static_cast<uint16_t*>(a.mins) + smi;
      if (mode == 0) continue;
      if (mode == 1) {
        for (int kk = lane_in_row; kk < a.d; kk += LPR) crow[kk] = 0;
        if (lane_in_row == 0) {
          *sp = 0;
          *mp = 0;
        }
        continue;
      }
      float lo = INFINITY, hi = -INFINITY;
#pragma unroll
      for (int cc = 0; cc < CPL; ++cc) {
        const int k0 = (cc * LPR + lane_in_row) * 8;
        if constexpr (PK) {
          if (k0 < a.d) {
            lo = mm<false>(lo, min8_f16(xh[k][cc]));
            hi = mm<true>(hi, max8_f16(xh[k][cc]));
          }
        } else if (k0 + 8 <= a.d) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            lo = mm<false>(lo, x[k][cc][i]);
            hi = mm<true>(hi, x[k][cc][i]);
          }
        } else {
          for (int i = 0; i < 8 && k0 + i < a.d; ++i) {  // the row's last, partial chunk
            lo = mm<false>(lo, x[k][cc][i]);
            hi = mm<true>(hi, x[k][cc][i]);
          }
        }
      }
      lo = group_reduce<LPR, false>(lo);
      hi = group_reduce<LPR, true>(hi);
      float step = (hi - lo) / 255.0f;
      if (step < 1e-8f) step = 1e-8f;  // NaN stays NaN, as torch.clamp_min
      const float rstep = 1.0f / step;  // correctly rounded
#pragma unroll
      for (int cc = 0; cc < CPL; ++cc) {
        const int k0 = (cc * LPR + lane_in_row) * 8;
        if (k0 >= a.d) continue;
        uint32_t w[2] = {0u, 0u};
        if constexpr (PK) {
          const float nlo = -lo;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float av = (i & 1) ? sub_f16<1>(xh[k][cc][i >> 1], nlo) : sub_f16<0>(xh[k][cc][i >> 1], nlo);
            w[i >> 2] = cvt_u8_rne(div_rn<true>(av, step, rstep), i & 3, w[i >> 2]);
          }
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            w[i >> 2] = cvt_u8_rne(div_rn<SRC == 0>(x[k][cc][i] - lo, step, rstep), i & 3, w[i >> 2]);
          }
        }
        if (a.vec && k0 + 8 <= a.d) {
          // non-temporal: the codes are read by a later scoring call, not by
          // this kernel (config 4's docs: 406.6 -> 400.3 us)
          __builtin_nontemporal_store(u32x2_t{w[0], w[1]}, reinterpret_cast<u32x2_t*>(crow + k0));
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
}

template <int SRC, int LPR, int CPL>
hipError_t launch_q(const QuantArgs& a, hipStream_t s) {
  constexpr int R = CPL == 1 ? 4 : (CPL == 2 ? 2 : 1);  // rows in flight per lane group
  constexpr int RPB = 256 / LPR * R;
  const int64_t Ld4 = (a.Ld + 3) & ~(int64_t)3;
  const int64_t gx = (Ld4 + RPB - 1) / RPB;
  // two docs per workgroup (config 4's docs: 403 -> 394 us; four or more were slower).
  // Rounding the product with the reciprocal and taking the correctly rounded
  // quotient only near half-integers cut the arithmetic, but its registers
  // halved the resident waves (394 -> 490 us).
  const int64_t gy = (a.B + 1) / 2 < 65535 ? (a.B + 1) / 2 : 65535;
  if (gx > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL((quantize_kernel<SRC, LPR, CPL, R>), dim3((unsigned)gx, (unsigned)gy), dim3(256), 0, s, a);
  return hipGetLastError();
}

// Rows wider than 4096 elements: one workgroup per token row, each thread
// taking elements tid, tid + 256, ...: the min and max meet across the
// workgroup, then a second pass over the row (from cache) writes the codes.
// Same arithmetic, element for element, as quantize_kernel.
template <int SRC>
__global__ void __launch_bounds__(256) quantize_wide_kernel(QuantArgs a) {
  __shared__ float wlo[4], whi[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool packed = a.tok_group != nullptr;
  const int64_t j = blockIdx.x;
  for (int64_t b = blockIdx.y; b < a.B; b += gridDim.y) {
    int64_t len = a.Ld;
    if (a.lengths && packed) {
      len = a.lengths[b];
      len = len < 0 ? 0 : (len > a.Ld ? a.Ld : len);
    }
    const int64_t jend = packed ? ((len + 3) & ~(int64_t)3) : a.Ld;
    if (j >= jend) continue;
    const int64_t obase = packed ? 4 * a.tok_group[b] : b * a.Ld;
    const int64_t orow = obase + j;
    if (packed && (orow < 0 || orow >= a.tok_rows)) continue;
    uint8_t* crow = a.codes + orow * a.c_stride_l;
    const int64_t smi = packed ? orow : b * a.sm_stride_b + j;
    uint16_t* sp = static_cast<uint16_t*>(a.scales) + smi;
    uint16_t* mp = static_cast<uint16_t*>(a.mins) + smi;
    if (j >= len) {  // packed: zero rows up to the next multiple of 4
      for (int64_t k = tid; k < a.d; k += 256) crow[k] = 0;
      if (tid == 0) {
        *sp = 0;
        *mp = 0;
      }
      continue;
    }
    const char* src = static_cast<const char*>(a.src) + (b * a.s_stride_b + j * a.s_stride_l) * a.esz;
    float lo = INFINITY, hi = -INFINITY;
    for (int64_t k = tid; k < a.d; k += 256) {
      const float x = src_elem<SRC>(src, k);
      lo = mm<false>(lo, x);
      hi = mm<true>(hi, x);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      lo = mm<false>(lo, __shfl_xor(lo, off));
      hi = mm<true>(hi, __shfl_xor(hi, off));
    }
    if (lane == 0) {
      wlo[wave] = lo;
      whi[wave] = hi;
    }
    __syncthreads();
    lo = mm<false>(mm<false>(wlo[0], wlo[1]), mm<false>(wlo[2], wlo[3]));
    hi = mm<true>(mm<true>(whi[0], whi[1]), mm<true>(whi[2], whi[3]));
    __syncthreads();  // wlo / whi are rewritten for the next doc
    float step = (hi - lo) / 255.0f;
    if (step < 1e-8f) step = 1e-8f;
    const float rstep = 1.0f / step;
    for (int64_t k = tid; k < a.d; k += 256) {
      crow[k] = (uint8_t)cvt_u8_rne(div_rn<SRC == 0>(src_elem<SRC>(src, k) - lo, step, rstep), 0, 0u);
    }
    if (tid == 0) {
      *sp = __builtin_bit_cast(uint16_t, (_Float16)step);
      *mp = __builtin_bit_cast(uint16_t, (_Float16)lo);
    }
  }
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
  if (chunks <= 256) return launch_q<SRC, 64, 4>(a, s);
  if (chunks <= 512) return launch_q<SRC, 64, 8>(a, s);  // d <= 4096
  const int64_t Ld4 = (a.Ld + 3) & ~(int64_t)3;
  const int64_t gy = a.B < 65535 ? a.B : 65535;
  if (Ld4 > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL(quantize_wide_kernel<SRC>, dim3((unsigned)Ld4, (unsigned)gy), dim3(256), 0, s, a);
  return hipGetLastError();
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
