// Device-side building blocks shared by every flash_maxsim kernel on gfx950
// (CDNA4, wave64): operand vector types, raw buffer resources, the fp16/bf16
// MFMA wrapper, exact uint8 -> fp16 code conversion and wave reductions.
//
// Fragment convention of the 16x16x32 form (v_mfma_f32_16x16x32_{f16,bf16}),
// used by every forward kernel:
//   lane l = 16*g + c   (c = l % 16, g = l / 16)
//   A operand (16 x 32, M x K): lane l holds row c, k = 8*g .. 8*g+7
//   B operand (32 x 16, K x N): lane l holds col c, k = 8*g .. 8*g+7
//   C/D       (16 x 16)       : lane l holds rows 4*g .. 4*g+3 of col c
// A k-step t of a d-wide row therefore covers k = 32*t + 8*g .. +7 for lane l.
// Any permutation of k applied identically to A and B leaves A*B unchanged, so
// both operands are loaded with the same (row, 32*t + 8*g) addressing.
//
// The 32x32x16 form (v_mfma_f32_32x32x16_{f16,bf16}): lane l = 32*g + c
// (c = l % 32, g = l / 32) holds row (A) / column (B) c and 8 k values; result
// register v of lane l is row 8*(v/4) + 4*g + v%4 of column c.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fmx {

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x3_t __attribute__((ext_vector_type(3)));

// Element kinds of the document operand.
enum Kind : int { KIND_F16 = 0, KIND_BF16 = 1, KIND_U8 = 2 };

template <int KIND> struct KindInfo;
template <> struct KindInfo<KIND_F16> { static constexpr int esz = 2; static constexpr bool bf = false; };
template <> struct KindInfo<KIND_BF16> { static constexpr int esz = 2; static constexpr bool bf = true; };
// uint8 codes are widened to fp16 and multiplied against an fp16 query.
template <> struct KindInfo<KIND_U8> { static constexpr int esz = 1; static constexpr bool bf = false; };

// Raw (unswizzled, stride 0) buffer resource. Word 3 = 0x00020000 selects the
// 32-bit data format gfx9-family buffer instructions expect. A load whose byte
// offset is >= num_records returns zeros without touching memory; the kernels
// use that both for the doc-length tail and for k >= d.
constexpr uint32_t kBufWord3 = 0x00020000u;
constexpr uint32_t kOOB = 0x80000000u;  // kernels keep num_records < 2^31

typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           (int)kBufWord3);
}

__device__ __forceinline__ u32x4_t ld16(rsrc_t r, uint32_t voff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0);
}
__device__ __forceinline__ u32x2_t ld8(rsrc_t r, uint32_t voff) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, voff, 0, 0);
}
__device__ __forceinline__ u32x3_t ld12(rsrc_t r, uint32_t voff) {
  return __builtin_amdgcn_raw_buffer_load_b96(r, voff, 0, 0);
}
__device__ __forceinline__ uint32_t ld4(rsrc_t r, uint32_t voff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, 0, 0);
}
__device__ __forceinline__ uint16_t ld2(rsrc_t r, uint32_t voff) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, voff, 0, 0);
}

// LDS DMA: 16 bytes per lane from the buffer straight into LDS, lane l's at
// lds + 16 l (lds is wave-uniform); NT: with the non-temporal cache policy
// (the lines are not kept in the caches), else the default one. It counts on
// vmcnt like any buffer load; this wave's LDS reads see the data once vmcnt
// has dropped past the instruction (wait_vmem below).
template <bool NT>
__device__ __forceinline__ void dma16_lds(rsrc_t r, void* lds, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0,
                                           NT ? 2 : 0);
}

// Waits until at most N vector-memory instructions of this wave are in
// flight (vmcnt(N); the other counters at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmem() {
  static_assert(N >= 0 && N < 64, "vmcnt is six bits");
  __builtin_amdgcn_s_waitcnt(0x0f70 | (N & 15) | ((N >> 4) << 14));
}

// Waits for this wave's LDS (and scalar-memory) operations (lgkmcnt(0)).
__device__ __forceinline__ void wait_lds() { __builtin_amdgcn_s_waitcnt(0xc07f); }

// Wave-uniform read of an input that no kernel of the launch writes, through
// the constant address space: the compiler may then use a scalar load, which
// counts on lgkmcnt. A vector load of it in a kernel that also stores would
// be waited for with a vmcnt that also drains the loads issued before it.
template <typename T>
__device__ __forceinline__ T ld_uniform(const T* p) {
  return *(const __attribute__((address_space(4))) T*)p;
}

// v of lane `src` (0..63), per lane (ds_bpermute: the LDS crossbar, no LDS memory).
__device__ __forceinline__ uint32_t lane_fetch(uint32_t v, int src) {
  return (uint32_t)__builtin_amdgcn_ds_bpermute(src * 4, (int)v);
}

// 16x16x32 MFMA, fp32 accumulate. Operands travel as raw 128-bit registers.
template <bool BF>
__device__ __forceinline__ f32x4_t mfma16x16x32(u32x4_t a, u32x4_t b, f32x4_t c) {
  if constexpr (BF) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
}

// 32x32x16 MFMA, fp32 accumulate.
template <bool BF>
__device__ __forceinline__ f32x16_t mfma32x32x16(u32x4_t a, u32x4_t b, f32x16_t c) {
  if constexpr (BF) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
}

// IEEE maximum (NaN-propagating, as torch.max): v_maximum3_f32 on gfx950, with
// no canonicalisation of MFMA results in front of it.
__device__ __forceinline__ float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// Running max over the four result rows of one MFMA fragment, as a chain of
// two v_maximum3_f32 (m, r0, r1) and (m, r2, r3). IEEE maximum is commutative
// and associative (NaN propagates, -0 < +0), so the result does not depend on
// the fold order; the chain form issues one VALU op fewer than a tree.
__device__ __forceinline__ float fold_max4(float m, float r0, float r1, float r2, float r3) {
  m = vmax(vmax(m, r0), r1);
  return vmax(vmax(m, r2), r3);
}

// Eight uint8 codes -> eight fp16 values 1024 + code, exactly: v_perm places
// code byte c under exponent byte 0x64, which is the fp16 value 1024 + c
// (1024 + c < 2048 fits the 11-bit significand). The uint8 kernels multiply
// these biased values on the MFMA and remove the bias in the per-token affine
// epilogue: Q . (1024 + c) = Q . c + 1024 * sum(Q), so with the stored
// (scale, min) of a token, Q . (scale * c + min) = scale * Q . (1024 + c) +
// (min - 1024 * scale) * sum(Q). Four VALU ops per 8 codes, no fp16 subtract.
__device__ __forceinline__ u32x4_t codes_to_f16_biased(u32x2_t raw) {
  const uint32_t hi = 0x64646464u;
  u32x4_t h;
  h[0] = __builtin_amdgcn_perm(hi, raw[0], 0x04010400u);
  h[1] = __builtin_amdgcn_perm(hi, raw[0], 0x04030402u);
  h[2] = __builtin_amdgcn_perm(hi, raw[1], 0x04010400u);
  h[3] = __builtin_amdgcn_perm(hi, raw[1], 0x04030402u);
  return h;
}

// Bias of codes_to_f16_biased.
constexpr float kCodeBias = 1024.0f;

// Biased codes (codes_to_f16_biased) dequantised to fp16 as the reference's
// int8 kernel dequantises before its dot product (flash_maxsim_quant.py:89):
// code * scale + min rounded once (one v_pk_add_f16 removes the bias exactly,
// one v_pk_fma_f16 rounds). sc_bits / mn_bits: fp16 bits in the low half.
__device__ __forceinline__ u32x4_t dequant_biased_f16(u32x4_t h, uint32_t sc_bits, uint32_t mn_bits) {
  typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
  const h2_t sc = __builtin_bit_cast(h2_t, (sc_bits & 0xffffu) * 0x10001u);
  const h2_t mn = __builtin_bit_cast(h2_t, (mn_bits & 0xffffu) * 0x10001u);
  const h2_t bias = {(_Float16)kCodeBias, (_Float16)kCodeBias};
  u32x4_t o;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // bit_cast a copy: clang casts the first element for a vector subscript
    const uint32_t hi = h[i];
    const h2_t c = __builtin_bit_cast(h2_t, hi) - bias;
    const uint32_t v = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(c, sc, mn));
    o[i] = v;
  }
  return o;
}

__device__ __forceinline__ float half_bits_to_float(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}
__device__ __forceinline__ float bf16_bits_to_float(uint32_t bits16) {
  return __builtin_bit_cast(float, bits16 << 16);
}

// Row sums of a 16-token fp16 query block held as B-fragments qf[0..KS-1]:
// an MFMA against an all-ones A operand puts sum_k Q[c, k] (fp32 accumulate)
// in every result row of column c, so lane (c, g) gets its query token's sum
// in KS matrix instructions instead of 16 VALU ops per fragment.
template <int KS>
__device__ __forceinline__ float query_row_sum(const u32x4_t (&qf)[KS]) {
  const u32x4_t ones = {0x3c003c00u, 0x3c003c00u, 0x3c003c00u, 0x3c003c00u};  // fp16 1.0
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < KS; ++t) acc = mfma16x16x32<false>(ones, qf[t], acc);
  // The four result rows hold the same sum, so their max is that sum exactly.
  // Reading all four right away keeps none of the MFMA's result registers
  // dead: a dead one can be reassigned by the compiler across a branch while
  // the MFMA is still to write it.
  return fold_max4(acc[0], acc[1], acc[2], acc[3], acc[0]);
}

// Mask keeping the first n (0..8) 16-bit elements of an 8-element fragment.
__device__ __forceinline__ u32x4_t prefix_mask16(int n) {
  u32x4_t m;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    m[w] = (2 * w + 2 <= n) ? 0xffffffffu : ((2 * w + 1 <= n) ? 0x0000ffffu : 0u);
  }
  return m;
}

// Cross-row exchanges on the VALU (no LDS round trip, unlike ds_bpermute):
// v_permlane16_swap / v_permlane32_swap of a value with itself leave, in
// every lane l, the value of lane l & ~16 (resp. ~32) in `lo` and that of
// lane l | 16 (resp. | 32) in `hi`. A commutative combine of lo and hi is the
// combine of a lane with its partner l ^ 16 (l ^ 32), bitwise equal in both.
__device__ __forceinline__ void halves16(uint32_t x, uint32_t& lo, uint32_t& hi) {
  const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  lo = r[0];
  hi = r[1];
}
__device__ __forceinline__ void halves32(uint32_t x, uint32_t& lo, uint32_t& hi) {
  const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  lo = r[0];
  hi = r[1];
}
__device__ __forceinline__ void halves16(float x, float& lo, float& hi) {
  uint32_t a, b;
  halves16(__builtin_bit_cast(uint32_t, x), a, b);
  lo = __builtin_bit_cast(float, a);
  hi = __builtin_bit_cast(float, b);
}
__device__ __forceinline__ void halves32(float x, float& lo, float& hi) {
  uint32_t a, b;
  halves32(__builtin_bit_cast(uint32_t, x), a, b);
  lo = __builtin_bit_cast(float, a);
  hi = __builtin_bit_cast(float, b);
}

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

// Sum over the 64 lanes of a full wave, the same bits in every lane: within
// 16-lane rows by DPP (quad xor 1, quad xor 2, half-row mirror, row mirror;
// each step adds a lane to a partner holding the same partial), then across
// rows by the permlane swaps.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_mov<0xB1>(v);   // quad_perm(1, 0, 3, 2)
  v += dpp_mov<0x4E>(v);   // quad_perm(2, 3, 0, 1)
  v += dpp_mov<0x141>(v);  // row_half_mirror
  v += dpp_mov<0x140>(v);  // row_mirror
  float lo, hi;
  halves16(v, lo, hi);
  v = lo + hi;
  halves32(v, lo, hi);
  return lo + hi;
}

// Sum over each aligned group of lq lanes (lq a power of two up to 64, the
// same for the whole wave), in every lane of the group: the first log2(lq)
// steps of wave_sum.
__device__ __forceinline__ float group_sum(float v, int lq) {
  if (lq > 1) v += dpp_mov<0xB1>(v);
  if (lq > 2) v += dpp_mov<0x4E>(v);
  if (lq > 4) v += dpp_mov<0x141>(v);
  if (lq > 8) v += dpp_mov<0x140>(v);
  float lo, hi;
  if (lq > 16) {
    halves16(v, lo, hi);
    v = lo + hi;
  }
  if (lq > 32) {
    halves32(v, lo, hi);
    v = lo + hi;
  }
  return v;
}

// Running max of a lane's value over the four lanes c, c+16, c+32, c+48 (the
// four row groups of an MFMA result column), left in every lane.
__device__ __forceinline__ float max_over_groups(float v) {
  float lo, hi;
  halves16(v, lo, hi);
  v = vmax(lo, hi);
  halves32(v, lo, hi);
  return vmax(lo, hi);
}

// Running (max, first index) over similarities s of increasing index j, with
// torch.max's NaN rule: a NaN is the max and the first NaN keeps it (once m
// is NaN nothing replaces it), otherwise only a strictly larger value moves
// the index. !(s <= m) is true for s > m and for a NaN s.
__device__ __forceinline__ void argmax_fold(float s, int j, float& m, int& mi) {
  if (m == m && !(s <= m)) {
    m = s;
    mi = j;
  }
}

// (value, index) max where ties go to the smaller index and NaN beats every
// number (two NaNs: the smaller index): combining per-lane first-occurrence
// maxima this way yields the global first occurrence of torch.max.
__device__ __forceinline__ void argmax_merge(float& v, int& i, float ov, int oi) {
  const bool vn = v != v, on = ov != ov;
  const bool take = on ? (!vn || oi < i) : (!vn && (ov > v || (ov == v && oi < i)));
  if (take) {
    v = ov;
    i = oi;
  }
}

// argmax_merge over the four row groups (lanes c, c+16, c+32, c+48), merged
// as (group 0 with 1, 2 with 3), then (0-1 with 2-3): the lower group always
// the first operand. Lanes of group 0 hold the result.
__device__ __forceinline__ void argmax_over_groups(float& v, int& ix) {
  float lo, hi;
  uint32_t ilo, ihi;
  halves16(v, lo, hi);
  halves16((uint32_t)ix, ilo, ihi);
  v = lo;
  ix = (int)ilo;
  argmax_merge(v, ix, hi, (int)ihi);
  halves32(v, lo, hi);
  halves32((uint32_t)ix, ilo, ihi);
  v = lo;
  ix = (int)ilo;
  argmax_merge(v, ix, hi, (int)ihi);
}

}  // namespace fmx
