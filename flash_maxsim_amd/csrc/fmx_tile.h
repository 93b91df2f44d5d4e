// Doc-tile staging shared by the streaming and split-d forward kernels.
//
// A tile is 16 consecutive doc tokens. Lane (c, g) loads token row
// tile*16 + c at the k offsets of its fragment slots (A-operand layout), plus,
// for uint8 docs, the fp16 scale and min of tokens tile*16 + 4g .. +3 (the rows
// it owns in the MFMA result layout). Tokens at or past the doc length, and
// k >= d, come back as zeros from the buffer range check.
#pragma once

#include <type_traits>

#include "fmx_device.h"
#include "fmx_kernels.h"

namespace fmx {

template <int KIND, int KS>
struct Tile {
  static constexpr bool kU8 = KIND == KIND_U8;
  typename std::conditional<kU8, u32x2_t, u32x4_t>::type v[KS];
  u32x2_t s, m;  // uint8 docs only: fp16 bits of 4 consecutive tokens
};

// Buffer resources of one doc row of the document operand.
struct DocRes {
  rsrc_t d;       // token rows, num_records = len * row bytes
  rsrc_t s, m;    // uint8 docs: scales / mins of the doc
  uint32_t rowb;  // bytes per token row
  int sm_vec;     // scales/mins are read 4 tokens per 8-byte load
};

template <int KIND>
__device__ __forceinline__ DocRes make_doc_res(const void* D, int64_t drow, int64_t sd_b, int64_t sd_l,
                                               int len, const uint16_t* scales, const uint16_t* mins,
                                               int64_t sm_b, int sm_vec) {
  constexpr int ESZ = KindInfo<KIND>::esz;
  DocRes r;
  r.rowb = (uint32_t)(sd_l * ESZ);
  r.d = make_rsrc((const char*)D + drow * sd_b * ESZ, (uint32_t)len * r.rowb);
  r.sm_vec = sm_vec;
  if constexpr (KIND == KIND_U8) {
    const uint32_t n = sm_vec ? (uint32_t)((len + 3) & ~3) : (uint32_t)len;
    r.s = make_rsrc(scales + drow * sm_b, n * 2u);
    r.m = make_rsrc(mins + drow * sm_b, n * 2u);
  } else {
    r.s = r.d;
    r.m = r.d;
  }
  return r;
}

template <int KIND, int KS>
__device__ __forceinline__ void load_tile(Tile<KIND, KS>& T, const DocRes& r, int tile, int c, int g,
                                          const uint32_t (&koff)[KS]) {
  const uint32_t base = (uint32_t)(tile * 16 + c) * r.rowb;
#pragma unroll
  for (int t = 0; t < KS; ++t) {
    if constexpr (KIND == KIND_U8) {
      T.v[t] = ld8(r.d, base + koff[t]);
    } else {
      T.v[t] = ld16(r.d, base + koff[t]);
    }
  }
  if constexpr (KIND == KIND_U8) {
    const uint32_t o = (uint32_t)(tile * 16 + 4 * g) * 2u;
    if (r.sm_vec) {
      T.s = ld8(r.s, o);
      T.m = ld8(r.m, o);
    } else {
      T.s[0] = (uint32_t)ld2(r.s, o) | ((uint32_t)ld2(r.s, o + 2) << 16);
      T.s[1] = (uint32_t)ld2(r.s, o + 4) | ((uint32_t)ld2(r.s, o + 6) << 16);
      T.m[0] = (uint32_t)ld2(r.m, o) | ((uint32_t)ld2(r.m, o + 2) << 16);
      T.m[1] = (uint32_t)ld2(r.m, o + 4) | ((uint32_t)ld2(r.m, o + 6) << 16);
    }
  }
}

// Byte offset of query token slot `tok` of doc b's pass in the Q buffer
// resource: row tok of Q, or row qidx[b, tok] for sparse scoring. Slots past
// Lq and out-of-range indices map past the resource, so they read as zeros.
__device__ __forceinline__ uint32_t query_row_offset(const FwdArgs& a, int b, int tok) {
  if (tok >= a.Lq) return kOOB;
  int row = tok;
  if (a.qidx) row = a.qidx[(int64_t)b * a.si_b + (int64_t)tok * a.si_k];
  if ((unsigned)row >= (unsigned)a.Lq_rows) return kOOB;
  return (uint32_t)((int64_t)row * a.sq_l * 2);
}

// A-operand fragment of k-step t as fp16/bf16 bits.
template <int KIND, int KS>
__device__ __forceinline__ u32x4_t tile_operand(const Tile<KIND, KS>& T, int t) {
  if constexpr (KIND == KIND_U8) {
    return codes_to_f16(T.v[t]);
  } else {
    return T.v[t];
  }
}

// fp32 scale and min of result row i (0..3) of this lane (uint8 docs).
__device__ __forceinline__ float tile_scale(u32x2_t s, int i) {
  const uint32_t w = s[i >> 1];
  return half_bits_to_float((i & 1) ? (w >> 16) : (w & 0xffffu));
}

}  // namespace fmx
