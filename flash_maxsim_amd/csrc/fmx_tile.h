// Doc-tile staging shared by the streaming and split-d forward kernels.
//
// A tile is 16 consecutive doc tokens. Lane (c, g) loads token row
// tile*16 + c at the k offsets of its fragment slots (A-operand layout), plus,
// for uint8 docs, the fp16 scale and min of tokens tile*16 + 4g .. +3 (the rows
// it owns in the MFMA result layout). Tokens at or past the doc length, and
// k >= d, come back as zeros from the buffer range check.
//
// Fragment slot t of lane group g covers k = frag_k0(t, g) .. +7:
//  * fp16/bf16: 32t + 8g, one 16-byte load per slot;
//  * uint8: slots are paired, 64*(t/2) + 16g + 8*(t%2), so one 16-byte load of
//    16 codes feeds slots t and t+1 and a wave's load instruction covers 64
//    contiguous bytes of each of 16 rows (KS is even for uint8 docs).
// The query operand is loaded with the same k order, so Q * D^T is unchanged.
#pragma once

#include <type_traits>

#include "fmx_device.h"
#include "fmx_kernels.h"

namespace fmx {

template <int KIND>
__device__ __forceinline__ int frag_k0(int t, int g) {
  if constexpr (KIND == KIND_U8) {
    return 64 * (t >> 1) + 16 * g + 8 * (t & 1);
  } else {
    return 32 * t + 8 * g;
  }
}

// Fragment slot (t, g) whose 8 k values start at k (k a multiple of 8).
template <int KIND>
__device__ __forceinline__ void frag_slot(int k, int& t, int& g) {
  if constexpr (KIND == KIND_U8) {
    t = 2 * (k >> 6) + ((k >> 3) & 1);
    g = (k >> 4) & 3;
  } else {
    t = k >> 5;
    g = (k >> 3) & 3;
  }
}

template <int KIND, int KS>
struct Tile {
  static constexpr bool kU8 = KIND == KIND_U8;
  static_assert(!kU8 || KS % 2 == 0, "uint8 tiles pair their k-steps");
  u32x4_t v[kU8 ? KS / 2 : KS];
  u32x2_t s, m;  // uint8 docs only: fp16 bits of 4 consecutive tokens
};

// Buffer resources of one doc row of the document operand.
struct DocRes {
  rsrc_t d;       // token rows, num_records = len * row bytes
  rsrc_t s, m;    // uint8 docs: scales / mins of the doc
  uint32_t rowb;  // bytes per token row
  uint32_t ss, sm;  // uint8 docs without VEC: byte offset (0 or 2) of the doc's first
                    // scale / min in s / m, whose bases are rounded down to 4 bytes
};

// tok_group[drow], taken as wave-uniform (drow is): the buffer resources built
// from it must sit in scalar registers. A kernel that also stores to memory
// in the same loop gets a vector load here, whose result the compiler would
// otherwise treat as varying per lane (and wrap every load in a per-lane loop).
__device__ __forceinline__ int64_t tok_group_of(const FwdArgs& a, int64_t drow) {
  const int64_t v = a.tok_group[drow];
  return (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(v >> 32)) << 32) |
                   (uint32_t)__builtin_amdgcn_readfirstlane((int)v));
}

// scores[qi, column of doc b]: b itself, or doc_ids[b] for packed docs laid
// out in another order than they are numbered (an id outside [0, B) is not
// written).
__device__ __forceinline__ void store_score(const FwdArgs& a, int64_t qi, int64_t b, float v) {
  int64_t col = b;
  if (a.doc_ids) {
    const int32_t id = a.doc_ids[b];
    if ((uint32_t)id >= (uint32_t)a.B) return;
    col = id;
  }
  a.scores[qi * a.ss_n + col * a.ss_b] = v;
}

// First element of doc row `drow` of the document operand: drow * sd_b, or
// for packed docs the start of its token group, 4 * tok_group[drow] rows in.
// UNIFORM reads tok_group through tok_group_of (the doc resources below); the
// tiled kernel keeps the plain load (the extra lane reads cost it 2 %).
template <bool UNIFORM = false>
__device__ __forceinline__ int64_t doc_elem0(const FwdArgs& a, int64_t drow) {
  return a.tok_group ? 4 * (UNIFORM ? tok_group_of(a, drow) : a.tok_group[drow]) * a.sd_l : drow * a.sd_b;
}

// VEC (uint8 docs; FwdArgs::vec): code rows are 16-byte aligned and
// scales/mins are read 4 tokens per 8-byte load. Otherwise codes are read 8
// bytes and scales 2 bytes at a time. fp16/bf16 docs always use 16-byte loads.
// Packed docs: the rows a doc's reads may reach are clamped to the rows of D,
// so a start past the end reads zeros instead of memory past the tensor.
template <int KIND, bool VEC>
__device__ __forceinline__ DocRes make_doc_res(const FwdArgs& a, int64_t drow, int len) {
  constexpr int ESZ = KindInfo<KIND>::esz;
  DocRes r;
  r.rowb = (uint32_t)(a.sd_l * ESZ);
  int64_t avail = INT64_MAX;  // token rows from the doc's start to the end of D
  if (a.tok_group) {
    const int64_t t0 = 4 * tok_group_of(a, drow);
    avail = t0 < 0 ? 0 : (a.tok_rows > t0 ? a.tok_rows - t0 : 0);
  }
  const int64_t drows = len < avail ? len : avail;
  r.d = make_rsrc((const char*)a.D + (avail > 0 ? doc_elem0<true>(a, drow) * ESZ : 0), (uint32_t)drows * r.rowb);
  r.ss = 0u;
  r.sm = 0u;
  if constexpr (KIND == KIND_U8) {
    const int64_t sm0 = a.tok_group ? (avail > 0 ? 4 * tok_group_of(a, drow) : 0) : drow * a.sm_b;
    int64_t n = VEC ? (int64_t)((len + 3) & ~3) : (int64_t)len;
    if (n > avail) n = avail;
    if constexpr (VEC) {
      r.s = make_rsrc(a.scales + sm0, (uint32_t)n * 2u);
      r.m = make_rsrc(a.mins + sm0, (uint32_t)n * 2u);
    } else {
      // 2-byte aligned rows: the resources start at the 4-byte boundary at or
      // below the doc's first value and end at the one at or above its last
      // (never a new page: pages are 4-byte multiples), so the aligned 12-byte
      // loads of load_tile stay in range for every valid token.
      const uintptr_t ps = reinterpret_cast<uintptr_t>(a.scales + sm0);
      const uintptr_t pm = reinterpret_cast<uintptr_t>(a.mins + sm0);
      r.ss = (uint32_t)(ps & 3u);
      r.sm = (uint32_t)(pm & 3u);
      r.s = make_rsrc(reinterpret_cast<const void*>(ps & ~(uintptr_t)3), ((uint32_t)n * 2u + r.ss + 3u) & ~3u);
      r.m = make_rsrc(reinterpret_cast<const void*>(pm & ~(uintptr_t)3), ((uint32_t)n * 2u + r.sm + 3u) & ~3u);
    }
  } else {
    r.s = r.d;
    r.m = r.d;
  }
  return r;
}

// SM (uint8): also load the tile's scales and mins (else the caller fills T.s, T.m).
// C16 (uint8 without VEC): code rows are 16-byte aligned, so codes still come
// 16 bytes per load while the scales take the unaligned path.
// ROWSM (uint8): T.s[0] / T.m[0] hold the scale / min of the lane's own token
// row, tile*16 + c (for dequantising its A-fragment), instead of tokens
// tile*16 + 4g .. +3 (its result rows).
template <int KIND, int KS, bool VEC, bool SM = true, bool C16 = VEC, bool ROWSM = false>
__device__ __forceinline__ void load_tile(Tile<KIND, KS>& T, const DocRes& r, int tile, int c, int g,
                                          const uint32_t (&koff)[KS]) {
  const uint32_t base = (uint32_t)(tile * 16 + c) * r.rowb;
  if constexpr (KIND == KIND_U8) {
#pragma unroll
    for (int h = 0; h < KS / 2; ++h) {
      if constexpr (VEC || C16) {
        T.v[h] = ld16(r.d, base + koff[2 * h]);
      } else {
        const u32x2_t lo = ld8(r.d, base + koff[2 * h]);
        const u32x2_t hi = ld8(r.d, base + koff[2 * h + 1]);
        T.v[h] = u32x4_t{lo[0], lo[1], hi[0], hi[1]};
      }
    }
  } else {
#pragma unroll
    for (int t = 0; t < KS; ++t) T.v[t] = ld16(r.d, base + koff[t]);
  }
  if constexpr (KIND == KIND_U8 && SM && ROWSM) {
    const uint32_t o = (uint32_t)(tile * 16 + c) * 2u;
    T.s[0] = ld2(r.s, r.ss + o);
    T.m[0] = ld2(r.m, r.sm + o);
  } else if constexpr (KIND == KIND_U8 && SM) {
    const uint32_t o = (uint32_t)(tile * 16 + 4 * g) * 2u;
    if constexpr (VEC) {
      T.s = ld8(r.s, o);
      T.m = ld8(r.m, o);
    } else {
      // the four values sit r.ss (r.sm) bytes into the 4-byte aligned 12 bytes
      // at o: one load per array and two byte-funnel shifts
      const u32x3_t s3 = ld12(r.s, o), m3 = ld12(r.m, o);
      T.s = u32x2_t{__builtin_amdgcn_alignbyte(s3[1], s3[0], r.ss), __builtin_amdgcn_alignbyte(s3[2], s3[1], r.ss)};
      T.m = u32x2_t{__builtin_amdgcn_alignbyte(m3[1], m3[0], r.sm), __builtin_amdgcn_alignbyte(m3[2], m3[1], r.sm)};
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

// Doc-operand fragment of k-step t as fp16/bf16 bits; uint8 codes come out
// biased (1024 + code, see codes_to_f16_biased).
template <int KIND, int KS>
__device__ __forceinline__ u32x4_t tile_operand(const Tile<KIND, KS>& T, int t) {
  if constexpr (KIND == KIND_U8) {
    const u32x4_t w = T.v[t >> 1];
    return codes_to_f16_biased((t & 1) ? u32x2_t{w[2], w[3]} : u32x2_t{w[0], w[1]});
  } else {
    return T.v[t];
  }
}

// fp32 scale of result row i (0..3) of this lane (uint8 docs).
__device__ __forceinline__ float tile_scale(u32x2_t s, int i) {
  const uint32_t w = s[i >> 1];
  return half_bits_to_float((i & 1) ? (w >> 16) : (w & 0xffffu));
}

// Affine epilogue constants of result row i: with biased codes,
// S = scale * U + (min - 1024 * scale) * sum(Q); returns (scale, min - 1024 * scale).
__device__ __forceinline__ void tile_affine(const u32x2_t& s, const u32x2_t& m, int i, float& sc, float& off) {
  sc = tile_scale(s, i);
  off = fmaf(-kCodeBias, sc, tile_scale(m, i));
}

}  // namespace fmx
