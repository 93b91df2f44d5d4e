// Tiled MaxSim forward for many query rows (MFMA-bound regime), d <= 256.
//
// Same contract as _maxsim_fwd_kernel (reference flash_maxsim/flash_maxsim.py:
// 80-146) for single queries with long Lq (config 2: Lq = 1024) and for
// batched scoring (flash_maxsim.py:233-250, config 3), where the reference
// re-streams every doc once per (query, 16..128-token block).
//
// The Nq*Lq query rows are flattened and cut into row blocks of NW waves x
// 16*NB rows. A persistent workgroup of NW waves keeps its row block in
// VGPRs as MFMA B-fragments and walks a fixed set of docs (doc group g: docs
// g, g+G, g+2G, ...). Each doc streams in 64-token tiles: global -> VGPR
// staging -> LDS (double-buffered, rows padded by 16 bytes so the 16 rows of a
// fragment read fall in distinct banks), then every wave reads the A-fragments
// of each 16-token subtile from LDS and runs NB*KS MFMAs against its rows,
// folding the results into per-row running maxima (+ first index). The next
// tile's global loads are in flight while the current one computes; the tile
// sequence runs across doc boundaries without draining.
// At a doc's last tile the row maxima go to LDS (double-buffered by doc
// parity) and, after the tile barrier, each wave sums the rows of its queries:
// a query inside the row block is written to scores, a query straddling row
// blocks to a partial slot that a second kernel adds in row-block order.
//
// uint8 docs (single queries, reference flash_maxsim_quant.py:60-101) take
// the same path: each chunk of eight codes is dequantised to fp16 (code *
// scale + min, one fp16 rounding, as the reference's kernel dequantises before
// its dot product, flash_maxsim_quant.py:89) while it moves from the staging
// registers to LDS, so the tile in LDS and every step after it are the fp16
// kernel's, and the scores equal the fp16 path's on the dequantised docs.
//
// blockIdx -> (row block, doc group) is XCD-aware when the plan says so: the
// eight XCDs take workgroups round-robin, so all row blocks of doc group g are
// put on XCD g % 8 and read each doc tile through the same L2.
//
// The 16x16x32 MFMA form is used on purpose. The 32x32x16 form retires twice
// the flops per instruction, but its 16-register results have to be folded out
// of accumulation registers, and at the register budget of two waves per SIMD
// a wave can then hold only half the query rows, doubling the LDS reads per
// flop. On random data, where the GPU runs power-limited, this layout measured
// faster (config 2: 182 us, against 218-275 us for 32x32x16 variants).
#include "fmx_kernels.h"
#include "fmx_tile.h"

namespace fmx {
namespace {

constexpr int kTiledNW = 8;                  // waves per workgroup
// Workgroups per CU: one (two waves per SIMD), or two (four waves per SIMD) for
// row blocks of up to 32 rows per wave at d <= 128, whose registers fit 128
// VGPRs: their per-tile work is short next to the waits on their tile loads,
// which a second workgroup hides (Nq = 8 x 32 tokens over 5000 docs 112.6 ->
// 99.7 us, a 200-token query 108.5 -> 94.8 us).
// Four-wave workgroups (NW = 4) run three to a CU (three waves per SIMD, 168
// VGPRs) with 48 or 64 rows per wave at d <= 128: 192- and 256-row blocks
// with twelve waves per CU where an eight-wave workgroup has eight (Nq = 8 x
// 32 over 5000 docs 100.1 -> 92.7 us, Nq = 16 x 32 171.1 -> 163.9 us), and
// with 16 or 32 rows per wave for blocks of at most 128 rows (tiled_fwd_plan).
constexpr int tiled_wpc(int nw, int nb, int ks) { return nw == 4 ? 3 : (ks == 4 && nb <= 2) ? 2 : 1; }
// waves per SIMD: a CU holds wpc workgroups of nw waves over its four SIMDs
constexpr int tiled_waves_per_simd(int nw, int nb, int ks) { return tiled_wpc(nw, nb, ks) * nw / 4; }
constexpr int kTileTokens = 64;

// A-fragments of 16-token subtile s from an LDS tile with ROWB-byte rows.
// SWZ: the 16-byte chunk of column j of row r sits at chunk position
// j ^ (r % 16) (rows unpadded; the 16 rows of a fragment read fall in distinct
// banks); otherwise at position j of a row padded by 16 bytes.
template <int KS, int ROWB, bool SWZ>
__device__ __forceinline__ void read_frags(u32x4_t (&af)[KS], const unsigned char* base, int s, int c, int g) {
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) {
    const int j = kk * 4 + g;
    af[kk] = *reinterpret_cast<const u32x4_t*>(base + (s * 16 + c) * ROWB + (SWZ ? (j ^ c) : j) * 16);
  }
}

// The same for a doc's partial last tile: rows past `last` (the tile's last
// row inside the doc) read row `last` again. Their scores repeat that row's,
// which leaves a running maximum unchanged, so the fold needs no mask.
template <int KS, int ROWB, bool SWZ>
__device__ __forceinline__ void read_frags_upto(u32x4_t (&af)[KS], const unsigned char* base, int s, int last,
                                                int c, int g) {
  const int r = s * 16 + c < last ? s * 16 + c : last;
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) {
    const int j = kk * 4 + g;
    af[kk] = *reinterpret_cast<const u32x4_t*>(base + r * ROWB + (SWZ ? (j ^ (r & 15)) : j) * 16);
  }
}

// S for one subtile against every query block of the wave; k-step outer so the
// NB accumulation chains are independent and issue back to back.
template <bool BF, int NB, int KS>
__device__ __forceinline__ void subtile_mfma(const u32x4_t (&af)[KS], const u32x4_t (&qf)[NB][KS],
                                             f32x4_t (&acc)[NB]) {
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) acc[nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] = mfma16x16x32<BF>(af[kk], qf[nb][kk], acc[nb]);
  }
}

// Running max (and first index) of one result fragment: rows rowj .. rowj+3.
template <bool ARGMAX>
__device__ __forceinline__ void fold_rows(f32x4_t acc, int rowj, int len, bool tail, float& m, int& mi) {
  if (tail) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (rowj + i >= len) acc[i] = -INFINITY;
  }
  if constexpr (ARGMAX) {
#pragma unroll
    for (int i = 0; i < 4; ++i) argmax_fold(acc[i], rowj + i, m, mi);
  } else {
    m = fold_max4(m, acc[0], acc[1], acc[2], acc[3]);
  }
}

// uint8 docs: a chunk of eight codes in registers with the fp16 bits of its
// token's scale (low half) and min (high half); a thread's chunks share one
// token, whose scale and min only its chunk 0 holds.
struct U8Chunk {
  u32x2_t codes;
  uint32_t sm;
};

// Buffer resources of the doc a tile comes from: token rows, and for uint8
// docs the doc's scales and mins (else copies of d, unused).
struct TileRes {
  rsrc_t d, s, m;
};

// Eight uint8 codes dequantised to fp16 as the reference's int8 kernel does
// before its dot product (flash_maxsim_quant.py:89, code * scale + min in
// fp16): code c is exact as fp16 (1024 + c, less 1024), then one fp16 fma
// rounds c * scale + min once.
__device__ __forceinline__ u32x4_t dequant8_f16(u32x2_t codes, uint32_t sm) {
  return dequant_biased_f16(codes_to_f16_biased(codes), sm, sm >> 16);
}

// Workgroup barrier once this wave's LDS accesses have completed, without
// the workgroup fence of __syncthreads(), which also waits for every vector
// memory load in flight (vmcnt(0)). The empty asm statements keep the
// compiler from moving memory accesses across it.
__device__ __forceinline__ void barrier_lds() {
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt and expcnt unconstrained
  __builtin_amdgcn_s_barrier();
  __asm__ volatile("" ::: "memory");
}

template <int KIND, int NW, int NB, int KS, bool KMASK, bool ARGMAX>
__global__ void __launch_bounds__(NW * 64)
__attribute__((amdgpu_waves_per_eu(tiled_waves_per_simd(NW, NB, KS), tiled_waves_per_simd(NW, NB, KS))))
tiled_fwd_kernel(FwdArgs a, int nRB, int G, int xcd_map) {
  constexpr int TJ = kTileTokens;
  // Scores of exact-width rows (no k masking, no argmax) stream global -> LDS
  // with buffer loads that write LDS directly (16 bytes per lane, one 1 KB run
  // per wave instruction), into a chunk-swizzled layout. Rows with masked k
  // chunks, and the argmax instances (whose registers do not fit the twice
  // unrolled tile loop the DMA path needs), stage through VGPRs into
  // 16-byte-padded rows.
  // The smallest row blocks (16 rows per wave at d <= 128, no argmax) keep
  // PR = 4 tiles in flight in a register ring instead: their tiles compute in
  // a fraction of an HBM round trip, and the per-tile barrier of the DMA path
  // waits for the one tile in flight (Nq = 2 x 32 tokens over 5000 docs:
  // 92.5 -> 82.2 us). From 32 rows per wave on, the VGPR staging and LDS
  // stores cost more than the deeper ring gains (Nq = 8 x 32: +3 %).
  // uint8 docs (single queries, no argmax) always stage through VGPRs, where
  // each chunk of eight codes is dequantised to fp16 on its way to LDS; the
  // MFMA and everything after it are the fp16 kernel's. Their row blocks of
  // up to 32 rows per wave take the register ring too, whose barrier leaves
  // the ring's loads in flight where the plain staging loop's workgroup fence
  // drains them every tile (128-token query over 5000 docs of 77 tokens
  // 28.3 -> 25.7 us, 200 tokens over 2000 docs of 300: 45.3 -> 41.3 us);
  // with 64 rows per wave the ring spills.
  constexpr bool U8 = KIND == KIND_U8;
  static_assert(!(U8 && ARGMAX), "uint8 docs are scored without argmax");
  constexpr int ESZ = KindInfo<KIND>::esz;
  using stage_t = std::conditional_t<U8, U8Chunk, u32x4_t>;
  constexpr bool RING = !ARGMAX && KS == 4 && (NB == 1 || (U8 && NB <= 2));
  constexpr int PR = 4;
  constexpr bool DMA = !KMASK && !ARGMAX && !RING && !U8;
  constexpr int ROWB = 64 * KS + (DMA ? 0 : 16);  // LDS bytes per token row
  constexpr int BUFB = TJ * ROWB;          // LDS bytes per tile buffer
  constexpr int CPR = 4 * KS;              // 16-byte chunks per token row
  constexpr int CPT = TJ * CPR / (NW * 64);  // chunks per thread per tile
  constexpr int R = NW * NB * 16;          // rows per row block
  constexpr bool BF = KindInfo<KIND>::bf;
  static_assert(CPT * NW * 64 == TJ * CPR, "tile must split evenly over the workgroup");
  // Two tile buffers as separate arrays. On the DMA path each is named at
  // compile time in the twice unrolled tile loop: the compiler then sees that
  // a ds_read of one buffer cannot alias the DMA writes in flight to the
  // other, and places no wait for those writes in front of it.
  // The staging path keeps both buffers in one array indexed at run time.
  // DMA3: a third buffer (two tiles in flight) for eight-wave blocks, where
  // the workgroups per CU still fit the CU's 160 KB with it (config 3 900 ->
  // 889 us, config 2 172.7 -> 171.6 us; four-wave blocks of 128 rows lost
  // 2-3 %: their three workgroups per CU already overlap the tile loads).
  constexpr int RMB = 2 * (ARGMAX ? 1 : 4) * NW * NB * 16 * 4;  // bytes of the row-maxima buffers
  constexpr bool DMA3 = DMA && NW == 8 && tiled_wpc(NW, NB, KS) * (3 * BUFB + RMB) <= 160 * 1024;
  __shared__ __attribute__((aligned(16))) unsigned char lds0[DMA ? BUFB : 16];
  __shared__ __attribute__((aligned(16))) unsigned char lds1[DMA ? BUFB : 16];
  __shared__ __attribute__((aligned(16))) unsigned char lds2[DMA3 ? BUFB : 16];
  __shared__ __attribute__((aligned(16))) unsigned char ldsa[DMA ? 16 : 2 * BUFB];
  // Row maxima of a finished doc (double-buffered by doc parity). Scores:
  // the four row groups' maxima of each row side by side (RG = 4), merged by
  // the reader of the row; argmax: merged before they are written (RG = 1).
  constexpr int RG = ARGMAX ? 1 : 4;
  __shared__ __attribute__((aligned(16))) float rowmax[2][RG * R];
  __shared__ int rowidx[ARGMAX ? 2 : 1][ARGMAX ? R : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15, g = lane >> 4;

  int rb, grp;
  if (xcd_map) {
    const int x = blockIdx.x & 7, k = blockIdx.x >> 3;
    rb = k % nRB;
    grp = x + 8 * (k / nRB);
  } else {
    rb = blockIdx.x % nRB;
    grp = blockIdx.x / nRB;
  }
  if (grp >= G || grp >= a.B) return;

  const int64_t rows_total = (int64_t)a.Nq * a.Lq;
  const int64_t row0 = (int64_t)rb * R;
  const int64_t row_end = row0 + R < rows_total ? row0 + R : rows_total;
  const int64_t qfirst = row0 / a.Lq, qlast = (row_end - 1) / a.Lq;  // queries of this row block

  // Partial 8-wide group when d % 8 != 0.
  const int kp = a.d & ~7;
  const bool has_partial = KMASK && (a.d & 7) != 0;

  // ---- this wave's query rows (B operand), loaded once ----
  u32x4_t qf[NB][KS];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int64_t r = row0 + wave * NB * 16 + nb * 16 + c;
    const bool rv = r < rows_total;
    const int64_t qi = rv ? r / a.Lq : 0;
    const int64_t q = rv ? r - qi * a.Lq : 0;
    const uint16_t* qrow = static_cast<const uint16_t*>(a.Q) + qi * a.sq_n + q * a.sq_l;
#pragma unroll
    for (int t = 0; t < KS; ++t) {
      const int k0 = 32 * t + 8 * g;
      u32x4_t v = {0u, 0u, 0u, 0u};
      if (rv && (!KMASK || k0 < a.d)) v = *reinterpret_cast<const u32x4_t*>(qrow + k0);
      if (has_partial && k0 == kp) v &= prefix_mask16(a.d & 7);
      qf[nb][t] = v;
    }
  }

  // ---- tile loader: chunk k of this thread = tid + k*512 -> (row, 16-byte column) ----
  const uint32_t rowb = (uint32_t)(a.sd_l * ESZ);
  auto tile_rsrc = [&](int b, int len) {
    int64_t rows = len;
    const char* base = static_cast<const char*>(a.D);
    int64_t sm0 = 0;  // uint8: first scale / min of the doc
    if (a.tok_group) {  // packed docs: clamp to the rows of D
      const int64_t t0 = 4 * ld_uniform(a.tok_group + b);
      const int64_t avail = t0 < 0 ? 0 : (a.tok_rows > t0 ? a.tok_rows - t0 : 0);
      if (rows > avail) rows = avail;
      if (avail > 0) {
        base += t0 * a.sd_l * ESZ;
        sm0 = t0;
      }
    } else {
      base += doc_elem0(a, b) * ESZ;
      sm0 = (int64_t)b * a.sm_b;
    }
    TileRes r;
    r.d = make_rsrc(base, (uint32_t)rows * rowb);
    if constexpr (U8) {
      r.s = make_rsrc(a.scales + sm0, (uint32_t)rows * 2u);
      r.m = make_rsrc(a.mins + sm0, (uint32_t)rows * 2u);
    } else {
      r.s = r.d;
      r.m = r.d;
    }
    return r;
  };
  auto doc_len = [&](int b) {
    int l = a.lengths ? ld_uniform(a.lengths + b) : a.Ld;
    return l < 0 ? 0 : (l > a.Ld ? a.Ld : l);
  };
  stage_t stage[CPT];
  // Chunk k of this thread. fp16/bf16: chunks tid + k * (threads), so each
  // load instruction of a wave covers 1 KB of consecutive chunks. uint8: the
  // thread's CPT chunks are adjacent in one token row (CPR % CPT == 0), so it
  // loads that row's scale and min once per tile instead of once per chunk
  // (a wave still reads whole rows: 8 rows x 128 bytes at d = 128).
  static_assert(!U8 || CPR % CPT == 0, "a uint8 thread's chunks share one token row");
  auto chunk_of = [&](int k) __attribute__((always_inline)) { return U8 ? tid * CPT + k : tid + k * NW * 64; };
  auto load_tile_regs = [&](stage_t (&dst)[CPT], const TileRes& rd, int t) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int chunk = chunk_of(k);
      const int row = chunk / CPR, cc = chunk - (chunk / CPR) * CPR;
      const int e0 = cc * 8;
      uint32_t off = (uint32_t)(t * TJ + row) * rowb + (uint32_t)(e0 * ESZ);
      if (KMASK && e0 >= a.d) off = kOOB;
      if constexpr (U8) {
        dst[k].codes = ld8(rd.d, off);
        if (k == 0) {  // the row's scale and min, kept with chunk 0
          const uint32_t so = (uint32_t)(t * TJ + row) * 2u;
          dst[0].sm = (uint32_t)ld2(rd.s, so) | ((uint32_t)ld2(rd.m, so) << 16);
        }
      } else {
        dst[k] = ld16(rd.d, off);
      }
    }
  };
  // The partial 8-wide chunk (d % 8 != 0) is masked here, when the loaded
  // value is used anyway, so a load is never waited for right after issue.
  auto store_tile_lds = [&](const stage_t (&src)[CPT], unsigned char* dst) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int chunk = chunk_of(k);
      const int row = chunk / CPR, cc = chunk - (chunk / CPR) * CPR;
      u32x4_t v;
      if constexpr (U8) {
        v = dequant8_f16(src[k].codes, src[0].sm);
      } else {
        v = src[k];
      }
      if (has_partial && cc * 8 == kp) v &= prefix_mask16(a.d & 7);
      *reinterpret_cast<u32x4_t*>(dst + row * ROWB + cc * 16) = v;
    }
  };
  // DMA: instruction k of wave w fills chunk positions (k*NW + w)*64 .. +63 of
  // the buffer; lane l's position holds column (position % CPR) ^ (row % 16).
  auto dma_tile = [&](const TileRes& rd, int t, unsigned char* dst) {
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int slot = (k * NW + wave) * 64 + lane;
      const int row = slot / CPR, pos = slot - (slot / CPR) * CPR;
      const int col = pos ^ (row & 15);
      const uint32_t off = (uint32_t)(t * TJ + row) * rowb + (uint32_t)(col * 16);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rd.d, (__attribute__((address_space(3))) void*)(dst + (k * NW + wave) * 1024), 16, off, 0, 0, 0);
    }
  };
  // Every wave's DMA writes of the next tile are in LDS before the barrier.
  auto dma_wait = [&]() {
    if constexpr (DMA) __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
  };

  float m[NB];
  int mi[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    m[nb] = -INFINITY;
    mi[nb] = 0;
  }

  // ---- doc / tile walk ----
  int b = grp;
  int len = doc_len(b);
  int nt = len > 0 ? (len + TJ - 1) / TJ : 1;  // an empty doc still takes one fully masked tile
  TileRes rd = tile_rsrc(b, len);
  int t = 0, par = 0;

  // Tile t of doc b from the LDS tile at base, folded into the running maxima.
  auto compute_tile = [&](const unsigned char* base) __attribute__((always_inline)) {
    const int j0 = t * TJ;
    if (j0 + TJ <= len) {
      // full tile: branch-free, A-fragments of subtile s+1 read while s computes
      u32x4_t af[2][KS];
      read_frags<KS, ROWB, DMA>(af[0], base, 0, c, g);
#pragma unroll
      for (int s = 0; s < TJ / 16; ++s) {
        if (s + 1 < TJ / 16) read_frags<KS, ROWB, DMA>(af[(s + 1) & 1], base, s + 1, c, g);
        f32x4_t acc[NB];
        subtile_mfma<BF, NB, KS>(af[s & 1], qf, acc);
        const int rowj = j0 + s * 16 + 4 * g;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) fold_rows<ARGMAX>(acc[nb], rowj, len, false, m[nb], mi[nb]);
      }
    } else {
      // a doc's last, partial tile: its ns subtiles (none for an empty doc)
      // with the same one-ahead fragment reads. Rows past len repeat the
      // doc's last row (scores only: no mask in the fold), or are masked
      // (argmax instances). Each subtile's MFMAs and fold sit in one block
      // after its branch.
      // (With the largest row blocks the second fragment buffer does not fit
      // the register budget; those read each subtile's fragments in turn.)
      constexpr int AB = NB * KS <= 20 ? 2 : 1;
      constexpr bool REPEAT = !ARGMAX;
      const int ns = len > j0 ? (len - j0 + 15) >> 4 : 0;
      const int last = len - 1 - j0;
      u32x4_t af[AB][KS];
      auto frags = [&](u32x4_t (&dst)[KS], int s) __attribute__((always_inline)) {
        if constexpr (REPEAT) {
          read_frags_upto<KS, ROWB, DMA>(dst, base, s, last, c, g);
        } else {
          read_frags<KS, ROWB, DMA>(dst, base, s, c, g);
        }
      };
      if (AB == 2 && ns > 0) frags(af[0], 0);
#pragma unroll
      for (int s = 0; s < TJ / 16; ++s) {
        if (s < ns) {
          if (AB == 1) {
            frags(af[0], s);
          } else if (s + 1 < ns) {
            frags(af[(s + 1) % AB], s + 1);
          }
          f32x4_t acc[NB];
          subtile_mfma<BF, NB, KS>(af[s % AB], qf, acc);
          const int rowj = j0 + s * 16 + 4 * g;
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) fold_rows<ARGMAX>(acc[nb], rowj, len, !REPEAT, m[nb], mi[nb]);
        }
      }
    }
  };
  // At a doc's last tile: its row maxima to rowmax[par], running maxima reset.
  // Scores write every lane's group maximum (one conflict-free LDS store per
  // query block, no lane exchanges: the per-doc epilogue runs while no MFMA
  // does, so its instruction count matters).
  auto finish_doc = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int row = wave * NB * 16 + nb * 16 + c;
      if constexpr (ARGMAX) {
        float v = m[nb];
        int ix = mi[nb];
        argmax_over_groups(v, ix);
        if (g == 0) {
          rowmax[par][row] = v;
          rowidx[par][row] = ix;
        }
      } else {
        rowmax[par][4 * row + g] = m[nb];
      }
      m[nb] = -INFINITY;
      mi[nb] = 0;
    }
  };
  // Maximum of row r (block-relative) of rowmax[par].
  auto row_max = [&](int r) __attribute__((always_inline)) -> float {
    if constexpr (ARGMAX) {
      return rowmax[par][r];
    } else {
      const f32x4_t q = *reinterpret_cast<const f32x4_t*>(&rowmax[par][4 * r]);
      return fold_max4(q[0], q[1], q[2], q[3], q[0]);
    }
  };
  // After the barrier that follows finish_doc: per-query sums of doc b over
  // this row block.
  auto doc_sums = [&]() __attribute__((always_inline)) {
    if constexpr (!ARGMAX) {
      const int lq = (int)a.Lq;
      if ((lq & (lq - 1)) == 0 && lq <= 64) {
        // Lq divides 64 and so every row block (a multiple of 64 rows): each
        // 64-row window of the block holds whole queries, summed by one
        // group sum per window. The per-query loop below costs every wave
        // about 50 instructions per query per doc, issued while no MFMA runs;
        // what counts is that instruction count, not the latency of the
        // reads and lane exchanges (config 3, 20 queries per row block, and
        // the four-group row maxima of finish_doc together: -1.6 %; 16
        // queries of 32 tokens over 100-token docs -6.6 %).
        const int nrows = (int)(row_end - row0);
        const int lsh = __builtin_ctz((unsigned)lq);
        for (int w0 = wave * 64; w0 < nrows; w0 += NW * 64) {
          const int r = w0 + lane;
          const bool in = r < nrows;
          const float v = row_max(in ? r : 0);
          const float sum = group_sum(in ? v : 0.f, lq);
          if (in && (lane & (lq - 1)) == 0) {
            const int64_t qi = (row0 + r) >> lsh;
            store_score(a, qi, b, sum);
          }
        }
        par ^= 1;
        return;
      }
    }
    for (int64_t qi = qfirst + wave; qi <= qlast; qi += NW) {
      const int64_t ra = qi * a.Lq > row0 ? qi * a.Lq : row0;
      const int64_t rz = (qi + 1) * a.Lq < row_end ? (qi + 1) * a.Lq : row_end;
      float sum = 0.f;
      for (int64_t r = ra + lane; r < rz; r += 64) {
        sum += row_max((int)(r - row0));
        if constexpr (ARGMAX) a.argmax[(qi * a.B + b) * a.Lq + (r - qi * a.Lq)] = rowidx[par][r - row0];
      }
      sum = wave_sum(sum);
      if (lane == 0) {
        const bool whole = ra == qi * a.Lq && rz == (qi + 1) * a.Lq;
        if (whole) {
          store_score(a, qi, b, sum);
        } else {
          a.partial[(int64_t)rb * a.Nq * a.B + qi * a.B + b] = sum;
        }
      }
    }
    par ^= 1;
  };

  if constexpr (RING) {
    // Register ring: tile j of the walk is loaded into ring slot j % PR, PR
    // tiles ahead of the tile being computed, and written to LDS buffer j % 2
    // one step before it is computed. A prefetch cursor (pb, pt) runs ahead
    // of (b, t); past the end of the walk it loads from an empty range (zeros,
    // no memory access), so every step issues the same loads and the compiler
    // waits for exactly the slot it stores. The barrier skips the workgroup
    // fence of __syncthreads(), whose vmcnt(0) would drain the ring.
    stage_t ring[PR][CPT];
    int pb = b, pt = 0, pnt = nt;
    TileRes prd = rd;
    const rsrc_t z = make_rsrc(a.D, 0u);
    const TileRes nul = {z, z, z};
    auto fetch = [&](stage_t (&dst)[CPT]) __attribute__((always_inline)) {
      const bool have = pb < a.B;
      load_tile_regs(dst, have ? prd : nul, pt);
      if (!have) return;
      if (++pt >= pnt) {
        pb += G;
        pt = 0;
        if (pb < a.B) {
          const int l = doc_len(pb);
          pnt = l > 0 ? (l + TJ - 1) / TJ : 1;
          prd = tile_rsrc(pb, l);
        }
      }
    };
#pragma unroll
    for (int j = 0; j < PR; ++j) fetch(ring[j]);
    store_tile_lds(ring[0], ldsa);
    barrier_lds();
    // Tile i = (the step's slot S) mod PR: compute it from buffer S % 2, load
    // tile i + PR into its slot, store tile i + 1 into the other buffer.
    auto step = [&](auto slot_tag) __attribute__((always_inline)) -> bool {
      constexpr int S = decltype(slot_tag)::value;
      fetch(ring[S]);  // slot S held tile i, stored to LDS by the previous step
      compute_tile(ldsa + (S & 1) * BUFB);
      const bool last = t + 1 >= nt;
      if (last) finish_doc();
      store_tile_lds(ring[(S + 1) % PR], ldsa + ((S + 1) & 1) * BUFB);
      barrier_lds();
      if (last) doc_sums();
      if (last) {
        b += G;
        if (b >= a.B) return false;
        len = doc_len(b);
        nt = len > 0 ? (len + TJ - 1) / TJ : 1;
        t = 0;
      } else {
        ++t;
      }
      return true;
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1 % PR>;
    using S2 = std::integral_constant<int, 2 % PR>;
    using S3 = std::integral_constant<int, 3 % PR>;
    static_assert(PR == 4, "the unrolled walk below names four slots");
    while (step(S0{}) && step(S1{}) && step(S2{}) && step(S3{})) {
    }
  } else if constexpr (DMA3) {
    // Three buffers, two tiles in flight: tile j of the walk lands in buffer
    // j % 3. While tile j computes, tile j + 2's loads go into the buffer tile
    // j - 1 was read from (before the previous barrier), and the barrier
    // waits only for tile j + 1 (vmcnt(CPT): tile j + 2's CPT load
    // instructions may stay in flight). A prefetch cursor (pb, pt) runs two
    // tiles ahead; past the end of the walk it loads from an empty range
    // (zeros into LDS, no memory access), so every step issues the same loads.
    int pb = b, pt = 0, pnt = nt;
    TileRes prd = rd;
    const rsrc_t z = make_rsrc(a.D, 0u);
    auto issue = [&](unsigned char* dst) __attribute__((always_inline)) {
      const bool have = pb < a.B;
      const TileRes r = {have ? prd.d : z, z, z};
      dma_tile(r, have ? pt : 0, dst);
      if (!have) return;
      if (++pt >= pnt) {
        pb += G;
        pt = 0;
        if (pb < a.B) {
          const int l = doc_len(pb);
          pnt = l > 0 ? (l + TJ - 1) / TJ : 1;
          prd = tile_rsrc(pb, l);
        }
      }
    };
    issue(lds0);
    issue(lds1);
    wait_vmem<CPT>();  // tile 0 is in LDS; tile 1 may be in flight
    barrier_lds();
    auto step = [&](unsigned char* const cur, unsigned char* const ahead) __attribute__((always_inline)) -> bool {
      issue(ahead);
      compute_tile(cur);
      const bool last = t + 1 >= nt;
      if (last) finish_doc();
      wait_vmem<CPT>();  // this wave's loads of the next tile are in LDS
      barrier_lds();     // so are every wave's; every wave is done with cur
      if (last) doc_sums();
      if (last) {
        b += G;
        if (b >= a.B) return false;
        len = doc_len(b);
        nt = len > 0 ? (len + TJ - 1) / TJ : 1;
        t = 0;
      } else {
        ++t;
      }
      return true;
    };
    while (step(lds0, lds2) && step(lds1, lds0) && step(lds2, lds1)) {
    }
  } else if constexpr (DMA) {
    dma_tile(rd, 0, lds0);
    dma_wait();
    __syncthreads();
    // One tile: compute from buffer cur while the next tile fills nxt.
    auto step = [&](unsigned char* const cur, unsigned char* const nxt) __attribute__((always_inline)) -> bool {
      int nb_doc = b, nt_tile = t + 1, nlen = len;
      if (nt_tile >= nt) {
        nb_doc = b + G;
        nt_tile = 0;
      }
      const bool has_next = nb_doc < a.B;
      TileRes rd_next = rd;
      if (has_next) {
        if (nb_doc != b) {
          nlen = doc_len(nb_doc);
          rd_next = tile_rsrc(nb_doc, nlen);
        }
        dma_tile(rd_next, nt_tile, nxt);  // nxt was last read before the previous barrier
      }
      compute_tile(cur);
      const bool last = t + 1 >= nt;
      if (last) finish_doc();
      dma_wait();
      __syncthreads();
      if (last) doc_sums();
      if (!has_next) return false;
      if (nb_doc != b) {
        b = nb_doc;
        len = nlen;
        nt = len > 0 ? (len + TJ - 1) / TJ : 1;
        rd = rd_next;
      }
      t = nt_tile;
      return true;
    };
    while (step(lds0, lds1) && step(lds1, lds0)) {
    }
  } else {
    // staging path: the tile loop as a plain loop over a run-time buffer index
    load_tile_regs(stage, rd, 0);
    store_tile_lds(stage, ldsa);
    __syncthreads();
    int buf = 0;
    while (true) {
      int nb_doc = b, nt_tile = t + 1, nlen = len;
      if (nt_tile >= nt) {
        nb_doc = b + G;
        nt_tile = 0;
      }
      const bool has_next = nb_doc < a.B;
      TileRes rd_next = rd;
      if (has_next) {
        if (nb_doc != b) {
          nlen = doc_len(nb_doc);
          rd_next = tile_rsrc(nb_doc, nlen);
        }
        load_tile_regs(stage, rd_next, nt_tile);
      }
      compute_tile(ldsa + buf * BUFB);
      const bool last = t + 1 >= nt;
      if (last) finish_doc();
      if (has_next) store_tile_lds(stage, ldsa + (buf ^ 1) * BUFB);
      __syncthreads();
      if (last) doc_sums();
      if (!has_next) break;
      if (nb_doc != b) {
        b = nb_doc;
        len = nlen;
        nt = len > 0 ? (len + TJ - 1) / TJ : 1;
        rd = rd_next;
      }
      t = nt_tile;
      buf ^= 1;
    }
  }
}

// scores of queries that straddle row blocks: sum of their partial slots in
// row-block order.
__global__ void __launch_bounds__(256) tiled_sum_parts_kernel(FwdArgs a, int R) {
  const int64_t items = (int64_t)a.Nq * a.B;
  const int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= items) return;
  const int64_t qi = item / a.B, b = item - qi * a.B;
  const int64_t rb0 = qi * a.Lq / R, rb1 = ((qi + 1) * a.Lq - 1) / R;
  if (rb0 == rb1) return;  // written directly by its row block
  float s = 0.f;
  for (int64_t rb = rb0; rb <= rb1; ++rb) s += a.partial[rb * items + item];
  store_score(a, qi, b, s);
}

template <int KIND, int NW, int NB, int KS, bool KMASK, bool ARGMAX>
hipError_t launch_one(const FwdArgs& a, const TiledPlan& p, hipStream_t s) {
  hipLaunchKernelGGL((tiled_fwd_kernel<KIND, NW, NB, KS, KMASK, ARGMAX>), dim3((unsigned)p.grid), dim3(NW * 64), 0,
                     s, a, p.nRB, p.G, p.xcd_map);
  if (p.straddle) {
    const int64_t items = (int64_t)a.Nq * a.B;
    hipLaunchKernelGGL(tiled_sum_parts_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, s, a,
                       p.rows_per_block);
  }
  return hipGetLastError();
}

template <int KIND, int NW, int NB, int KS>
hipError_t dispatch_flags(const FwdArgs& a, const TiledPlan& p, bool am, hipStream_t s) {
  const bool kmask = a.d != 32 * KS;
  if constexpr (KIND == KIND_U8) {
    if (am) return hipErrorInvalidValue;
    return kmask ? launch_one<KIND, NW, NB, KS, true, false>(a, p, s) : launch_one<KIND, NW, NB, KS, false, false>(a, p, s);
  } else {
    if (kmask) {
      return am ? launch_one<KIND, NW, NB, KS, true, true>(a, p, s) : launch_one<KIND, NW, NB, KS, true, false>(a, p, s);
    }
    return am ? launch_one<KIND, NW, NB, KS, false, true>(a, p, s) : launch_one<KIND, NW, NB, KS, false, false>(a, p, s);
  }
}

template <int KIND>
hipError_t dispatch(const FwdArgs& a, const TiledPlan& p, bool am, hipStream_t s) {
  if (p.nw == 4) {
    if (p.ks != 4) return hipErrorInvalidValue;
    switch (p.nb) {
      case 4: return dispatch_flags<KIND, 4, 4, 4>(a, p, am, s);
      case 3: return dispatch_flags<KIND, 4, 3, 4>(a, p, am, s);
      case 2: return dispatch_flags<KIND, 4, 2, 4>(a, p, am, s);
      case 1: return dispatch_flags<KIND, 4, 1, 4>(a, p, am, s);
      default: return hipErrorInvalidValue;
    }
  }
  if (p.ks == 4) {
    switch (p.nb) {
      case 8: return dispatch_flags<KIND, kTiledNW, 8, 4>(a, p, am, s);
      case 6: return dispatch_flags<KIND, kTiledNW, 6, 4>(a, p, am, s);
      case 5: return dispatch_flags<KIND, kTiledNW, 5, 4>(a, p, am, s);
      case 4: return dispatch_flags<KIND, kTiledNW, 4, 4>(a, p, am, s);
      case 3: return dispatch_flags<KIND, kTiledNW, 3, 4>(a, p, am, s);
      case 2: return dispatch_flags<KIND, kTiledNW, 2, 4>(a, p, am, s);
      case 1: return dispatch_flags<KIND, kTiledNW, 1, 4>(a, p, am, s);
      default: break;
    }
  } else if (p.ks == 8) {
    switch (p.nb) {
      case 4: return dispatch_flags<KIND, kTiledNW, 4, 8>(a, p, am, s);
      case 3: return dispatch_flags<KIND, kTiledNW, 3, 8>(a, p, am, s);
      case 2: return dispatch_flags<KIND, kTiledNW, 2, 8>(a, p, am, s);
      case 1: return dispatch_flags<KIND, kTiledNW, 1, 8>(a, p, am, s);
      default: break;
    }
  }
  return hipErrorInvalidValue;
}

}  // namespace

// Batched queries over shared docs read each doc once here instead of once per
// query (Nq = 2, Lq = 32: 93 against 103 us; Nq = 4: 96 against 198 us at
// B = 5000, Ld = 300); a single query comes here once it needs more than one
// pass of the streaming kernel (Lq = 200: 108 against 164 us). Below that the
// streaming kernel loads its query tile once per workgroup of one or two
// docs; with eight-wave blocks that load outweighed what the persistent tiled
// workgroups lose elsewhere only over short docs (d <= 128, 5000 docs: 128
// rows over 77-token docs 33.3 -> 25.3 us, at d = 96 45.8 -> 24.8 us; 32 rows
// over 77 tokens stay faster streamed). With four-wave blocks for up to 128
// rows (tiled_fwd_plan) the tiled kernel also takes single queries of 65-128
// rows over docs of up to 512 tokens and of 33-64 rows over docs of up to 160
// (5000 docs: 128 rows over 300 tokens 82.7 ->
// 71.0 us, over 200 tokens 54.1 -> 41.3 us; 96 rows over 300 tokens 79.1 ->
// 69.4 us; 64 rows over 150 tokens 37.7 -> 34.5 us); 33-64 rows over longer
// docs stay streamed (64 rows over 300 tokens 69.2 against 70.4 us, 48 rows
// 64.8 against 70.8, 40 rows over 200 tokens equal).
bool tiled_fwd_applicable(int64_t Nq, int64_t Lq, int64_t Ld, int d) {
  if (d < 1 || d > 256) return false;
  if (Nq > 1 || Lq > 16 * stream_fwd_nqb(1 << 20, d)) return true;
  return d <= 128 && ((Lq > 32 && Ld <= 160) || (Lq > 64 && Ld <= 512));
}

// uint8 docs (single queries): the tiled kernel from 65 query rows over docs
// of up to 128 tokens, and at d <= 128 from 129 rows (several streaming
// passes) over docs of up to 512 tokens. 5000 docs of 77 tokens: 128 rows
// 35.6 -> 31.3 us, 80 rows 33.9 -> 30.4, 256 rows 92.8 -> 42.7, d = 256
// 98.3 -> 90.3; 128 rows over 64/96/128 tokens 29.7 -> 23.3, 35.9 -> 33.1,
// 39.7 -> 37.1 us; 2000 docs of 300 tokens under 200 rows 59.3 -> 49.0 us,
// 301 tokens under 300 rows 85.4 -> 78.4 us, 1000 of 300 under 512 rows
// -20 %. The streaming kernel stays faster for 64 rows over 77 tokens (24.7
// against 29.3 us), 128 rows over 200 tokens (-5 %), 512 rows over 1024
// tokens (-8 %), 128 rows over 300 tokens at d = 256 (67.0 against 104.6 us)
// and any query of up to 64 rows over longer docs.
bool tiled_u8_applicable(int64_t Lq, int64_t Ld, int d) {
  if (d < 1 || d > 256 || Lq <= 64) return false;
  if (Ld <= 128) return true;
  return d <= 128 && Lq > 16 * stream_fwd_nqb(1 << 20, d) && Ld <= 512;
}

bool tiled_fwd_possible(int64_t Nq, int64_t Lq, int d) {
  return d >= 1 && d <= 256 && (Nq > 1 || Lq > 32);
}

// Picks waves per workgroup (NW), rows per wave (NB) and doc groups (G).
// `slots` workgroups run at once (tiled_wpc per CU). The slowest workgroup's
// time is
// about docs-per-group x (rows-per-block + R0): MFMA work per row plus a
// per-doc streaming cost worth R0 = 545 rows (fitted: 256 query rows over
// 5000 docs of 300 tokens take 118, 152, 195 and 231 us with 256-, 512-, 768-
// and 1024-row blocks). NB is thus chosen to cut the flattened query rows into
// nearly full row blocks (3200 rows of config 3: five blocks of 640, where
// 512-row blocks leave a quarter-full seventh and idle CUs), but no smaller
// than the streaming cost makes worthwhile (512 rows: one 512-row block, not
// two of 256). The XCD-aware mapping puts all row blocks of a doc group on one
// XCD (G a multiple of 8, nRB * G / 8 workgroups per XCD), so each doc tile is
// fetched once per XCD L2; without it the row blocks of a doc meet in the
// shared last-level cache instead, which is counted as a few percent of extra
// cost. Workgroups sharing a CU share its MFMA rate, so a row costs wpc times
// as much. A four-wave workgroup issues a doc tile's loads from half as many
// waves, and its per-doc cost is R0 = 700 rows (fitted on 256- to 512-row
// batches over 5000 docs, which it runs 6 % faster, and 300- and 512-row
// queries over 1000 docs, which it runs 4 to 7 % slower).
TiledPlan tiled_fwd_plan(int64_t Nq, int64_t B, int64_t Lq, int d, int cus) {
  TiledPlan best = {};
  const int ks = d <= 128 ? 4 : 8;
  constexpr int kNB = 7;
  const int nbs4[kNB] = {8, 6, 5, 4, 3, 2, 1}, nbs8[kNB] = {4, 3, 2, 1, 1, 1, 1};
  const int* nbs = ks == 4 ? nbs4 : nbs8;
  constexpr double kR0 = 545.0, kR0NW4 = 700.0;
  const int64_t rows = Nq * Lq;
  double best_cost = 0;
  bool have = false;
  for (int i = 0; i < kNB + 2; ++i) {
    // the last two candidates: four-wave workgroups with NB = 4 and 3 (d <= 128)
    const int nw = i < kNB ? kTiledNW : 4;
    if (nw == 4 && ks != 4) continue;
    for (int xcd = 1; xcd >= 0; --xcd) {
      TiledPlan p = {};
      p.ks = ks;
      p.nw = nw;
      p.nb = i < kNB ? nbs[i] : (i == kNB ? 4 : 3);
      p.rows_per_block = nw * 16 * p.nb;
      const int wpc = tiled_wpc(nw, p.nb, ks);
      const int slots = (cus > 0 ? cus : 256) * wpc;
      const int per_xcd = slots / 8;
      p.nRB = (int)((rows + p.rows_per_block - 1) / p.rows_per_block);
      int G;
      if (xcd) {
        if (p.nRB > per_xcd || B < 8) continue;
        G = 8 * (per_xcd / p.nRB);
        if (G > B) G = (int)(B - B % 8);
        p.grid = 8 * p.nRB * (G / 8);
      } else {
        G = slots / p.nRB;
        if (G < 1) G = 1;
        if (G > B) G = (int)B;
        p.grid = p.nRB * G;
      }
      p.xcd_map = xcd;
      p.G = G;
      const double rounds = (double)(((int64_t)p.grid + slots - 1) / slots);
      const double cost = (double)((B + G - 1) / G) * ((double)p.rows_per_block * wpc + (nw == 4 ? kR0NW4 : kR0)) *
                          rounds * (xcd ? 1.0 : 1.04);
      if (!have || cost < best_cost) {
        best = p;
        best_cost = cost;
        have = true;
      }
    }
  }
  // At most 128 query rows in all at d <= 128 (single queries over short
  // docs, a few batched queries): one block of four waves with 16 or 32 rows
  // each, three workgroups per CU, instead of one eight-wave 128-row block
  // per CU pair (5000 docs of 77 tokens: 64 rows 25.9 -> 21.0 us, 48 rows
  // 25.6 -> 20.8, 128 rows 27.9 -> 21.5, 80 rows 27.1 -> 20.3; 20000 docs
  // under 64 rows 88.1 -> 71.4 us; 96 rows over 150 tokens 42.6 -> 32.0 us;
  // 4 x 32 and 2 x 64 rows over 300-token docs 83.3 -> 70.3 and 69.7 us;
  // uint8 -5 %). The cost model above fits larger blocks and does not see
  // the empty rows of a part-filled one.
  if (rows <= 128 && ks == 4) {
    best = TiledPlan{};
    best.ks = 4;
    best.nw = 4;
    best.nb = rows <= 64 ? 1 : 2;
    best.rows_per_block = 64 * best.nb;
    best.nRB = 1;
    const int slots = (cus > 0 ? cus : 256) * tiled_wpc(4, 1, 4);
    int G = 8 * (slots / 8);
    if (G > B) G = (int)(B - B % 8);
    if (G >= 8) {
      best.xcd_map = 1;
    } else {
      G = (int)B;
      best.xcd_map = 0;
    }
    best.G = G;
    best.grid = G;
  }
  // queries straddling row blocks need the partial-sum pass
  best.straddle = 0;
  for (int64_t qi = 0; qi < Nq && !best.straddle; ++qi) {
    if ((qi * Lq) / best.rows_per_block != ((qi + 1) * Lq - 1) / best.rows_per_block) best.straddle = 1;
  }
  return best;
}

size_t tiled_fwd_workspace_bytes(const TiledPlan& p, int64_t Nq, int64_t B) {
  return p.straddle ? (size_t)p.nRB * (size_t)Nq * (size_t)B * sizeof(float) : 0;
}

hipError_t launch_tiled_fwd(int kind, const FwdArgs& a, const TiledPlan& p, bool with_argmax, hipStream_t s) {
  switch (kind) {
    case KIND_F16: return dispatch<KIND_F16>(a, p, with_argmax, s);
    case KIND_BF16: return dispatch<KIND_BF16>(a, p, with_argmax, s);
    case KIND_U8: return dispatch<KIND_U8>(a, p, with_argmax, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fmx
