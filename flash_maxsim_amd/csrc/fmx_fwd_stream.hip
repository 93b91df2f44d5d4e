// Streaming MaxSim forward for d <= 256 (the HBM-bound small-query regime).
//
// Replaces the per-(query, doc) Triton program of _maxsim_fwd_kernel
// (reference flash_maxsim/flash_maxsim.py:80-146) and _maxsim_int8_kernel
// (flash_maxsim/flash_maxsim_quant.py:40-98).
//
// One workgroup of four waves scores one (query, doc) pair for one pass of up
// to 16*NQB query tokens:
//  * the pass's query tile (16*NQB tokens x 32*KS dims) sits in VGPRs as MFMA
//    B-fragments for the whole doc; the workgroup loads it once (each wave a
//    quarter of the fragments, exchanged through LDS while the first doc
//    tiles are in flight);
//  * the doc's 16-token tiles are dealt round-robin to the four waves, which
//    load them with 128-bit (fp16/bf16) or 64-bit (uint8) buffer loads straight
//    into VGPRs, P tiles deep, so no LDS round trip sits on the HBM stream;
//  * S = D_tile * Q^T runs on v_mfma_f32_16x16x32 with fp32 accumulation and
//    each lane folds its 4 result rows into a running per-query-token max
//    (plus the first index reaching it, when argmax is requested);
//  * at the end lanes merge across row groups with cross-lane shuffles, waves
//    merge through LDS, and wave 0 sums over query tokens into one fp32 score.
// uint8 docs use S = scale_j * (Q . (1024 + codes_j)) + (min_j - 1024 * scale_j)
// * sum_k Q_k, with the codes widened to the fp16 values 1024 + code exactly
// (one v_perm per two codes); this equals Q . dequantize(codes) up to fp32
// rounding.
// Queries longer than 16*NQB tokens run as blockIdx.y passes whose partial sums
// a second kernel adds in pass order.
// Single uint8 queries of 65-128 tokens over padded docs at d in (64, 128] run
// stream_u8_shared_kernel instead: its four waves share each doc tile through
// LDS and hold 32 query rows each (see there).
#include "fmx_kernels.h"
#include "fmx_tile.h"

namespace fmx {
namespace {

constexpr int kStreamWaves = 4;
// Tiles in flight per wave. Deeper uint8 rings (half the bytes per tile) cost
// the third wave per SIMD, which hides more of the per-tile dequant work than
// the extra bytes in flight gain. fp16/bf16 tiles of 8 k-steps (d > 128) hold
// 8 KB each: two in flight keep two or more waves per SIMD (four cost d = 192
// and d = 256 with 64-token queries a quarter of their speed, at one wave).
// uint8 passes of a full 128-VGPR query tile (128 rows at d <= 128) keep four
// tiles in flight in at most 242 VGPRs, two waves per SIMD (config 4's docs
// under a 128-token query 117 -> 114 us, 5000 docs of 512 tokens 104 -> 102 us
// against two tiles; three measured no better than two).
template <int KIND, int NQB, int KS>
constexpr int stream_depth() {
  return (KIND != KIND_U8 && KS >= 8) ? 2 : 4;
}

// Doc tiles through a per-wave LDS ring (stream_fwd_kernel's DMA path) for
// rows of exactly 128 elements scored without argmax, outside the two-tile
// ring of short doc pairs (PD = 2): fp16/bf16 with two tiles in flight per
// wave (8 KB of LDS each), uint8 with the group scale loads' four (2 KB each).
template <int KIND, int KS, bool KMASK, bool ARGMAX, int PD>
constexpr bool stream_dma_fp() {
  return KIND != KIND_U8 && KS == 4 && !KMASK && !ARGMAX && PD == 0;
}
constexpr int kStreamDmaDepth = 2;
// Docs of this many bytes or more (docs x Ld x d x element size) outgrow the
// 256 MB last-level cache: their LDS ring loads are non-temporal, and uint8
// docs take the LDS ring only from here. Smaller doc sets, scored again by
// the next call, are read with the default policy and stay in that cache.
constexpr int64_t kLlcBytes = (int64_t)1 << 28;

int64_t stream_doc_bytes(const FwdArgs& a, int esz) {
  const int64_t rows = a.tok_group ? a.tok_rows : (int64_t)(a.shared_docs ? 1 : a.Nq) * a.B * a.Ld;
  return rows * a.d * esz;
}

// KMASK: d is not exactly 32*KS, so fragment slots past d must read as zero.
// VEC: uint8 vector load path (FwdArgs::vec); true for fp16/bf16.
// DOCS = 2 (one pass, no argmax; uint8 docs of one query, and fp16/bf16 docs
// of one query or per-query docs, with a full 128-VGPR query tile or of up to
// 256 tokens): the workgroup scores docs 2p and 2p+1 of a query as one tile
// sequence (the first doc's tiles, then the second's),
// so its query tile, row sums and load ring carry over from one doc to the
// next instead of being rebuilt and refilled per doc.
// JOINT (two uint8 docs with aligned rows): one buffer range covers the
// pair's scale rows (padded: adjacent rows; packed: wherever the two token
// groups start), so the group scale loads (below) take one instruction per
// array instead of one per doc.
// Waves per SIMD asked of the compiler: three for the one-doc uint8 instance
// of 64 query rows (batched or sparse queries of 33-64 tokens; 188 VGPRs
// allowed two, and fitting 168 costs one spill: measured as the two passes of
// Lq = 128, 139 -> 125 us). The two-doc instance would spill 9 registers in
// its loop at that budget (75 -> 116 us). Two for the uint8 instances of a
// full 128-VGPR query tile (see stream_depth).
template <int KIND, int NQB, int KS, bool VEC, int DOCS>
constexpr int stream_min_waves() {
  if (KIND == KIND_U8 && VEC && NQB == 4 && KS == 4 && DOCS == 1) return 3;
  return (KIND == KIND_U8 && NQB * KS >= 32) ? 2 : 1;
}

// PD: ring depth other than stream_depth's (0: stream_depth's).
template <int KIND, int NQB, int KS, bool KMASK, bool ARGMAX, bool VEC, int DOCS = 1, bool JOINT = false, int PD = 0,
          bool C16 = VEC, bool U8RING = true, bool NT = true>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(stream_min_waves<KIND, NQB, KS, VEC, DOCS>())))
stream_fwd_kernel(FwdArgs a) {
  // DMA: each wave's ring lives in LDS. A tile's 16 rows of 256 bytes come by
  // LDS DMA loads of whole 128-byte lines (four rows per instruction, 16-byte
  // chunks swizzled by row, chunk j of row r at j ^ r, so the fragment reads
  // spread over all banks) with the nt cache policy (NT), and the MFMA fragments
  // are read from LDS. With whole lines per load instruction the nt policy
  // streams them: config 1 60.8 -> 55.2 us, per-query docs 61.7 -> 56.0 us,
  // Q[128,128] over 1000 docs of 1024 tokens 46.8 -> 44.1 us (a plain read of
  // config 1's docs: 60.1 -> 55.5 us with nt). The VGPR ring's loads follow
  // the MFMA fragment order, which touches each line with two instructions;
  // nt made those 17 % slower. Short doc pairs (the PD = 2 ring) keep VGPR
  // tiles: 5000 docs of 77 tokens 18.3 -> 19.9 us through LDS. uint8 tiles
  // take the same path (below). NT = false: the default cache policy, for doc
  // sets the last-level cache holds (kLlcBytes; the medium row, 262 MB:
  // 44.3 -> 41.9 us).
  constexpr bool DMA_FP = stream_dma_fp<KIND, KS, KMASK, ARGMAX, PD>();
  constexpr int NW = kStreamWaves, P = PD ? PD : (DMA_FP ? kStreamDmaDepth : stream_depth<KIND, NQB, KS>()),
                QROWS = NQB * 16;
  constexpr int ESZ = KindInfo<KIND>::esz;
  constexpr bool BF = KindInfo<KIND>::bf;
  constexpr bool U8 = KIND == KIND_U8;
  static_assert(DOCS == 1 || (DOCS == 2 && !ARGMAX), "two docs per workgroup: scores only");
  // DQ: uint8 instances of eight query blocks (d <= 128, queries of more than
  // 64 tokens) dequantise each tile's codes to fp16 before the MFMAs, as the
  // reference's kernel does (flash_maxsim_quant.py:89), instead of applying
  // the affine map to every result: that costs 2 packed ops per code pair
  // (per k-step) against 2 VALU ops per result row and query block, so it
  // pays where query blocks outnumber k-steps (Q[96,128] over 300-token docs
  // 63.6 -> 59.7 us, 200-token docs -7 %, config 4's docs -2 %; at d = 256
  // with four query blocks it lost 3.6 %).
  constexpr bool DQ = U8 && NQB >= 8;
  // group scale loads (below): the four-tile ring, and the two-tile ring of
  // short doc pairs when one range covers both docs' scales (JOINT)
  constexpr bool GSM = U8 && VEC && !DQ && (P == 4 || (P == 2 && JOINT));
  static_assert(!GSM || P == 4 || P == 2, "group scale loads map 16 lanes per tile slot");
  static_assert(!JOINT || DOCS == 2, "a joint scale range serves two-doc group loads");
  // uint8 DMA tiles: 16 code rows of 128 bytes (two load instructions of 8
  // rows each), chunk j of row r at j ^ (r % 8); the scales and mins keep the
  // group loads into registers.
  // (uint8 queries of up to 32 tokens: config 4 62.2 -> 57.9 us, packed
  // 64.3 -> 58.6 us; 33-64-token queries lost 5-10 % and keep the VGPR ring).
  // U8RING = false keeps the VGPR ring for smaller uint8 workloads, and
  // NT = false takes the default cache policy for smaller fp16/bf16 doc sets
  // (the launch's choices, kLlcBytes).
  constexpr bool DMA = DMA_FP || (U8RING && U8 && NQB <= 2 && KS == 4 && !KMASK && !ARGMAX && PD == 0 && GSM);
  constexpr int RB = U8 ? 128 : 256;       // bytes of a tile row
  constexpr int TB = 16 * RB;              // bytes of a tile
  constexpr int TI = TB / 1024;            // DMA instructions per tile
  constexpr int CPR = RB / 16;             // 16-byte chunks per row
  // vector-memory instructions between two tiles' DMA loads in the steady
  // state besides the tiles': a group's scale and min loads
  constexpr int GL = GSM ? ((JOINT || DOCS == 1) ? 2 : 4) : 0;
  __shared__ __attribute__((aligned(16))) unsigned char dring[DMA ? NW * P * TB : 16];
  __shared__ float red_m[DOCS][NW][QROWS];
  __shared__ int red_i[ARGMAX ? NW : 1][QROWS];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, g = lane >> 4;
  // The passes of one (query, doc) pair are adjacent workgroups, so the doc
  // streams from HBM once and the later passes find it in cache.
  // Workgroups go to the eight XCDs round-robin: x = 8 * (npass * grp + p) + k
  // is pass p of item 8 * grp + k, so all passes of an item share an XCD's L2
  // and start back to back.
  const int npass = (a.Lq + QROWS - 1) / QROWS;
  int xi = blockIdx.x, pass = 0;
  if (DOCS == 1 && npass > 1) {
    const int x = blockIdx.x, k = x & 7, r = x >> 3;
    const int grp = r / npass;
    pass = r - grp * npass;
    xi = 8 * grp + k;
    if (xi >= a.Nq * a.B) return;  // uniform over the workgroup, before any barrier
  }
  int qi, b;
  if constexpr (DOCS == 2) {
    // workgroup xi: docs 2p and 2p + 1 of query qi (per-query docs: that
    // query's own docs, rows qi * B + b); a single query skips the division
    qi = 0;
    b = 2 * xi;
    if (!U8 && a.Nq > 1) {
      const int pairs = (a.B + 1) / 2;
      qi = xi / pairs;
      b = 2 * (xi - qi * pairs);
    }
  } else if (a.shared_docs && a.Nq > 1) {
    // Queries of one doc run back to back so the doc streams from HBM once
    // and the other queries find it in cache.
    b = xi / a.Nq;
    qi = xi - b * a.Nq;
  } else if (a.Nq == 1) {
    qi = 0;  // no integer division (a few dozen instructions) before the first loads
    b = xi;
  } else {
    qi = xi / a.B;
    b = xi - qi * a.B;
  }
  const int item = qi * a.B + b;  // row of argmax / partial, as in the reference
  const int64_t drow = a.shared_docs ? (int64_t)b : (int64_t)item;
  auto doc_length = [&](int64_t row) {
    const int l = a.lengths ? a.lengths[row] : a.Ld;
    return l < 0 ? 0 : (l > a.Ld ? a.Ld : l);
  };
  const int len0 = doc_length(drow);
  const bool two = DOCS == 2 && b + 1 < a.B;  // second doc of the workgroup
  const int len1 = two ? doc_length(drow + 1) : 0;
  const int nt0 = (len0 + 15) >> 4;
  const int ntiles = nt0 + ((len1 + 15) >> 4);  // tile sequence: doc 0's, then doc 1's
  const int my_n = ntiles > wave ? (ntiles - wave + NW - 1) / NW : 0;

  // Partial 8-wide group (d % 8 != 0): fragment slot tp of lane group gp.
  const int kp = a.d & ~7;
  int tp, gp;
  frag_slot<KIND>(kp, tp, gp);
  const u32x4_t pmask = prefix_mask16(g == gp ? (a.d & 7) : 8);
  const bool has_partial = KMASK && (a.d & 7) != 0;

  // ---- query tile of this pass (B operand) ----
  const int q0 = pass * QROWS;
  const rsrc_t rq = make_rsrc((const char*)a.Q + (int64_t)qi * a.sq_n * 2, (uint32_t)(a.Lq_rows * a.sq_l * 2));
  // Each wave loads every NW-th fragment of the query tile; the fragments
  // meet in LDS once the first doc tiles are in flight (q_exchange), so the
  // workgroup issues the query loads once instead of once per wave.
  // QALIAS (fp16 rings): the LDS ring's last slot of every wave holds the
  // fragments during the exchange (its first tile is loaded after it), so the
  // workgroup's LDS is the ring's and four workgroups share a CU instead of
  // three. The uint8 ring keeps its own buffer: at four workgroups per CU its
  // packed-layout stream ran 2 % slower (more concurrent doc streams).
  constexpr int NF = NQB * KS, FPW = (NF + NW - 1) / NW;
  constexpr bool QALIAS = DMA_FP && NF * 1024 <= NW * TB;
  __shared__ u32x4_t qs_own[QALIAS ? 1 : NF][QALIAS ? 1 : 64];
  // fragment f's 64 lanes: in wave (f % NW)'s last ring slot, or in qs_own
  auto qfrag = [&](int f) -> u32x4_t* {
    if constexpr (QALIAS) {
      return reinterpret_cast<u32x4_t*>(dring + (f % NW) * P * TB + (P - 1) * TB + (f / NW) * 1024);
    } else {
      return &qs_own[f][0];
    }
  };
  u32x4_t qv[FPW];
#pragma unroll
  for (int j = 0; j < FPW; ++j) {
    const int f = wave + NW * j;
    qv[j] = u32x4_t{0u, 0u, 0u, 0u};
    if (f < NF) {
      const int nb = f / KS, t = f - (f / KS) * KS;
      const uint32_t rowoff = query_row_offset(a, b, q0 + nb * 16 + c);
      const int k0 = frag_k0<KIND>(t, g);
      if constexpr (KMASK) {
        qv[j] = ld16(rq, k0 < a.d ? rowoff + (uint32_t)(k0 * 2) : kOOB);
        if (has_partial && t == tp) qv[j] &= pmask;
      } else {
        qv[j] = ld16(rq, rowoff + (uint32_t)(k0 * 2));
      }
    }
  }
  u32x4_t qf[NQB][KS];
  float qsum[NQB];
  auto q_exchange = [&]() {
#pragma unroll
    for (int j = 0; j < FPW; ++j) {
      const int f = wave + NW * j;
      if (f < NF) qfrag(f)[lane] = qv[j];
    }
    __syncthreads();
#pragma unroll
    for (int nb = 0; nb < NQB; ++nb) {
#pragma unroll
      for (int t = 0; t < KS; ++t) qf[nb][t] = qfrag(nb * KS + t)[lane];
      qsum[nb] = 0.f;
      if constexpr (U8 && !DQ) {
        qsum[nb] = query_row_sum<KS>(qf[nb]);
      }
    }
  };

  // ---- doc stream ----
  const DocRes dr0 = make_doc_res<KIND, VEC>(a, drow, len0);
  const DocRes dr1 = DOCS == 2 ? make_doc_res<KIND, VEC>(a, two ? drow + 1 : drow, len1) : dr0;
  uint32_t koff[KS];
#pragma unroll
  for (int t = 0; t < KS; ++t) {
    const int k0 = frag_k0<KIND>(t, g);
    // Slots past d read as zeros instead of touching the next row.
    koff[t] = (KMASK && k0 >= a.d) ? kOOB : (uint32_t)(k0 * ESZ);
  }
  // Sequence position -> (doc, tile of that doc); uniform over the wave.
  // Positions past the sequence read an empty range (zeros, no memory access).
  constexpr bool FIXED = !ARGMAX;  // fixed refill pattern (below)
  const rsrc_t nul = make_rsrc(a.D, 0u);
  unsigned char* const myring = dring + (DMA ? wave * P * TB : 0);
  auto seq_load = [&](Tile<KIND, KS>& T, int sq, int slot) {
    const bool past = sq >= ntiles;
    const bool in1 = DOCS == 2 && sq >= nt0;
    // Selects over values: a conditional over the DocRes structs themselves
    // selects their addresses and moves them to scratch memory.
    const rsrc_t d0 = dr0.d, d1 = dr1.d, s0 = dr0.s, s1 = dr1.s, n0 = dr0.m, n1 = dr1.m;
    DocRes r;
    r.d = past ? nul : (in1 ? d1 : d0);
    r.s = past ? nul : (in1 ? s1 : s0);
    r.m = past ? nul : (in1 ? n1 : n0);
    r.rowb = dr0.rowb;
    r.ss = in1 ? dr1.ss : dr0.ss;
    r.sm = in1 ? dr1.sm : dr0.sm;
    if constexpr (DMA) {
      const int tile = past ? 0 : (in1 ? sq - nt0 : sq);
#pragma unroll
      for (int k = 0; k < TI; ++k) {  // instruction k: rows (1024 / RB) k .. +(1024 / RB) - 1
        const int row = (1024 / RB) * k + lane / CPR, pos = lane % CPR, col = pos ^ (row % CPR);
        const uint32_t off = (uint32_t)(tile * 16 + row) * r.rowb + (uint32_t)(col * 16);
        dma16_lds<NT>(r.d, myring + slot * TB + k * 1024, off);
      }
    } else {
      load_tile<KIND, KS, VEC, !GSM, C16, DQ>(T, r, past ? 0 : (in1 ? sq - nt0 : sq), c, g, koff);
    }
  };
  // GSM: the scales and mins of a group of P = 4 tiles come with one dword
  // load per array (per doc of the workgroup) instead of two 8-byte loads per
  // tile: lane l loads dword l % 8 of tile slot l / 16 (tokens 2(l % 8) and
  // 2(l % 8) + 1), and each tile's lanes fetch the two dwords of their four
  // rows from those lanes. The stream issues a quarter fewer load
  // instructions, which is what bounds it.
  rsrc_t rsj = nul, rmj = nul;  // JOINT: scale / min rows of both docs
  uint32_t jo0 = 0u, jo1 = kOOB;  // byte offset of each doc's rows in them (kOOB: none)
  if constexpr (JOINT) {
    int64_t lo, hi;  // token rows of the scale arrays the range covers
    if (a.tok_group) {
      // Packed docs: each doc's rows (its length rounded up to 4, within the
      // tokens of D) wherever its token group starts; the range spans both.
      const int64_t t0 = 4 * tok_group_of(a, drow), t1 = two ? 4 * tok_group_of(a, drow + 1) : t0;
      auto rows_at = [&](int64_t t, int len) {
        const int64_t avail = t < 0 ? 0 : (a.tok_rows > t ? a.tok_rows - t : 0);
        const int64_t n = (len + 3) & ~3;
        return n < avail ? n : avail;
      };
      const int64_t n0 = rows_at(t0, len0), n1 = two ? rows_at(t1, len1) : 0;
      lo = n0 ? t0 : (n1 ? t1 : 0);
      if (n1 && t1 < lo) lo = t1;
      hi = lo;
      if (n0 && t0 + n0 > hi) hi = t0 + n0;
      if (n1 && t1 + n1 > hi) hi = t1 + n1;
      jo0 = n0 ? (uint32_t)((t0 - lo) * 2) : kOOB;
      jo1 = n1 ? (uint32_t)((t1 - lo) * 2) : kOOB;
    } else {
      // Padded docs: doc 1's rows start sm_b tokens after doc 0's.
      lo = drow * a.sm_b;
      hi = lo + (two ? a.sm_b + ((len1 + 3) & ~3) : ((len0 + 3) & ~3));
      jo1 = (uint32_t)(a.sm_b * 2);
    }
    rsj = make_rsrc(a.scales + lo, (uint32_t)((hi - lo) * 2));
    rmj = make_rsrc(a.mins + lo, (uint32_t)((hi - lo) * 2));
  }
  auto group_sm = [&](int ig, uint32_t& gs, uint32_t& gm) {
    const int sq = wave + NW * (ig + (lane >> 4));
    const bool past = sq >= ntiles || (lane >> 4) >= P;  // P = 2: lanes 32-63 idle
    const bool in1 = DOCS == 2 && sq >= nt0;
    const uint32_t off = (uint32_t)((in1 ? sq - nt0 : sq) * 32 + (lane & 7) * 4);
    if constexpr (JOINT) {
      // a doc without rows in the range reads zeros (kOOB + off stays past it)
      const uint32_t o = past ? kOOB : (in1 ? jo1 : jo0) + off;
      gs = ld4(rsj, o);
      gm = ld4(rmj, o);
    } else if constexpr (DOCS == 2) {
      const uint32_t o0 = (past || in1) ? kOOB : off, o1 = (!past && in1) ? off : kOOB;
      gs = ld4(dr0.s, o0) | ld4(dr1.s, o1);  // out-of-range lanes read zeros
      gm = ld4(dr0.m, o0) | ld4(dr1.m, o1);
    } else {
      gs = ld4(dr0.s, past ? kOOB : off);
      gm = ld4(dr0.m, past ? kOOB : off);
    }
  };
  auto tile_sm = [&](Tile<KIND, KS>& T, uint32_t gs, uint32_t gm, int slot) {
    const int src = 16 * slot + 2 * g;  // dwords 2g, 2g+1: tokens 4g .. 4g+3
    T.s = u32x2_t{lane_fetch(gs, src), lane_fetch(gs, src + 1)};
    T.m = u32x2_t{lane_fetch(gm, src), lane_fetch(gm, src + 1)};
  };

  float m[NQB];  // running max of the wave's current doc
  int mi[NQB];
  int cur = 0;   // doc of the wave's running max
#pragma unroll
  for (int nb = 0; nb < NQB; ++nb) {
    m[nb] = -INFINITY;
    mi[nb] = 0;
  }
  // Doc dd's maxima of this wave, merged over the four row groups, into
  // red_m[dd][wave] (scores only). Two-doc workgroups flush doc 0's when the
  // wave reaches doc 1, so the tile loop carries one set of running maxima.
  auto flush_max = [&](int dd) {
#pragma unroll
    for (int nb = 0; nb < NQB; ++nb) {
      const float v = max_over_groups(m[nb]);
      if (g == 0) red_m[dd][wave][nb * 16 + c] = v;
    }
  };

  // Tile i of the wave's sequence from ring slot T. The slot's refill (tile
  // i + P) is issued after the operands are taken and before the MFMAs:
  // REFILL_ANY loads it whether or not it exists (past the end: the empty
  // range), REFILL_IF only if it exists, REFILL_NONE not at all.
  enum { REFILL_NONE, REFILL_IF, REFILL_ANY };
  // slot: T's ring position; wait_tag: the vector-memory instructions issued
  // after this tile's DMA loads (DMA path)
  auto process = [&](auto mode_tag, Tile<KIND, KS>& T, int i, int slot, auto wait_tag)
                     __attribute__((always_inline)) {
    constexpr int MODE = decltype(mode_tag)::value;
    const int sq = wave + NW * i;
    const bool in1 = DOCS == 2 && sq >= nt0;
    const int tile = in1 ? sq - nt0 : sq;
    const int len = in1 ? len1 : len0;
    if (DOCS == 2 && in1 && cur == 0) {  // first tile of doc 1 for this wave
      flush_max(0);
#pragma unroll
      for (int nb = 0; nb < NQB; ++nb) m[nb] = -INFINITY;
      cur = 1;
    }
    u32x4_t af[KS];
    if constexpr (DMA) {
      // the tile is in LDS once at most wait_tag newer loads are in flight;
      // its fragments are in registers before the slot is refilled
      wait_vmem<decltype(wait_tag)::value>();
      if constexpr (U8) {
        // codes of k-steps 2h, 2h + 1: bytes 64h + 16g .. +15 of row c (frag_k0)
#pragma unroll
        for (int h = 0; h < KS / 2; ++h)
          T.v[h] = *reinterpret_cast<const u32x4_t*>(myring + slot * TB + c * RB + (((4 * h + g) ^ (c % CPR)) * 16));
      } else {
#pragma unroll
        for (int t = 0; t < KS; ++t)
          af[t] = *reinterpret_cast<const u32x4_t*>(myring + slot * TB + c * RB + (((4 * t + g) ^ (c % CPR)) * 16));
      }
      wait_lds();
    }
#pragma unroll
    for (int t = 0; t < KS; ++t) {
      if constexpr (!DMA_FP) af[t] = tile_operand<KIND, KS>(T, t);
      if constexpr (DQ) af[t] = dequant_biased_f16(af[t], T.s[0], T.m[0]);
      if constexpr (KMASK && !U8) {
        if (has_partial && t == tp) af[t] &= pmask;
      }
    }
    float sc[4], off[4];
    if constexpr (U8 && !DQ) {
#pragma unroll
      for (int r = 0; r < 4; ++r) tile_affine(T.s, T.m, r, sc[r], off[r]);
    }
    // uint8 codes were converted into registers of their own, so the slot is
    // free; fp16/bf16 MFMAs read the slot itself (the compiler keeps a copy).
    if constexpr (MODE == REFILL_ANY) seq_load(T, wave + NW * (i + P), slot);
    if constexpr (MODE == REFILL_IF) {
      if (i + P < my_n) seq_load(T, wave + NW * (i + P), slot);
    }
    const int row0 = tile * 16 + 4 * g;
    // S of this tile against every query block, folded into the running
    // maxima. TAIL (the doc's last, partial tile) masks rows past len.
    // The two instances are chosen by a branch before the MFMAs, so each
    // keeps its MFMAs and the first VALU reads of their results in one
    // basic block: the compiler inserts the MFMA-to-VALU wait states within
    // a block, and a branch between the two (a conditional mask after the
    // MFMAs) let it place the reads too early.
    auto score_tile = [&](auto tail_tag) __attribute__((always_inline)) {
      constexpr bool TAIL = decltype(tail_tag)::value;
#pragma unroll
      for (int nb = 0; nb < NQB; ++nb) {
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < KS; ++t) acc = mfma16x16x32<BF>(af[t], qf[nb][t], acc);
        if constexpr (U8 && !DQ) {
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[r] = fmaf(sc[r], acc[r], off[r] * qsum[nb]);
        }
        if constexpr (TAIL) {
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[r] = row0 + r < len ? acc[r] : -INFINITY;
        }
        if constexpr (ARGMAX) {
#pragma unroll
          for (int r = 0; r < 4; ++r) argmax_fold(acc[r], row0 + r, m[nb], mi[nb]);
        } else {
          m[nb] = fold_max4(m[nb], acc[0], acc[1], acc[2], acc[3]);
        }
      }
    };
    if (tile * 16 + 16 > len) {
      score_tile(std::true_type{});
    } else {
      score_tile(std::false_type{});
    }
  };
  using RefillNone = std::integral_constant<int, REFILL_NONE>;
  using RefillIf = std::integral_constant<int, REFILL_IF>;
  using RefillAny = std::integral_constant<int, REFILL_ANY>;

  Tile<KIND, KS> buf[P];
  // The first P tiles are loaded unconditionally (past the wave's sequence:
  // the empty range), so the wait before the query exchange counts exactly
  // the tile loads issued after the query loads and waits for the query alone.
  uint32_t gsc = 0, gmc = 0, gsn = 0, gmn = 0;  // group scales / mins: current, next
  if constexpr (GSM) group_sm(0, gsc, gmc);
#pragma unroll
  for (int s = 0; s < (QALIAS ? P - 1 : P); ++s) seq_load(buf[s], wave + NW * s, s);
  q_exchange();
  if constexpr (QALIAS) {
    __syncthreads();  // every wave has its fragments: the last slots take their tiles
    seq_load(buf[P - 1], wave + NW * (P - 1), P - 1);
  }
  if constexpr (FIXED) {
    // A fixed load pattern: every group of P tiles that has a next group
    // refills all P slots, so the compiler's wait before each tile counts the
    // P-1 tiles still in flight behind it (a conditional load makes it wait
    // for all of them). The empty-range loads past the end cost issue slots,
    // which long docs amortise (Q[128,128] x 1024-token docs: 52.7 -> 49.4 us)
    // and short ones no longer lose (config 1: 61.2 -> 60.9 us). The argmax
    // instances keep conditional loads: the fixed pattern's registers cost
    // them a wave per SIMD.
    int i0 = 0;
    for (; i0 + P < my_n; i0 += P) {
      if constexpr (GSM) group_sm(i0 + P, gsn, gmn);
#pragma unroll
      for (int s = 0; s < P; ++s) {
        if constexpr (GSM) tile_sm(buf[s], gsc, gmc, s);
        // in the steady state P - 1 tiles' loads follow each tile's
        process(RefillAny{}, buf[s], i0 + s, s, std::integral_constant<int, TI * (P - 1) + GL>{});
      }
      gsc = gsn;
      gmc = gmn;
    }
    // the last group refills nothing: P - 1 - s tiles' loads follow tile s's
    auto last = [&](auto s_tag) __attribute__((always_inline)) {
      constexpr int s = decltype(s_tag)::value;
      if constexpr (s < P) {
        if (i0 + s < my_n) {
          if constexpr (GSM) tile_sm(buf[s], gsc, gmc, s);
          process(RefillNone{}, buf[s], i0 + s, s, std::integral_constant<int, TI * (P - 1 - s)>{});
        }
      }
    };
    static_assert(P <= 4, "the last group is unrolled for up to four slots");
    last(std::integral_constant<int, 0>{});
    last(std::integral_constant<int, 1>{});
    last(std::integral_constant<int, 2>{});
    last(std::integral_constant<int, 3>{});
  } else {
    for (int i0 = 0; i0 < my_n; i0 += P) {
#pragma unroll
      for (int s = 0; s < P; ++s)
        if (i0 + s < my_n) process(RefillIf{}, buf[s], i0 + s, s, std::integral_constant<int, 0>{});
    }
  }

  // ---- merge the four row groups of each query token, then the four waves ----
  if constexpr (ARGMAX) {
#pragma unroll
    for (int nb = 0; nb < NQB; ++nb) {
      float v = m[nb];
      int ix = mi[nb];
      argmax_over_groups(v, ix);
      if (g == 0) {
        red_m[0][wave][nb * 16 + c] = v;
        red_i[wave][nb * 16 + c] = ix;
      }
    }
  } else if constexpr (DOCS == 2) {
    if (cur == 0) {  // the wave never reached doc 1
      flush_max(0);
#pragma unroll
      for (int nb = 0; nb < NQB; ++nb) m[nb] = -INFINITY;
    }
    flush_max(1);
  } else {
    flush_max(0);
  }
  __syncthreads();
  const int dd = DOCS == 2 ? wave : 0;  // wave 0 sums doc 0, wave 1 doc 1
  if (wave < DOCS && (dd == 0 || two)) {
    float part = 0.f;
    for (int r = lane; r < QROWS; r += 64) {
      float v = red_m[dd][0][r];
      int ix = ARGMAX ? red_i[0][r] : 0;
#pragma unroll
      for (int w = 1; w < NW; ++w) {
        if constexpr (ARGMAX) {
          argmax_merge(v, ix, red_m[0][w][r], red_i[w][r]);
        } else {
          v = vmax(v, red_m[dd][w][r]);
        }
      }
      const int q = q0 + r;
      if (q < a.Lq) {
        part += v;
        if constexpr (ARGMAX) a.argmax[(int64_t)item * a.Lq + q] = ix;
      }
    }
    const float total = wave_sum(part);
    if (lane == 0) {
      if (npass == 1) {
        store_score(a, qi, b + dd, total);
      } else {
        a.partial[(int64_t)pass * a.Nq * a.B + item] = total;
      }
    }
  }
}

// scores[qi, b] = sum over passes p (in order) of partial[p][qi*B + b].
__global__ void __launch_bounds__(256) sum_passes_kernel(FwdArgs a, int npass) {
  const int64_t items = (int64_t)a.Nq * a.B;
  const int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= items) return;
  float s = 0.f;
  for (int p = 0; p < npass; ++p) s += a.partial[(int64_t)p * items + item];
  const int64_t qi = item / a.B, b = item - qi * a.B;
  store_score(a, qi, b, s);
}


// uint8 docs of one query with a full 128-row query tile (Lq in (64, 128],
// d in (64, 128], vector path, padded docs), one doc per workgroup. The four
// waves share each 16-token doc tile instead of each holding all 128 query
// rows: wave w loads tokens 4w .. 4w+3 of the tile (lane (c, g): token
// 4w + g, codes 8c .. 8c+7), dequantises them to fp16 as the reference does
// (flash_maxsim_quant.py:89) and writes them to LDS; after one barrier every
// wave reads the whole dequantised tile as MFMA A-fragments and multiplies it
// by its own 32 query rows (two 16-row blocks). A wave then needs 80 VGPRs
// instead of 242, so up to six share a SIMD instead of two and hide each
// other's dequantisation, LDS and MFMA latency (config 4's docs under a
// 128-token query 113.6 -> 104.4 us, 5000 docs of 512 tokens 103.1 -> 97.7
// us, Q[96, 128] over 300-token docs 59.8 -> 53.1 us, one box).
// Token rows past the doc's length load its last row again: a duplicate of a
// valid row leaves the max unchanged, so no tile needs a mask.
// Measured and not kept: two waves of 64 rows (LDS reads halved: within 1 %),
// two tiles per barrier, the next tile's LDS reads issued before this tile's
// MFMAs (+16 VGPRs: slower), several docs per workgroup as one tile sequence
// (its cursor arithmetic cost more than the shared ring saved).
constexpr int kShRow = 272;  // LDS bytes per dequantised token row; 256 + 16 spreads a b128 read's lanes over all banks

// NT: the code loads (four whole 128-byte rows per wave instruction) are
// non-temporal, for doc sets past the last-level cache (kLlcBytes: config 4's
// docs 105.9 -> 101.8 us, 5000 docs of 512 tokens 96.6 -> 94.0 us; smaller
// sets lost up to 13 % with it, no longer found in that cache by the next call).
template <int P, bool NT>
__global__ void __launch_bounds__(256) stream_u8_shared_kernel(FwdArgs a) {
  static_assert(kStreamWaves == 4, "four waves of 32 query rows and 4 tile tokens each");
  __shared__ __attribute__((aligned(16))) unsigned char tl[2][16 * kShRow];
  __shared__ float part[kStreamWaves];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, g = lane >> 4;
  const int b = blockIdx.x;
  int len = a.lengths ? a.lengths[b] : a.Ld;
  len = len < 0 ? 0 : (len > a.Ld ? a.Ld : len);
  const int nt = (len + 15) >> 4;

  // B-fragments of query rows 32 * wave + 16 * nb + c, k-step t: k = 32t + 8g .. +7
  const rsrc_t rq = make_rsrc(a.Q, (uint32_t)(a.Lq_rows * a.sq_l * 2));
  const int kp = a.d & ~7;
  u32x4_t qf[2][4];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const uint32_t rowoff = query_row_offset(a, b, 32 * wave + 16 * nb + c);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int k0 = 32 * t + 8 * g;
      qf[nb][t] = ld16(rq, k0 < a.d ? rowoff + (uint32_t)(k0 * 2) : kOOB);
      if (k0 == kp) qf[nb][t] &= prefix_mask16(a.d & 7);
    }
  }

  const DocRes dr = make_doc_res<KIND_U8, true>(a, b, len);
  const rsrc_t nul = make_rsrc(a.D, 0u);
  // the lane's token row within a tile, the doc's last row, its byte in a row
  // (codes at k >= d meet zero query values)
  const int r0 = 4 * wave + g, rlast = len - 1;
  const uint32_t kb = (uint32_t)(8 * c) < (uint32_t)a.d ? (uint32_t)(8 * c) : kOOB;
  struct Slot {
    u32x2_t v;
    uint32_t s, m;
  };
  auto load = [&](Slot& S, int tile) {
    int row = tile * 16 + r0;
    row = row < rlast ? row : rlast;
    const bool past = tile >= nt;  // the empty range: no access, a fixed load count
    S.v = __builtin_amdgcn_raw_buffer_load_b64(past ? nul : dr.d, (uint32_t)row * dr.rowb + kb, 0, NT ? 2 : 0);
    S.s = ld2(past ? nul : dr.s, (uint32_t)row * 2u);
    S.m = ld2(past ? nul : dr.m, (uint32_t)row * 2u);
  };
  typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
  auto stage = [&](const Slot& S, int buf) {
    // dequant_biased_f16 with the scale and min taken from the low halves by
    // the packed ops' operand selects instead of widened first
    const u32x4_t h = codes_to_f16_biased(S.v);
    const _Float16 sc = __builtin_bit_cast(_Float16, (uint16_t)S.s), mn = __builtin_bit_cast(_Float16, (uint16_t)S.m);
    const h2_t sc2 = {sc, sc}, mn2 = {mn, mn};
    const h2_t bias = {(_Float16)kCodeBias, (_Float16)kCodeBias};
    u32x4_t o;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t hi = h[i];
      const h2_t cd = __builtin_bit_cast(h2_t, hi) - bias;
      o[i] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(cd, sc2, mn2));
    }
    *reinterpret_cast<u32x4_t*>(&tl[buf][r0 * kShRow + 16 * c]) = o;
  };
  float m[2] = {-INFINITY, -INFINITY};
  auto score = [&](int buf) {
    u32x4_t af[4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
      af[t] = *reinterpret_cast<const u32x4_t*>(&tl[buf][c * kShRow + (32 * t + 8 * g) * 2]);
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < 4; ++t) acc = mfma16x16x32<false>(af[t], qf[nb][t], acc);
      m[nb] = fold_max4(m[nb], acc[0], acc[1], acc[2], acc[3]);
    }
  };

  // Tile i: loaded into ring slot i % P, staged into LDS buffer i & 1 (P is
  // even), scored after the barrier. A buffer is rewritten two tiles later,
  // after the next barrier, by which point every wave has read it.
  static_assert(P % 2 == 0, "ring slots map to LDS buffers by parity");
  Slot ring[P];
#pragma unroll
  for (int s = 0; s < P; ++s) load(ring[s], s);
  int i0 = 0;
  for (; i0 + P < nt; i0 += P) {
#pragma unroll
    for (int s = 0; s < P; ++s) {
      stage(ring[s], s & 1);
      load(ring[s], i0 + s + P);
      __syncthreads();
      score(s & 1);
    }
  }
#pragma unroll
  for (int s = 0; s < P; ++s) {
    if (i0 + s < nt) {  // uniform over the workgroup
      stage(ring[s], s & 1);
      __syncthreads();
      score(s & 1);
    }
  }

  // per wave: sum over its valid query rows of the max over the doc (-inf
  // for an empty doc); then the four waves' sums in order
  float sum = 0.f;
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const float v = max_over_groups(m[nb]);
    if (g == 0 && 32 * wave + 16 * nb + c < a.Lq) sum += v;
  }
  sum = wave_sum(sum);
  if (lane == 0) part[wave] = sum;
  __syncthreads();
  if (threadIdx.x == 0) {
    float total = part[0];
#pragma unroll
    for (int w = 1; w < kStreamWaves; ++w) total += part[w];
    store_score(a, 0, b, total);
  }
}

template <int KIND, int NQB, int KS, bool KMASK, bool ARGMAX, bool VEC = true, bool C16 = VEC>
hipError_t launch_one(const FwdArgs& a, hipStream_t s) {
  constexpr int QROWS = NQB * 16;
  const int npass = (a.Lq + QROWS - 1) / QROWS;
  const int64_t items = (int64_t)a.Nq * a.B;
  if constexpr (KIND == KIND_U8 && !ARGMAX) {
    // uint8 docs of one query in one pass: two docs per workgroup.
    // d in (64, 128] and 65-128 query tokens over padded docs: the shared-tile kernel.
    if constexpr (NQB == 8 && KS == 4 && VEC) {
      if (a.Nq == 1 && npass == 1 && !a.qidx && !a.tok_group) {
        if (stream_doc_bytes(a, 1) >= kLlcBytes) {
          hipLaunchKernelGGL((stream_u8_shared_kernel<4, true>), dim3((unsigned)a.B), dim3(256), 0, s, a);
        } else {
          hipLaunchKernelGGL((stream_u8_shared_kernel<4, false>), dim3((unsigned)a.B), dim3(256), 0, s, a);
        }
        return hipGetLastError();
      }
    }
    if (a.Nq == 1 && npass == 1 && !a.qidx) {
      const dim3 grid((unsigned)((a.B + 1) / 2));
      // One scale range per pair when its offsets stay below 2^31 bytes: a
      // pair of padded scale rows, or the whole packed scale array.
      const int64_t sm_rows = a.tok_group ? a.tok_rows : a.sm_b + a.Ld;
      // Without VEC (scale rows not 8-byte aligned, e.g. Ld % 4 != 0) but with
      // 16-byte code rows (C16), codes still come 16 bytes per load, which
      // halves the load instructions that bound this stream (Lq = 32 over
      // 5000 docs of 77 tokens 19.9 -> 15.5 us, 20000 docs 65.6 -> 48.2 us,
      // 301-token docs 55.8 -> 38.5 us).
      constexpr bool GROUPS = VEC && stream_depth<KIND, NQB, KS>() == 4;  // group scale loads
      if (a.Ld <= 128) {
        // Docs of up to 128 tokens: a two-tile ring.
        // The deeper ring's fixed refill pattern issues loads past a short
        // pair's tiles and its fill is paid per workgroup (5000 docs of 77
        // tokens: 22.0 -> 19.3 us, 20000: 77.9 -> 65.5 us, a 64-token query
        // -20 %, 128-token docs -5 %); longer docs keep it (200 tokens: +4 %
        // with two tiles, config 4: +7.5 %).
        // With aligned scale rows one range covers both docs' scales and the
        // ring's two tiles take their scales with one load per array (128-
        // token docs 18.6 -> 17.3 us, 20000 docs of 76 tokens 44.6 -> 43.4 us).
        if (VEC && sm_rows * 2 + 64 < ((int64_t)1 << 31)) {
          hipLaunchKernelGGL((stream_fwd_kernel<KIND, NQB, KS, KMASK, ARGMAX, VEC, 2, VEC, 2, C16>), grid, dim3(256),
                             0, s, a);
        } else {
          hipLaunchKernelGGL((stream_fwd_kernel<KIND, NQB, KS, KMASK, ARGMAX, VEC, 2, false, 2, C16>), grid, dim3(256),
                             0, s, a);
        }
      } else if (GROUPS && sm_rows * 2 + 64 < ((int64_t)1 << 31)) {
        // The LDS ring (queries of up to 32 tokens, d = 128) takes 32 KB of
        // LDS per workgroup, four workgroups per CU against eight: it pays
        // once the stream is long, and costs where start-up and the last
        // round of workgroups weigh more (1000-10000 docs of 300-1024 tokens,
        // ring against VGPR ring: 300 tokens 16.0 / 32.0 / 67.6 against
        // 17.0 / 36.1 / 67.7 us, 512 tokens 22.3 / 57.5 / 112.0 against
        // 26.2 / 54.3 / 100.7 us, 1024 tokens 40.7 / 111.8 / 217.8 against
        // 45.1 / 100.0 / 194.5 us for 2000 / 5000 / 10000 docs; config 4
        // 61.5 against 57.9 us).
        bool ring = true;
        if constexpr (NQB <= 2 && KS == 4 && !KMASK) ring = stream_doc_bytes(a, 1) >= kLlcBytes;
        if (ring) {
          hipLaunchKernelGGL((stream_fwd_kernel<KIND, NQB, KS, KMASK, ARGMAX, VEC, 2, GROUPS>), grid, dim3(256), 0, s,
                             a);
        } else {
          hipLaunchKernelGGL((stream_fwd_kernel<KIND, NQB, KS, KMASK, ARGMAX, VEC, 2, GROUPS, 0, VEC, false>), grid,
                             dim3(256), 0, s, a);
        }
      } else {
        hipLaunchKernelGGL((stream_fwd_kernel<KIND, NQB, KS, KMASK, ARGMAX, VEC, 2, false, 0, C16>), grid, dim3(256), 0,
                           s, a);
      }
      return hipGetLastError();
    }
  }
  if constexpr (KIND != KIND_U8 && !ARGMAX && NQB * KS >= 4) {
    // fp16/bf16 docs of one query whose query tile fills 128 VGPRs: two docs
    // per workgroup as well (Q[96..128, 128] x 5000 docs of 300 tokens:
    // 85.6 -> 76.4 and 91.5 -> 79.8 us; 1024-token docs unchanged); with
    // masked widths they fall to one (d = 96, Lq = 128: +10 %). Smaller tiles
    // lose a wave per SIMD to the second doc's registers, which costs long
    // docs (Lq = 32: 300-token docs +4.5 %, 1024 +2 %) but pays for docs of up
    // to 256 tokens, whose per-workgroup query load and ring start-up are then
    // shared by two docs (Lq = 32: 64-token docs 46.8 -> 32.4 us, 77 tokens
    // 26.7 -> 19.9 us, 160 tokens 60.9 -> 52.6 us; Lq = 16 and 64 over
    // 77-token docs -26 % and -17 %; d = 96: 77 tokens -30 %, 128 -22 %).
    // Per-query docs pair two of one query's docs (100 queries x 1000 docs
    // of 77 tokens: 577 -> 376 us).
    constexpr bool BIG = NQB * KS >= 32;
    if (!BIG && (a.Nq == 1 || !a.shared_docs) && npass == 1 && !a.qidx && a.Ld <= 128) {
      // docs of up to 128 tokens: a two-tile ring, as for uint8 (Lq = 32 over
      // 20000 docs of 77 tokens 75.8 -> 62.2 us, 10000 of 64 -19 %, 5000 of 77
      // -11 %; 128-token docs -1 %)
      hipLaunchKernelGGL((stream_fwd_kernel<KIND, NQB, KS, KMASK, ARGMAX, VEC, 2, false, 2>),
                         dim3((unsigned)(a.Nq * ((a.B + 1) / 2))), dim3(256), 0, s, a);
      return hipGetLastError();
    }
    if ((a.Nq == 1 || !a.shared_docs) && npass == 1 && !a.qidx && (BIG ? !KMASK : a.Ld <= 256)) {
      const dim3 grid((unsigned)(a.Nq * ((a.B + 1) / 2)));
      if constexpr (stream_dma_fp<KIND, KS, KMASK, ARGMAX, 0>()) {
        if (stream_doc_bytes(a, 2) < kLlcBytes) {  // cached doc sets: the default policy
          hipLaunchKernelGGL((stream_fwd_kernel<KIND, NQB, KS, KMASK, ARGMAX, VEC, 2, false, 0, VEC, true, false>),
                             grid, dim3(256), 0, s, a);
          return hipGetLastError();
        }
      }
      hipLaunchKernelGGL((stream_fwd_kernel<KIND, NQB, KS, KMASK, ARGMAX, VEC, 2>), grid, dim3(256), 0, s, a);
      return hipGetLastError();
    }
  }
  const int64_t grid = npass > 1 ? ((items + 7) / 8) * 8 * npass : items;
  bool cached = false;  // a doc set the last-level cache holds: the LDS ring's default policy
  if constexpr (stream_dma_fp<KIND, KS, KMASK, ARGMAX, 0>()) cached = stream_doc_bytes(a, KindInfo<KIND>::esz) < kLlcBytes;
  if constexpr (stream_dma_fp<KIND, KS, KMASK, ARGMAX, 0>()) {
    if (cached) {
      hipLaunchKernelGGL((stream_fwd_kernel<KIND, NQB, KS, KMASK, ARGMAX, VEC, 1, false, 0, C16, true, false>),
                         dim3((unsigned)grid), dim3(256), 0, s, a);
    }
  }
  if (!cached) {
    hipLaunchKernelGGL((stream_fwd_kernel<KIND, NQB, KS, KMASK, ARGMAX, VEC, 1, false, 0, C16>), dim3((unsigned)grid),
                       dim3(256), 0, s, a);
  }
  if (npass > 1) {
    hipLaunchKernelGGL(sum_passes_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, s, a, npass);
  }
  return hipGetLastError();
}

template <int KIND, int NQB, int KS>
hipError_t dispatch_flags(const FwdArgs& a, bool am, hipStream_t s) {
  if constexpr (KIND == KIND_U8) {
    (void)am;
    // FwdArgs::vec bit 0: the vector path; bit 1: 16-byte code rows only.
    // Rows of exactly 128 codes take the unmasked instance (its doc tiles
    // come through the LDS ring).
    if constexpr (KS == 4) {
      if ((a.vec & 1) && a.d == 128) return launch_one<KIND, NQB, KS, false, false, true>(a, s);
    }
    if (a.vec & 1) return launch_one<KIND, NQB, KS, true, false, true>(a, s);
    return (a.vec & 2) ? launch_one<KIND, NQB, KS, true, false, false, true>(a, s)
                       : launch_one<KIND, NQB, KS, true, false, false, false>(a, s);
  } else {
    const bool kmask = a.d != 32 * KS;
    if (kmask) return am ? launch_one<KIND, NQB, KS, true, true>(a, s) : launch_one<KIND, NQB, KS, true, false>(a, s);
    return am ? launch_one<KIND, NQB, KS, false, true>(a, s) : launch_one<KIND, NQB, KS, false, false>(a, s);
  }
}

template <int KIND, int KS>
hipError_t dispatch_nqb(const FwdArgs& a, bool am, hipStream_t s) {
  const int nqb = stream_fwd_nqb(a.Lq, a.d);
  switch (nqb) {
    case 1: return dispatch_flags<KIND, 1, KS>(a, am, s);
    case 2: return dispatch_flags<KIND, 2, KS>(a, am, s);
    case 4: return dispatch_flags<KIND, 4, KS>(a, am, s);
    default:
      if constexpr (KS <= 4) return dispatch_flags<KIND, 8, KS>(a, am, s);
      return hipErrorInvalidValue;
  }
}

template <int KIND>
hipError_t dispatch_ks(const FwdArgs& a, bool am, hipStream_t s) {
  switch (stream_fwd_ks(a.d)) {
    case 1:
      // uint8 tiles pair k-steps: d <= 32 runs as two, the second reading zeros.
      if constexpr (KIND == KIND_U8) {
        return dispatch_nqb<KIND, 2>(a, am, s);
      } else {
        return dispatch_nqb<KIND, 1>(a, am, s);
      }
    case 2: return dispatch_nqb<KIND, 2>(a, am, s);
    case 4: return dispatch_nqb<KIND, 4>(a, am, s);
    case 8: return dispatch_nqb<KIND, 8>(a, am, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

bool stream_fwd_supported(int d) { return d >= 1 && d <= 256; }

int stream_fwd_ks(int d) {
  const int ks = (d + 31) / 32;
  return ks <= 1 ? 1 : ks <= 2 ? 2 : ks <= 4 ? 4 : 8;
}

// Query tokens per pass: as many 16-token blocks as Lq needs, capped so the
// query tile stays within 128 VGPRs (NQB * KS <= 32). uint8 docs take the
// full tile too since their 128-row instance keeps two waves per SIMD (see
// stream_depth): one pass instead of two of 64 rows, whose second pass read
// the doc from L2 but repeated the code widening and affine epilogue (Lq =
// 128 over 5000 docs of 512 tokens: 121 -> 106 us; Lq = 96: 115 -> 101 us).
int stream_fwd_nqb(int Lq, int d) {
  const int need = (Lq + 15) / 16;
  const int cap = 32 / stream_fwd_ks(d);
  const int nqb = need <= 1 ? 1 : need <= 2 ? 2 : need <= 4 ? 4 : 8;
  return nqb < cap ? nqb : cap;
}

int stream_fwd_passes(int Lq, int d) {
  const int rows = 16 * stream_fwd_nqb(Lq, d);
  return (Lq + rows - 1) / rows;
}

hipError_t launch_stream_fwd(int kind, const FwdArgs& a, bool with_argmax, hipStream_t s) {
  switch (kind) {
    case KIND_F16: return dispatch_ks<KIND_F16>(a, with_argmax, s);
    case KIND_BF16: return dispatch_ks<KIND_BF16>(a, with_argmax, s);
    case KIND_U8: return dispatch_ks<KIND_U8>(a, false, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fmx
