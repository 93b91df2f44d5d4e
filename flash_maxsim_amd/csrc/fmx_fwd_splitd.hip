// Split-d MaxSim forward for large embeddings (256 < d <= 4096).
//
// Same contract as _maxsim_fwd_kernel / _maxsim_int8_kernel (reference
// flash_maxsim/flash_maxsim.py:80-146, flash_maxsim/flash_maxsim_quant.py:40-98)
// for shapes whose query tile does not fit one wave's registers. The reference
// covers those with small Triton blocks (flash_maxsim.py:29-34, any d_pad via the
// fallback of :71), its tests go to d = 2048.
//
// One workgroup of eight waves scores one (query, doc) pair for one pass of up
// to 16*NQB query tokens. Wave w owns the k-steps [w*KSW, (w+1)*KSW), i.e. the
// dims [32*KSW*w, 32*KSW*(w+1)): it holds that slice of the query tile in VGPRs
// and streams the same slice of every 16-token doc tile straight from HBM.
// Per tile each wave's MFMAs give a partial S over its slice; the partials
// meet in LDS, where wave nb sums the eight slices of
// query block nb in wave order (deterministic), applies the uint8 affine
// epilogue and the length mask, and folds the rows into its running max. The
// max therefore always sees the full-d similarity, never a partial one.
// The partial buffer is double-buffered by tile parity, so one barrier per
// tile suffices: tile t+2 rewrites tile t's buffer only after every wave has
// passed tile t+1's barrier, i.e. after it finished reducing tile t.
#include "fmx_kernels.h"
#include "fmx_tile.h"

namespace fmx {
namespace {

constexpr int kSplitWaves = 8;

// VEC: uint8 vector load path (FwdArgs::vec); true for fp16/bf16.
// PERSIST (one query, one pass, no query gather): a fixed grid of resident
// workgroups loads the query slice once and walks docs b, b + G, ...
template <int KIND, int NQB, int KSW, bool KMASK, bool ARGMAX, bool VEC, bool PERSIST = false, bool C16 = VEC>
__global__ void __launch_bounds__(512) splitd_fwd_kernel(FwdArgs a) {
  constexpr int NW = kSplitWaves, QROWS = NQB * 16;
  // Tiles in flight per wave: 2 when the query slice takes 128 VGPRs, which
  // leaves room for the pipelined tile's results next to the buffers.
  constexpr int P = (KSW >= 8 || NQB * KSW >= 32) ? 2 : 3;
  constexpr int ESZ = KindInfo<KIND>::esz;
  constexpr bool BF = KindInfo<KIND>::bf;
  constexpr bool U8 = KIND == KIND_U8;
  static_assert(NQB <= NW, "one owning wave per query block");
  __shared__ f32x4_t part[2][NW][NQB][64];
  __shared__ float qs_part[U8 ? NW : 1][QROWS];
  __shared__ float red_m[QROWS];
  __shared__ int red_i[ARGMAX ? QROWS : 1];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, g = lane >> 4;
  // Workgroups go to the eight XCDs round-robin. All U units (query, pass) of
  // one doc share an XCD and start back to back, so the doc streams from HBM
  // once and the other units read it from that XCD's L2: workgroup
  // x = 8 * (U * grp + u) + k runs unit u of doc slot 8 * grp + k, where a doc
  // slot is a shared doc (U = Nq * passes) or a (query, doc) pair (U = passes).
  const int npass = (a.Lq + QROWS - 1) / QROWS;
  const bool shared_q = a.shared_docs && a.Nq > 1;
  const int U = (shared_q ? a.Nq : 1) * npass;
  const int nslots = shared_q ? a.B : a.Nq * a.B;
  int slot = blockIdx.x, u = 0;
  if (U > 1) {
    const int x = blockIdx.x, k = x & 7, r = x >> 3;
    const int grp = r / U;
    u = r - grp * U;
    slot = 8 * grp + k;
    if (slot >= nslots) return;  // uniform over the workgroup, before any barrier
  }
  const int pass = u % npass;
  int qi, b;
  if (shared_q) {
    b = slot;
    qi = u / npass;
  } else {
    qi = slot / a.B;
    b = slot - qi * a.B;
  }
  const bool owner = wave < NQB;  // wave w reduces and maxes query block w

  const int tbase = wave * KSW;  // first global k-step of this wave (KSW is even)
  const int kp = a.d & ~7;
  int tp, gp;  // local slot of the partial group (out of range: another wave's)
  frag_slot<KIND>(kp - 32 * tbase, tp, gp);
  if (kp < 32 * tbase) tp = -1;
  const u32x4_t pmask = prefix_mask16(g == gp ? (a.d & 7) : 8);
  const bool has_partial = KMASK && (a.d & 7) != 0;

  // ---- query slice of this pass ----
  const int q0 = pass * QROWS;
  const rsrc_t rq = make_rsrc((const char*)a.Q + (int64_t)qi * a.sq_n * 2, (uint32_t)(a.Lq_rows * a.sq_l * 2));
  u32x4_t qf[NQB][KSW];
#pragma unroll
  for (int nb = 0; nb < NQB; ++nb) {
    const uint32_t rowoff = query_row_offset(a, b, q0 + nb * 16 + c);
#pragma unroll
    for (int t = 0; t < KSW; ++t) {
      const int k0 = 32 * tbase + frag_k0<KIND>(t, g);
      if constexpr (KMASK) {
        qf[nb][t] = ld16(rq, k0 < a.d ? rowoff + (uint32_t)(k0 * 2) : kOOB);
        if (has_partial && t == tp) qf[nb][t] &= pmask;
      } else {
        qf[nb][t] = ld16(rq, rowoff + (uint32_t)(k0 * 2));
      }
    }
  }
  float qsum = 0.f;  // owner waves, uint8 docs: full-d sum of query token 16*wave + c
  if constexpr (U8) {
#pragma unroll
    for (int nb = 0; nb < NQB; ++nb) {
      const float s = query_row_sum<KSW>(qf[nb]);
      if (g == 0) qs_part[wave][nb * 16 + c] = s;
    }
    __syncthreads();
    if (owner) {
#pragma unroll
      for (int w = 0; w < NW; ++w) qsum += qs_part[w][wave * 16 + c];
    }
  }

  for (;;) {
  const int item = qi * a.B + b;
  const int64_t drow = a.shared_docs ? (int64_t)b : (int64_t)item;
  int len = a.lengths ? a.lengths[drow] : a.Ld;
  // uniform: the loads below take it into scalar buffer resources
  len = __builtin_amdgcn_readfirstlane(len < 0 ? 0 : (len > a.Ld ? a.Ld : len));
  const int ntiles = (len + 15) >> 4;

  // ---- doc stream ----
  const DocRes dr = make_doc_res<KIND, VEC>(a, drow, len);
  uint32_t koff[KSW];
#pragma unroll
  for (int t = 0; t < KSW; ++t) {
    const int k0 = 32 * tbase + frag_k0<KIND>(t, g);
    koff[t] = (KMASK && k0 >= a.d) ? kOOB : (uint32_t)(k0 * ESZ);  // past d: zeros
  }

  float m = -INFINITY;
  int mi = 0;
  // Owner waves: folds tile rt (its eight partials in part[rt & 1]) into the
  // running max, with the uint8 affine constants of that tile.
  auto reduce_tile = [&](int rt, const float (&rsc)[4], const float (&roff)[4]) {
    if (!owner) return;
    f32x4_t S = part[rt & 1][0][wave][lane];
#pragma unroll
    for (int w = 1; w < NW; ++w) S += part[rt & 1][w][wave][lane];
    if constexpr (U8) {
#pragma unroll
      for (int r = 0; r < 4; ++r) S[r] = fmaf(rsc[r], S[r], roff[r] * qsum);
    }
    const int row0 = rt * 16 + 4 * g;
    if (rt * 16 + 16 > len) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (row0 + r >= len) S[r] = -INFINITY;
    }
    if constexpr (ARGMAX) {
#pragma unroll
      for (int r = 0; r < 4; ++r) argmax_fold(S[r], row0 + r, m, mi);
    } else {
      m = fold_max4(m, S[0], S[1], S[2], S[3]);
    }
  };

  // Software pipeline, one barrier per tile: a wave issues tile t's MFMAs,
  // then reduces tile t-1 (written before the previous barrier) while they
  // run, then stores tile t's partials. part[t & 1] is rewritten at tile t+2,
  // after every owner passed tile t+1's barrier, i.e. finished reducing t.
  Tile<KIND, KSW> buf[P];
  float psc[4] = {0.f, 0.f, 0.f, 0.f}, poff[4] = {0.f, 0.f, 0.f, 0.f};  // tile t-1 (uint8 docs)
  // Tile `tile` from ring slot T. Its slot's refill (tile + P) is issued
  // after the MFMAs have taken the operands (so they need no copy of their
  // own): REFILL_ANY whether or not that tile exists (past the doc it reads
  // zeros), REFILL_IF only if it does, REFILL_NONE not at all.
  enum { REFILL_NONE, REFILL_IF, REFILL_ANY };
  auto process = [&](auto mode_tag, auto sm_tag, Tile<KIND, KSW>& T, int tile) __attribute__((always_inline)) {
    constexpr int MODE = decltype(mode_tag)::value;
    constexpr bool SM = decltype(sm_tag)::value;  // this wave loads scales / mins
    u32x4_t af[KSW];
#pragma unroll
    for (int t = 0; t < KSW; ++t) {
      af[t] = tile_operand<KIND, KSW>(T, t);
      if constexpr (KMASK && !U8) {
        if (has_partial && t == tp) af[t] &= pmask;
      }
    }
    float sc[4] = {0.f, 0.f, 0.f, 0.f}, off[4] = {0.f, 0.f, 0.f, 0.f};
    if constexpr (U8 && SM) {
#pragma unroll
      for (int r = 0; r < 4; ++r) tile_affine(T.s, T.m, r, sc[r], off[r]);
    }
    f32x4_t acc[NQB];
#pragma unroll
    for (int nb = 0; nb < NQB; ++nb) {
      acc[nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < KSW; ++t) acc[nb] = mfma16x16x32<BF>(af[t], qf[nb][t], acc[nb]);
    }
    if constexpr (MODE == REFILL_ANY) load_tile<KIND, KSW, VEC, SM, C16>(T, dr, tile + P, c, g, koff);
    if constexpr (MODE == REFILL_IF) {
      if (tile + P < ntiles) load_tile<KIND, KSW, VEC, SM, C16>(T, dr, tile + P, c, g, koff);
    }
    // The first half of the query blocks finished first: store them, then
    // reduce the previous tile while the second half runs.
    constexpr int H = NQB / 2;
#pragma unroll
    for (int nb = 0; nb < H; ++nb) part[tile & 1][wave][nb][lane] = acc[nb];
    if (tile > 0) reduce_tile(tile - 1, psc, poff);
#pragma unroll
    for (int nb = H; nb < NQB; ++nb) part[tile & 1][wave][nb][lane] = acc[nb];
    if constexpr (U8) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        psc[r] = sc[r];
        poff[r] = off[r];
      }
    }
    __syncthreads();
  };
  using RefillNone = std::integral_constant<int, REFILL_NONE>;
  using RefillIf = std::integral_constant<int, REFILL_IF>;
  using RefillAny = std::integral_constant<int, REFILL_ANY>;
  // ntiles is uniform over the workgroup, so the barriers inside are safe.
  // FIXED: a fixed load pattern. The first P tiles are loaded, and every group
  // of P tiles that has a successor refills all P slots; tiles past the doc
  // read zeros from outside its buffer range without touching memory. The
  // compiler's wait before each tile then counts the tiles still in flight
  // behind it, where a conditional load makes it wait for all of them (a full
  // drain every other tile at P = 2). The largest masked instances keep
  // conditional loads (the fixed pattern's extra registers spill there), and
  // so do uint8 rows without 16-byte alignment (one wave per SIMD fewer).
  constexpr bool FIXED = VEC && !(KMASK && (NQB * KSW >= 32 || KSW >= 16));
  if constexpr (FIXED) {
    // uint8 docs: only the owner waves apply the affine epilogue, so only they
    // load the tiles' scales and mins; the others run a copy of the loop
    // without those loads (same tiles and barriers).
    auto run = [&](auto sm_tag) __attribute__((always_inline)) {
      constexpr bool SM = decltype(sm_tag)::value;
#pragma unroll
      for (int s = 0; s < P; ++s) load_tile<KIND, KSW, VEC, SM, C16>(buf[s], dr, s, c, g, koff);
      int i0 = 0;
      for (; i0 + P < ntiles; i0 += P) {
#pragma unroll
        for (int s = 0; s < P; ++s) process(RefillAny{}, sm_tag, buf[s], i0 + s);
      }
#pragma unroll
      for (int s = 0; s < P; ++s)
        if (i0 + s < ntiles) process(RefillNone{}, sm_tag, buf[s], i0 + s);
    };
    if constexpr (U8) {
      if (owner) {
        run(std::true_type{});
      } else {
        run(std::false_type{});
      }
    } else {
      run(std::true_type{});
    }
  } else {
#pragma unroll
    for (int s = 0; s < P; ++s)
      if (s < ntiles) load_tile<KIND, KSW, VEC, true, C16>(buf[s], dr, s, c, g, koff);
    for (int i0 = 0; i0 < ntiles; i0 += P) {
#pragma unroll
      for (int s = 0; s < P; ++s)
        if (i0 + s < ntiles) process(RefillIf{}, std::true_type{}, buf[s], i0 + s);
    }
  }
  if (ntiles > 0) reduce_tile(ntiles - 1, psc, poff);

  // ---- per query token: merge row groups, then sum the pass ----
  if (owner) {
    float v = m;
    int ix = mi;
    if constexpr (ARGMAX) {
      argmax_over_groups(v, ix);
    } else {
      v = max_over_groups(v);
    }
    if (g == 0) {
      red_m[wave * 16 + c] = v;
      if constexpr (ARGMAX) red_i[wave * 16 + c] = ix;
    }
  }
  __syncthreads();
  if (wave == 0) {
    float partsum = 0.f;
    for (int r = lane; r < QROWS; r += 64) {
      const int q = q0 + r;
      if (q < a.Lq) {
        partsum += red_m[r];
        if constexpr (ARGMAX) a.argmax[(int64_t)item * a.Lq + q] = red_i[r];
      }
    }
    const float total = wave_sum(partsum);
    if (lane == 0) {
      if (npass == 1) {
        store_score(a, qi, b, total);
      } else {
        a.partial[(int64_t)pass * a.Nq * a.B + item] = total;
      }
    }
  }
  if (!PERSIST) break;
  b += gridDim.x;
  if (b >= a.B) break;
  __syncthreads();  // red_m / red_i are rewritten for the next doc
  }
}

__global__ void __launch_bounds__(256) splitd_sum_passes_kernel(FwdArgs a, int npass) {
  const int64_t items = (int64_t)a.Nq * a.B;
  const int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= items) return;
  float s = 0.f;
  for (int p = 0; p < npass; ++p) s += a.partial[(int64_t)p * items + item];
  const int64_t qi = item / a.B, b = item - qi * a.B;
  store_score(a, qi, b, s);
}

template <int KIND, int NQB, int KSW, bool KMASK, bool ARGMAX, bool VEC = true, bool C16 = VEC>
hipError_t launch_one(const FwdArgs& a, hipStream_t s) {
  constexpr int QROWS = NQB * 16;
  const int npass = (a.Lq + QROWS - 1) / QROWS;
  const int64_t items = (int64_t)a.Nq * a.B;
  // One query in one pass: resident workgroups walk the docs with the query
  // slice loaded once (config 5: 201 -> 189 us), for query tiles of 64 rows
  // or more with aligned rows; smaller tiles gain nothing against more
  // workgroups per CU, and the masked 128-row instances would spill.
  if constexpr (NQB >= 4 && VEC && !(KMASK && NQB * KSW >= 32)) {
   if (npass == 1 && a.Nq == 1 && !a.qidx) {
    // resident workgroups per CU x CUs (cached per device)
    static int cache[64] = {0};
    int dev = 0;
    int n = 0;
    if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64) n = cache[dev];
    if (n == 0) {
      int cus = 0, per = 0;
      if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
              &per, reinterpret_cast<const void*>(splitd_fwd_kernel<KIND, NQB, KSW, KMASK, ARGMAX, VEC, true>), 512,
              0) != hipSuccess || per <= 0)
        per = 1;
      n = cus * per;
      if (dev >= 0 && dev < 64) cache[dev] = n;
    }
    const int64_t grid = a.B < n ? a.B : n;
    hipLaunchKernelGGL((splitd_fwd_kernel<KIND, NQB, KSW, KMASK, ARGMAX, VEC, true>), dim3((unsigned)grid), dim3(512),
                       0, s, a);
    return hipGetLastError();
   }
  }
  const int64_t U = (a.shared_docs && a.Nq > 1 ? a.Nq : 1) * (int64_t)npass;
  const int64_t nslots = a.shared_docs && a.Nq > 1 ? a.B : items;
  const int64_t grid = U > 1 ? ((nslots + 7) / 8) * 8 * U : items;
  hipLaunchKernelGGL((splitd_fwd_kernel<KIND, NQB, KSW, KMASK, ARGMAX, VEC, false, C16>), dim3((unsigned)grid),
                     dim3(512), 0, s, a);
  if (npass > 1) {
    hipLaunchKernelGGL(splitd_sum_passes_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, s, a,
                       npass);
  }
  return hipGetLastError();
}

template <int KIND, int NQB, int KSW>
hipError_t dispatch_flags(const FwdArgs& a, bool am, hipStream_t s) {
  const bool kmask = a.d != 32 * KSW * kSplitWaves;
  if constexpr (KIND == KIND_U8) {
    (void)am;
    if (a.vec & 1) {
      return kmask ? launch_one<KIND, NQB, KSW, true, false, true>(a, s)
                   : launch_one<KIND, NQB, KSW, false, false, true>(a, s);
    }
    // without the vector path: 16-byte code loads when the code rows allow (bit 1)
    if (a.vec & 2) {
      return kmask ? launch_one<KIND, NQB, KSW, true, false, false, true>(a, s)
                   : launch_one<KIND, NQB, KSW, false, false, false, true>(a, s);
    }
    return kmask ? launch_one<KIND, NQB, KSW, true, false, false>(a, s)
                 : launch_one<KIND, NQB, KSW, false, false, false>(a, s);
  } else {
    if (kmask) return am ? launch_one<KIND, NQB, KSW, true, true>(a, s) : launch_one<KIND, NQB, KSW, true, false>(a, s);
    return am ? launch_one<KIND, NQB, KSW, false, true>(a, s) : launch_one<KIND, NQB, KSW, false, false>(a, s);
  }
}

template <int KIND, int KSW>
hipError_t dispatch_nqb(const FwdArgs& a, bool am, hipStream_t s) {
  switch (splitd_fwd_nqb(a.Lq, a.d)) {
    case 1: return dispatch_flags<KIND, 1, KSW>(a, am, s);
    case 2:
      if constexpr (KSW <= 8) return dispatch_flags<KIND, 2, KSW>(a, am, s);
      return hipErrorInvalidValue;
    case 4:
      if constexpr (KSW <= 4) return dispatch_flags<KIND, 4, KSW>(a, am, s);
      return hipErrorInvalidValue;
    default:
      if constexpr (KSW <= 4) return dispatch_flags<KIND, 8, KSW>(a, am, s);
      return hipErrorInvalidValue;
  }
}

template <int KIND>
hipError_t dispatch_ksw(const FwdArgs& a, bool am, hipStream_t s) {
  switch (splitd_fwd_ksw(a.d)) {
    case 2: return dispatch_nqb<KIND, 2>(a, am, s);
    case 4: return dispatch_nqb<KIND, 4>(a, am, s);
    case 8: return dispatch_nqb<KIND, 8>(a, am, s);
    case 16: return dispatch_nqb<KIND, 16>(a, am, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

bool splitd_fwd_supported(int d) { return d > 256 && d <= 4096; }

// k-steps per wave: the eight slices of 32*KSW cover d.
int splitd_fwd_ksw(int d) {
  const int steps = (d + 31) / 32;
  const int ksw = (steps + kSplitWaves - 1) / kSplitWaves;
  return ksw <= 2 ? 2 : ksw <= 4 ? 4 : ksw <= 8 ? 8 : 16;
}

// Query blocks per pass, capped so the query slice stays within 128 VGPRs
// (64 at KSW >= 8, where the deeper doc fragments need the rest: at KSW = 16
// one block's slice and two 16-step tiles take 192 of the 256).
int splitd_fwd_nqb(int Lq, int d) {
  const int need = (Lq + 15) / 16;
  const int ksw = splitd_fwd_ksw(d);
  const int cap = ksw >= 16 ? 1 : ksw >= 8 ? 2 : 32 / ksw;
  const int nqb = need <= 1 ? 1 : need <= 2 ? 2 : need <= 4 ? 4 : 8;
  return nqb < cap ? nqb : cap;
}

int splitd_fwd_passes(int Lq, int d) {
  const int rows = 16 * splitd_fwd_nqb(Lq, d);
  return (Lq + rows - 1) / rows;
}

hipError_t launch_splitd_fwd(int kind, const FwdArgs& a, bool with_argmax, hipStream_t s) {
  switch (kind) {
    case KIND_F16: return dispatch_ksw<KIND_F16>(a, with_argmax, s);
    case KIND_BF16: return dispatch_ksw<KIND_BF16>(a, with_argmax, s);
    case KIND_U8: return dispatch_ksw<KIND_U8>(a, false, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fmx
