// Top-k of score rows: the step after MaxSim scoring. Callers of the
// reference rank its scores right away (torch topk / argsort over
// flash_maxsim's output); this kernel does that selection on the GPU.
//
// Order: scores descending, NaN first (as torch.topk ranks NaN above every
// number), ties to the smaller doc index. Each score becomes a 64-bit key,
//   key = ord(score) << 32 | ~index,
// where ord maps float bits to an unsigned integer in float order (NaN to the
// maximum), so the k largest keys are exactly the k best (score, index) pairs
// and all keys are distinct.
//
// A workgroup of 1024 threads holds a chunk of up to C = 1024*E keys in
// registers and finds its k largest by radix selection: passes over 8-bit
// digits (most significant first) build a 256-bin LDS histogram of the keys
// still matching the selected prefix, and one wave finds the bin that holds
// the k-th largest; selection stops as soon as that bin holds exactly the
// keys still needed. Keys are distinct, so the selected set is exactly the
// keys whose leading bits are >= the final prefix. A block scan compacts them
// into LDS. Intermediate levels write the chunk's k keys (unordered); the last
// level ranks them by counting (rank = keys greater than it; up to 1024 keys)
// or sorts them (bitonic, in LDS; k up to 8192) and writes values and indices
// best first. Rows longer than C run several levels, each C / k times shorter.
#include "fmx_device.h"
#include "fmx_kernels.h"

namespace fmx {
namespace {

// Inverse of ord_bits for numbers (NaN maps back to a canonical NaN, -0 to +0).
__device__ __forceinline__ float float_of(uint32_t o) {
  return __builtin_bit_cast(float, (o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}

// Float bits to an unsigned integer in float order: every NaN to the maximum
// (NaN ranks first), -0 to +0's value.
__device__ __forceinline__ uint32_t ord_bits(uint32_t u) {
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0xffffffffu;  // NaN ranks first
  if (u == 0x80000000u) u = 0u;                                // -0 ties with +0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

constexpr int kTopkThreads = 1024;
constexpr int kTopkMaxK = 8192;                  // FMX_MAX_TOPK
constexpr int kTopkCountK = 1024;                // ranked by counting up to this many keys
constexpr int kTopkC = kTopkThreads * 16;       // keys per chunk (16 per thread)
// A row of up to kTopkSmallN keys with k <= kTopkSmallK is selected by one
// 512-thread workgroup on the raw scores (select_small_row): two waves per
// SIMD, each step's latency hidden by the other wave.
constexpr int kTopkSmallThreads = 512;
constexpr int kTopkSmallN = kTopkSmallThreads * 16;
constexpr int kTopkSmallK = 128;

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_or0(int v) {
  // lanes whose source is outside the pattern (or in a masked row) read 0
  return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xf, false);
}

// Inclusive prefix sum over the 64 lanes of a full wave, all on the VALU:
// row_shr 1, 2, 4, 8 within each 16-lane row, then row_bcast:15 (rows 1, 3
// add the last lane of the row below) and row_bcast:31 (rows 2, 3 add lane 31).
__device__ __forceinline__ int wave_incl_scan(int v) {
  v += dpp_or0<0x111, 0xf>(v);
  v += dpp_or0<0x112, 0xf>(v);
  v += dpp_or0<0x114, 0xf>(v);
  v += dpp_or0<0x118, 0xf>(v);
  v += dpp_or0<0x142, 0xa>(v);
  v += dpp_or0<0x143, 0xc>(v);
  return v;
}

template <int NT>
__device__ __forceinline__ int block_exclusive_scan(int v, int* wave_tot, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int inc = wave_incl_scan(v);
  if (lane == 63) wave_tot[wave] = inc;
  __syncthreads();
  if (wave == 0) {
    const int t = lane < NT / 64 ? wave_tot[lane] : 0;
    const int ti = wave_incl_scan(t);
    if (lane < NT / 64) wave_tot[lane] = ti - t;  // exclusive wave offsets
    if (lane == NT / 64 - 1) *total = ti;
  }
  __syncthreads();
  return wave_tot[wave] + inc - v;
}

// min and max of a 32-bit unsigned value over a full wave (every lane gets both).
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ void wave_minmax_u32(uint32_t& mn, uint32_t& mx) {
  uint32_t a, b;
#define FMX_MM_STEP(CTRL)                      \
  a = dpp_u32<CTRL>(mn);                       \
  b = dpp_u32<CTRL>(mx);                       \
  mn = a < mn ? a : mn;                        \
  mx = b > mx ? b : mx;
  FMX_MM_STEP(0xB1)   // quad_perm(1, 0, 3, 2)
  FMX_MM_STEP(0x4E)   // quad_perm(2, 3, 0, 1)
  FMX_MM_STEP(0x141)  // row_half_mirror
  FMX_MM_STEP(0x140)  // row_mirror
#undef FMX_MM_STEP
  uint32_t lo, hi;
  halves16(mn, lo, hi);
  mn = lo < hi ? lo : hi;
  halves16(mx, lo, hi);
  mx = lo > hi ? lo : hi;
  halves32(mn, lo, hi);
  mn = lo < hi ? lo : hi;
  halves32(mx, lo, hi);
  mx = lo > hi ? lo : hi;
}

// Lower bound of the want-th best key's score half (the upper 32 bits) from
// the per-thread maxima m of those halves (0: a thread without keys). At
// least `want` maxima sit in the bin (of a 256-bin histogram over the 8 bits
// below the maxima's common prefix) that holds the want-th largest maximum or
// above it, so at least `want` keys reach that bin's lower edge. 0 when fewer
// than `want` threads hold keys. The largest maximum goes to *bmax.
// PRECLEARED: hist was zeroed before the call (no clearing pass), every wave
// scans the histogram itself (no broadcast of the bin), and the caller passes
// a barrier before it rewrites hist, wlo or whi (none at the end).
template <int NT, bool PRECLEARED = false>
__device__ __forceinline__ uint32_t maxima_bound(uint32_t m, int want, uint32_t* hist, uint64_t* wlo, uint64_t* whi,
                                                 int* bc, uint32_t* bmax = nullptr) {
  const int tid = threadIdx.x, lane = tid & 63;
  uint32_t mn = m == 0u ? 0xffffffffu : m, mx = m;
  wave_minmax_u32(mn, mx);
  if (lane == 0) {
    wlo[tid >> 6] = mn;
    whi[tid >> 6] = mx;
  }
  __syncthreads();
  mn = 0xffffffffu;
  mx = 0u;
  for (int w = 0; w < NT / 64; ++w) {
    mn = (uint32_t)wlo[w] < mn ? (uint32_t)wlo[w] : mn;
    mx = (uint32_t)whi[w] > mx ? (uint32_t)whi[w] : mx;
  }
  if (bmax) *bmax = mx;
  if (mx == 0u) return 0u;  // uniform: no barrier skipped by some threads only
  const int hb = mn == mx ? 8 : 32 - __builtin_clz(mn ^ mx);  // the maxima agree above bit hb
  const int sh = hb < 8 ? 0 : hb - 8;
  if constexpr (!PRECLEARED) {
    if (tid < 256) hist[tid] = 0u;
    __syncthreads();
  }
  if (m != 0u) atomicAdd(&hist[(m >> sh) & 255u], 1u);
  __syncthreads();
  const uint32_t hi = sh + 8 >= 32 ? 0u : (mx >> (sh + 8)) << (sh + 8);
  if constexpr (PRECLEARED) {
    // every wave scans the histogram itself: no broadcast, no further barrier
    uint32_t h[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) h[j] = hist[4 * lane + j];
    const int incl = wave_incl_scan((int)(h[0] + h[1] + h[2] + h[3]));
    uint32_t above = (uint32_t)(__builtin_amdgcn_readlane(incl, 63) - incl);
    int found = -1;
#pragma unroll
    for (int j = 3; j >= 0; --j) {
      if (above < (uint32_t)want && (uint32_t)want <= above + h[j]) found = 4 * lane + j;
      above += h[j];
    }
    const uint64_t who = __builtin_amdgcn_ballot_w64(found >= 0);  // one lane at most
    if (who == 0u) return 0u;
    const int bin = __builtin_amdgcn_readlane(found, __builtin_ctzll(who));
    return hi | ((uint32_t)bin << sh);
  }
  if (tid < 64) {
    // lane l holds bins 4l .. 4l+3; maxima in higher bins = total - inclusive prefix
    uint32_t h[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) h[j] = hist[4 * tid + j];
    const int incl = wave_incl_scan((int)(h[0] + h[1] + h[2] + h[3]));
    uint32_t above = (uint32_t)(__builtin_amdgcn_readlane(incl, 63) - incl);
    if (tid == 0) bc[0] = -1;
#pragma unroll
    for (int j = 3; j >= 0; --j) {
      if (above < (uint32_t)want && (uint32_t)want <= above + h[j]) bc[0] = 4 * tid + j;
      above += h[j];
    }
  }
  __syncthreads();
  const int bin = bc[0];
  __syncthreads();  // bc, hist, wlo and whi are rewritten later
  if (bin < 0) return 0u;
  return hi | ((uint32_t)bin << sh);
}

// Ranks the nsel distinct keys of sel[] (rank = keys greater) and writes the
// best k: values and indices best first (values given) or this chunk's k keys
// to keys_out. G lanes of one wave share a key's count, each comparing it
// against its share of the list in batches of eight 16-byte pairs whose LDS
// reads are all in flight before the first compare. The list is first padded
// with zero keys to a whole number of batches (0 is below every real key, so
// padding never counts); nsel <= kTopkCountK keeps the padded list inside sel.
template <int NT>
__device__ __forceinline__ void rank_and_write(uint64_t* sel, int nsel, int k, const float* scores_row,
                                               float* values_row, int64_t* indices_row, uint64_t* keys_chunk) {
  int G = 1;
  while (2 * G <= 64 && 2 * G * nsel <= NT) G *= 2;  // the groups of G lanes cover nsel in one pass
  const int span = 16 * G;  // keys one batch covers over the G lanes
  const int padded = (nsel + span - 1) / span * span;
  const int tid = threadIdx.x, part = tid & (G - 1);
  for (int t = nsel + tid; t < padded; t += NT) sel[t] = 0;
  __syncthreads();
  const ulonglong2* pairs = reinterpret_cast<const ulonglong2*>(sel);
  for (int j = tid / G; j < nsel; j += NT / G) {  // all G lanes of a group share j
    const uint64_t kv = sel[j];
    int cnt = 0;
    for (int p0 = part; 2 * p0 < padded; p0 += 8 * G) {
      ulonglong2 y[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) y[u] = pairs[p0 + u * G];
#pragma unroll
      for (int u = 0; u < 8; ++u) cnt += (int)(y[u].x > kv) + (int)(y[u].y > kv);
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1)
      if (o < G) cnt += __shfl_xor(cnt, o);
    if (part == 0 && cnt < k) {
      if (values_row) {
        const int64_t idx = (int64_t)(uint32_t)~(uint32_t)kv;  // a real key: a valid index of the row
        // The key's value, or, where the key lost the input's bits (zeros,
        // NaN), the input itself.
        float v = float_of((uint32_t)(kv >> 32));
        if (v == 0.f || v != v) v = scores_row[idx];
        values_row[cnt] = v;
        indices_row[cnt] = idx;
      } else {
        keys_chunk[cnt] = kv;
      }
    }
  }
}

// Selection of one row's k <= kTopkSmallK best scores by the small
// instance, on the raw float bits (slots past the row become -inf): no
// per-key order keys are formed. Each thread's largest score (a NaN-propagating
// maximum, so a NaN anywhere in the row is seen), a bound from those maxima
// (maxima_bound), then candidates and their rank by counting with G lanes
// per candidate. Every step is branch-free VALU arithmetic on the sign of a
// float difference, with +inf taken as the largest finite float (inf - inf
// would be a NaN): x >= T is the clear sign bit of x - T' (T' = T, or -0 for
// T = +0, so that -0 - T' = +0), and y > x the set sign bit of x - y (x and
// y with -0 made +0; the exact difference's sign survives rounding). Values
// that compare equal this way (+inf and the largest float included) collide
// in the rank and send the row to the exact path.
// Candidates are packed by one wave scan and one LDS atomic per wave; a lane
// writes every slot, non-candidates to a spare entry of its own. The rank
// buffer holds -inf past the candidates (x - (-inf) is +inf: never counted).
// Returns false, uniformly and after a barrier, when the row holds a NaN, the
// bound is -inf, there are more than kTopkCountK candidates, or two
// candidates of equal value fall inside the top k (the rank then cannot order
// them by index): the exact path runs instead.
template <int NT, int E>
__device__ bool select_small_row(uint32_t (&raw)[E], int left, int k, float* vrow, int64_t* irow,
                                 uint32_t* hist, uint64_t* wmin, uint64_t* wmax, int* bcast, uint32_t* nsel_lds) {
  constexpr int SPARE = kTopkCountK + 64;  // one spare entry per lane
  __shared__ __attribute__((aligned(16))) float rel[SPARE];
  __shared__ uint64_t pr[SPARE];  // index << 32 | score bits
  __shared__ int rk[kTopkCountK];
  __shared__ uint32_t slot[kTopkSmallK];
  __shared__ int flag[2];  // [0]: a NaN in the row, [1]: equal values inside the top k
  const int tid = threadIdx.x, lane = tid & 63;
#pragma unroll
  for (int t = tid; t < kTopkCountK; t += NT) rel[t] = -__builtin_inff();
  if (tid < 256) hist[tid] = 0u;
  if (tid < kTopkSmallK) slot[tid] = 0u;
  if (tid < 2) flag[tid] = 0;
  // (the LDS set-up above overlaps the loads; the first use of a score is here)
  // slots past the row become -inf (the exact path masks them by index)
#pragma unroll
  for (int e = 0; e < E; ++e)
    if (e * NT + tid >= left) raw[e] = 0xff800000u;
  const int want = left < k ? left : k;
  float m = -__builtin_inff();
#pragma unroll
  for (int e = 0; e < E; ++e) m = __builtin_elementwise_maximum(m, __builtin_bit_cast(float, raw[e]));
  if (__builtin_amdgcn_ballot_w64(m != m) != 0 && lane == 0) flag[0] = 1;
  // a thread without any key of the row holds no maximum (0)
  const uint32_t mo = tid < left ? ord_bits(__builtin_bit_cast(uint32_t, m)) : 0u;
  const uint32_t tau = maxima_bound<NT, true>(mo, want, hist, wmin, wmax, bcast);
  // Keys whose order reaches the bound are the scores >= T. A bound at or
  // below the order of -inf would admit the -inf that stands in for slots
  // past the row: such rows take the exact path.
  if (tau <= 0x007fffffu) return false;  // uniform
  constexpr float kBig = 3.40282347e38f;  // the largest finite float
  const float T = __builtin_fminf(float_of(tau), kBig);
  const float Tm = T == 0.f ? -0.f : T;
  uint32_t out = 0u;  // slots that are not candidates
#pragma unroll
  for (int e = 0; e < E; ++e)
    out += __builtin_bit_cast(uint32_t, __builtin_fminf(__builtin_bit_cast(float, raw[e]), kBig) - Tm) >> 31;
  const int cnt = E - (int)out;
  const int inc = wave_incl_scan(cnt);
  uint32_t base = 0u;
  if (lane == 63) base = atomicAdd(nsel_lds, (uint32_t)inc);
  uint32_t pos = __builtin_amdgcn_readlane(base, 63) + (uint32_t)(inc - cnt);
  const uint32_t spare = kTopkCountK + lane;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float x = __builtin_fminf(__builtin_bit_cast(float, raw[e]), kBig);
    const uint32_t no = __builtin_bit_cast(uint32_t, x - Tm) >> 31;
    const uint32_t p = pos < (uint32_t)(kTopkCountK - 1) ? pos : (uint32_t)(kTopkCountK - 1);
    const uint32_t a = no ? spare : p;  // branch-free: non-candidates write a spare entry
    pr[a] = ((uint64_t)(uint32_t)(e * NT + tid) << 32) | raw[e];
    rel[a] = x + 0.f;  // -0 becomes +0
    pos += 1u - no;
  }
  __syncthreads();
  const int nc = (int)*nsel_lds;
  if (flag[0] != 0 || nc > kTopkCountK || nc < want) return false;

  constexpr int RB = 8;                           // 16-byte reads per lane per batch
  constexpr int GMAX = kTopkCountK / (4 * RB);    // one batch of GMAX lanes spans the buffer
  // the largest power of two G <= GMAX with G * nc <= NT: the groups of G lanes cover nc in one pass
  const int fit = NT / (nc > 0 ? nc : 1);
  const int G = fit >= GMAX ? GMAX : fit <= 1 ? 1 : 1 << (31 - __builtin_clz(fit));
  const int span = 4 * RB * G;                       // divides kTopkCountK
  const int padded = (nc + span - 1) / span * span;  // <= kTopkCountK, as nc is
  const int part = tid & (G - 1);
  const f32x4_t* r4 = reinterpret_cast<const f32x4_t*>(rel);
  for (int j = tid / G; j < nc; j += NT / G) {  // all G lanes of a group share j
    const float xj = rel[j];
    uint32_t c = 0u;
    for (int q0 = part; 4 * q0 < padded; q0 += RB * G) {
      f32x4_t y[RB];
#pragma unroll
      for (int u = 0; u < RB; ++u) y[u] = r4[q0 + u * G];
#pragma unroll
      for (int u = 0; u < RB; ++u)
#pragma unroll
        for (int v = 0; v < 4; ++v) c += __builtin_bit_cast(uint32_t, xj - y[u][v]) >> 31;
    }
    int cc = (int)c;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1)
      if (o < G) cc += __shfl_xor(cc, o);
    if (part == 0) {
      rk[j] = cc;
      if (cc < k && atomicAdd(&slot[cc], 1u) != 0u) flag[1] = 1;
    }
  }
  __syncthreads();
  if (flag[1] != 0) return false;
  for (int t = tid; t < nc; t += NT) {
    const int r = rk[t];
    if (r < k) {
      const uint64_t v = pr[t];
      vrow[r] = __builtin_bit_cast(float, (uint32_t)v);  // the input's own bits (-0 stays -0)
      irow[r] = (int64_t)(v >> 32);
    }
  }
  return true;
}

// grid (chunks, rows). Level 0 (keys_in == null): row r's chunk c covers
// indices [c*C, c*C + C) of scores[r, :n]. Otherwise keys_in[r, :n] (0 = no key).
// Output: the chunk's k best keys to keys_out[r, c*k ...] (0-padded when the
// chunk holds fewer), or, at the last level, values and indices, best first.
// kTopkE: keys per thread (the chunk is 1024 * kTopkE keys); MAXK: capacity of
// the selection buffer, kTopkCountK or kTopkMaxK (k above kTopkCountK).
template <int NT, int kTopkE, int MAXK, bool SMALL = false>
__global__ void __launch_bounds__(NT) topk_level_kernel(const float* scores, int64_t s_stride,
                                                                 const uint64_t* keys_in, int64_t n, int k,
                                                                 uint64_t* keys_out, float* values,
                                                                 int64_t* indices, int64_t o_stride) {
  __shared__ uint32_t hist[256];
  __shared__ __attribute__((aligned(16))) uint64_t sel[MAXK];
  __shared__ int wave_tot[NT / 64];
  __shared__ uint64_t wmin[NT / 64], wmax[NT / 64];
  __shared__ int bcast[4];
  __shared__ uint32_t nsel_lds;  // candidates packed so far (cleared before the first barrier)
  const int64_t row = blockIdx.y;
  const int64_t c0 = (int64_t)blockIdx.x * (NT * kTopkE);
  const int tid = threadIdx.x;
  if (tid == 0) nsel_lds = 0u;

  // Every load is issued unconditionally, through a buffer resource over the
  // chunk (reads past the row return 0 without touching memory, then count as
  // no key), so all of a thread's loads are in flight together at one
  // instruction each; a load under a per-key branch waited for each in turn.
  const int64_t left64 = n - c0;
  const int left = left64 < (int64_t)NT * kTopkE ? (int)left64 : NT * kTopkE;  // keys of this chunk
  uint64_t key[kTopkE];
  int valid = 0;
  if (keys_in) {
    const rsrc_t r = make_rsrc(keys_in + row * n + c0, (uint32_t)left * 8u);
#pragma unroll
    for (int e = 0; e < kTopkE; ++e) {
      const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(r, (uint32_t)(tid + e * NT) * 8u, 0, 0);
      key[e] = ((uint64_t)v[1] << 32) | v[0];
    }
#pragma unroll
    for (int e = 0; e < kTopkE; ++e) valid += key[e] != 0;
  } else {
    const rsrc_t r = make_rsrc(scores + row * s_stride + c0, (uint32_t)left * 4u);
    uint32_t raw[kTopkE];
#pragma unroll
    for (int e = 0; e < kTopkE; ++e)  // constant offsets fold into the instructions' offset fields
      raw[e] = __builtin_amdgcn_raw_buffer_load_b32(r, (uint32_t)(tid + e * NT) * 4u, 0, 0);
    if constexpr (SMALL) {
      // the small instances run single-chunk rows at the last level only
      if (select_small_row<NT, kTopkE>(raw, left, k, values + row * o_stride, indices + row * o_stride, hist,
                                       wmin, wmax, bcast, &nsel_lds))
        return;
      __syncthreads();  // the exact path below packs its candidates again
      if (tid == 0) nsel_lds = 0u;
    }
    const uint32_t nidx = ~(uint32_t)(c0 + tid);  // ~index of key 0; key e: nidx - e * NT
#pragma unroll
    for (int e = 0; e < kTopkE; ++e) {
      const uint64_t kv = ((uint64_t)ord_bits(raw[e]) << 32) | (nidx - (uint32_t)(e * NT));
      key[e] = e * NT + tid < left ? kv : 0;
    }
  }
  // keys present in this chunk (0-keys are padding from an earlier level; at
  // level 0 every index below n is a key, none of them 0, so no count is needed)
  int total;
  if (!keys_in) {
    total = left;
  } else {
    int* tot = &bcast[3];
    block_exclusive_scan<NT>(valid, wave_tot, tot);
    total = *tot;
  }
  const int want = total < k ? total : k;
  const int64_t nout = (int64_t)gridDim.x * k;  // keys per row of the next level

  // ---- candidates: keys whose score half reaches a bound of the want-th ----
  // The bound comes from the per-thread maxima (maxima_bound). For the
  // scores of one query the candidates are a small multiple of want; when
  // they fit the selection buffer they are ranked directly and the radix
  // passes below are skipped (a row of 5000 scores, k = 100: loads, bound,
  // packing and ranking take about 5.7 us of wall clock inside the kernel).
  if (want > 0 && want < total) {
    uint32_t m = 0u;
#pragma unroll
    for (int e = 0; e < kTopkE; ++e) {
      const uint32_t h = (uint32_t)(key[e] >> 32);
      if (key[e] != 0 && h > m) m = h;
    }
    const uint32_t tau = maxima_bound<NT>(m, want, hist, wmin, wmax, bcast);
    int c = 0;
#pragma unroll
    for (int e = 0; e < kTopkE; ++e) c += key[e] != 0 && (uint32_t)(key[e] >> 32) >= tau;
    // Each wave reserves its candidates' slots with one LDS atomic (slot order
    // does not matter: ranking orders by key), one barrier instead of a block scan.
    const int inc = wave_incl_scan(c);
    int base = 0;
    if ((tid & 63) == 63) base = (int)atomicAdd(&nsel_lds, (uint32_t)inc);
    int pos = __builtin_amdgcn_readlane(base, 63) + inc - c;
#pragma unroll
    for (int e = 0; e < kTopkE; ++e) {
      if (key[e] != 0 && (uint32_t)(key[e] >> 32) >= tau) {
        if (pos < kTopkCountK) sel[pos] = key[e];
        ++pos;
      }
    }
    __syncthreads();
    const int nc = (int)nsel_lds;
    if (nc <= kTopkCountK) {  // uniform
      rank_and_write<NT>(sel, nc, want, values ? scores + row * s_stride : nullptr,
                     values ? values + row * o_stride : nullptr, values ? indices + row * o_stride : nullptr,
                     values ? nullptr : keys_out + row * nout + (int64_t)blockIdx.x * k);
      return;
    }
    __syncthreads();  // heavy ties: the radix passes below reuse the buffers
  }

  // ---- radix selection of the `want` largest keys ----
  // Digits start at the highest bit where the chunk's keys differ (block min
  // and max): scores of one query sit in a narrow range, and digits over their
  // common leading bits would put every key in one histogram bin.
  uint64_t prefix = 0;
  int shift = 64, krem = want;
  if (want > 0 && want < total) {
    // Min and max of the score halves (ord, the upper 32 bits of the keys)
    // first: when they differ, the smallest and largest keys differ at the
    // same highest bit. Keys of equal ord need the full 64-bit min and max.
    uint32_t hmn = 0xffffffffu, hmx = 0u;
#pragma unroll
    for (int e = 0; e < kTopkE; ++e) {
      if (key[e] != 0) {
        const uint32_t h = (uint32_t)(key[e] >> 32);
        hmn = h < hmn ? h : hmn;
        hmx = h > hmx ? h : hmx;
      }
    }
    wave_minmax_u32(hmn, hmx);
    if ((tid & 63) == 0) {
      wmin[tid >> 6] = hmn;
      wmax[tid >> 6] = hmx;
    }
    __syncthreads();
    hmn = (uint32_t)wmin[0];
    hmx = (uint32_t)wmax[0];
    for (int w = 1; w < NT / 64; ++w) {
      hmn = (uint32_t)wmin[w] < hmn ? (uint32_t)wmin[w] : hmn;
      hmx = (uint32_t)wmax[w] > hmx ? (uint32_t)wmax[w] : hmx;
    }
    uint64_t mn, mx;
    if (hmn != hmx) {
      mn = (uint64_t)hmn << 32;
      mx = (uint64_t)hmx << 32;
    } else {
      mn = ~(uint64_t)0;
      mx = 0;
#pragma unroll
      for (int e = 0; e < kTopkE; ++e) {
        if (key[e] != 0) {
          mn = key[e] < mn ? key[e] : mn;
          mx = key[e] > mx ? key[e] : mx;
        }
      }
#pragma unroll
      for (int s = 1; s < 64; s <<= 1) {
        const uint64_t omn = __shfl_xor(mn, s), omx = __shfl_xor(mx, s);
        mn = omn < mn ? omn : mn;
        mx = omx > mx ? omx : mx;
      }
      __syncthreads();  // every thread has read the 32-bit wave results
      if ((tid & 63) == 0) {
        wmin[tid >> 6] = mn;
        wmax[tid >> 6] = mx;
      }
      __syncthreads();
      mn = wmin[0];
      mx = wmax[0];
      for (int w = 1; w < NT / 64; ++w) {
        mn = wmin[w] < mn ? wmin[w] : mn;
        mx = wmax[w] > mx ? wmax[w] : mx;
      }
    }
    shift = 64 - __builtin_clzll(mn ^ mx);  // keys differ only below bit `shift` (mn != mx)
    prefix = shift == 64 ? 0 : mx >> shift;
  } else {
    krem = 0;  // nothing to choose: all or none of the keys
  }
  while (krem > 0 && shift > 0) {
    const int dbits = shift < 8 ? shift : 8;
    const int nshift = shift - dbits;
    if (tid < 256) hist[tid] = 0u;
    __syncthreads();
#pragma unroll
    for (int e = 0; e < kTopkE; ++e) {
      const uint64_t kv = key[e];
      if (kv != 0 && (shift == 64 || (kv >> shift) == prefix))
        atomicAdd(&hist[(uint32_t)(kv >> nshift) & ((1u << dbits) - 1u)], 1u);
    }
    __syncthreads();
    if (tid < 64) {
      // lane l holds bins 4l .. 4l+3; suffix sums from the top bin down
      uint32_t h[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) h[j] = hist[4 * tid + j];
      const uint32_t lane_tot = h[0] + h[1] + h[2] + h[3];
      // keys in bins of higher lanes: the total minus the inclusive prefix
      const int incl = wave_incl_scan((int)lane_tot);
      const uint32_t all = (uint32_t)__builtin_amdgcn_readlane(incl, 63);
      uint32_t above = all - (uint32_t)incl;
#pragma unroll
      for (int j = 3; j >= 0; --j) {
        if (above < (uint32_t)krem && (uint32_t)krem <= above + h[j]) {
          bcast[0] = 4 * tid + j;
          bcast[1] = krem - (int)above;       // still needed from this bin
          bcast[2] = (int)h[j];
        }
        above += h[j];
      }
    }
    __syncthreads();
    const int digit = bcast[0], need = bcast[1], inbin = bcast[2];
    __syncthreads();  // bcast is rewritten by the next pass
    prefix = (shift == 64 ? 0 : prefix << dbits) | (uint64_t)digit;
    shift = nshift;
    krem = need;
    if (inbin == need) break;  // every key of this bin is selected
  }

  // ---- compaction: keys whose leading (64 - shift) bits are >= prefix ----
  // (all keys when want == total, none when want == 0)
  int mine = 0;
#pragma unroll
  for (int e = 0; e < kTopkE; ++e) {
    const uint64_t kv = key[e];
    mine += kv != 0 && want > 0 && (shift == 64 ? true : (kv >> shift) >= prefix);
  }
  int nsel;
  int pos = block_exclusive_scan<NT>(mine, wave_tot, &bcast[3]);
  nsel = bcast[3];
#pragma unroll
  for (int e = 0; e < kTopkE; ++e) {
    const uint64_t kv = key[e];
    if (kv != 0 && want > 0 && (shift == 64 ? true : (kv >> shift) >= prefix)) {
      if (pos < MAXK) sel[pos] = kv;
      ++pos;
    }
  }
  if (nsel > want) nsel = want;  // exactly `want` by construction; never past sel
  __syncthreads();

  if (values && (MAXK <= kTopkCountK || nsel <= kTopkCountK)) {
    rank_and_write<NT>(sel, nsel, k, scores + row * s_stride, values + row * o_stride, indices + row * o_stride,
                   nullptr);
  } else if (values) {
    // More keys than ranking by counting handles in time (O(n^2)): a bitonic
    // sort of the selection, descending, padded with 0 keys (which sort last)
    // to a power of two, then the best k in order.
    if constexpr (MAXK > kTopkCountK) {
      int np = 1;
      while (np < nsel) np <<= 1;
      for (int t = nsel + tid; t < np; t += NT) sel[t] = 0;
      __syncthreads();
      for (int size = 2; size <= np; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
          for (int i = tid; i < np / 2; i += NT) {
            const int lo = 2 * i - (i & (stride - 1)), hi = lo + stride;
            const bool desc = (lo & size) == 0;  // every merge of the last size is descending
            const uint64_t x = sel[lo], y = sel[hi];
            if ((x < y) == desc) {
              sel[lo] = y;
              sel[hi] = x;
            }
          }
          __syncthreads();
        }
      }
      const float* scores_row = scores + row * s_stride;
      for (int t = tid; t < nsel && t < k; t += NT) {
        const uint64_t kv = sel[t];
        const int64_t idx = (int64_t)(uint32_t)~(uint32_t)kv;
        float v = float_of((uint32_t)(kv >> 32));
        if (v == 0.f || v != v) v = scores_row[idx];  // as rank_and_write
        values[row * o_stride + t] = v;
        indices[row * o_stride + t] = idx;
      }
    }
  } else {
    for (int t = tid; t < k; t += NT)
      keys_out[row * nout + (int64_t)blockIdx.x * k + t] = t < nsel ? sel[t] : 0;
  }
}

template <int MAXK>
hipError_t run_levels(const TopkArgs& a, hipStream_t s) {
  int64_t n = a.B;
  const uint64_t* in = nullptr;
  uint64_t* bufs[2] = {a.ws, a.ws + topk_ws_keys(a.Nq, a.B, a.k, kTopkC) / 2};
  int which = 0;
  while (true) {
    const int64_t chunks = (n + kTopkC - 1) / kTopkC;
    const bool last = chunks == 1;
    if (chunks > 0x7fffffff || a.Nq > 65535) return hipErrorInvalidValue;
    uint64_t* out = last ? nullptr : bufs[which];
    // a single chunk holds no more keys per thread than the row needs
    bool small = false;
    if constexpr (MAXK == kTopkCountK) small = last && n <= kTopkSmallN && a.k <= kTopkSmallK;
    if (small) {
      if constexpr (MAXK == kTopkCountK) {
        constexpr int T = kTopkSmallThreads;
        auto kern = n <= 8 * T ? topk_level_kernel<T, 8, MAXK, true>
                  : n <= 10 * T ? topk_level_kernel<T, 10, MAXK, true>
                  : n <= 12 * T ? topk_level_kernel<T, 12, MAXK, true> : topk_level_kernel<T, 16, MAXK, true>;
        hipLaunchKernelGGL(kern, dim3(1u, (unsigned)a.Nq), dim3(T), 0, s, a.scores, a.s_stride, in, n, a.k,
                           nullptr, a.values, a.indices, a.o_stride);
      }
    } else {
      constexpr int T = kTopkThreads;
      auto kern = n <= 4 * T ? topk_level_kernel<T, 4, MAXK>
                : n <= 8 * T ? topk_level_kernel<T, 8, MAXK> : topk_level_kernel<T, 16, MAXK>;
      hipLaunchKernelGGL(kern, dim3((unsigned)chunks, (unsigned)a.Nq), dim3(T), 0, s, a.scores, a.s_stride, in, n,
                         a.k, out, last ? a.values : nullptr, last ? a.indices : nullptr, a.o_stride);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || last) return e;
    in = out;
    n = chunks * a.k;
    which ^= 1;
  }
}

}  // namespace

int topk_chunk(int k) {
  (void)k;
  return kTopkC;
}

// Keys of both ping-pong buffers: level 1 holds ceil(B / C) * k keys per row,
// every later level fewer.
int64_t topk_ws_keys(int64_t Nq, int64_t B, int64_t k, int64_t C) {
  const int64_t chunks = (B + C - 1) / C;
  if (chunks <= 1) return 0;
  return 2 * Nq * chunks * k;
}

// k up to kTopkCountK keeps the 8 KB selection buffer; larger k the 64 KB one.
hipError_t launch_topk(const TopkArgs& a, hipStream_t s) {
  return a.k <= kTopkCountK ? run_levels<kTopkCountK>(a, s) : run_levels<kTopkMaxK>(a, s);
}

}  // namespace fmx
