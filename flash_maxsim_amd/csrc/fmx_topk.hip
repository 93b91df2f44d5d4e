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
// A workgroup of 1024 threads loads a chunk of C keys into LDS, bitonic-sorts
// it descending and writes its first k keys. Level 0 reads scores; further
// levels read the previous level's keys (C / k times fewer each level) until
// one chunk per row remains, whose workgroup writes values and indices.
#include "fmx_device.h"
#include "fmx_kernels.h"

namespace fmx {
namespace {

__device__ __forceinline__ uint32_t ord_of(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0xffffffffu;  // NaN ranks first
  if (u == 0x80000000u) u = 0u;                                // -0 ties with +0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Descending bitonic sort of C keys in LDS by 1024 threads.
template <int C>
__device__ __forceinline__ void bitonic_desc(uint64_t* keys) {
  for (int size = 2; size <= C; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
#pragma unroll
      for (int p = threadIdx.x; p < C / 2; p += 1024) {
        const int i = 2 * stride * (p / stride) + (p % stride);
        const int j = i + stride;
        const bool desc = (i & size) == 0;  // direction of this bitonic block
        const uint64_t a = keys[i], b = keys[j];
        if ((a < b) == desc) {
          keys[i] = b;
          keys[j] = a;
        }
      }
      __syncthreads();
    }
  }
}

// grid (chunks, rows). Level 0 (keys_in == null): row r's chunk c covers
// indices [c*C, c*C + C) of scores[r, :n]. Otherwise keys_in[r, :n].
// Output: the chunk's top min(k, count) keys to keys_out[r, c*k ...], padded
// with 0 (a key below every real one) up to k; or, at the last level, values
// and indices.
template <int C>
__global__ void __launch_bounds__(1024) topk_level_kernel(const float* scores, int64_t s_stride, const uint64_t* keys_in,
                                                          int64_t n, int k, uint64_t* keys_out, float* values,
                                                          int64_t* indices, int64_t o_stride) {
  __shared__ uint64_t keys[C];
  const int64_t row = blockIdx.y;
  const int64_t c0 = (int64_t)blockIdx.x * C;
  for (int t = threadIdx.x; t < C; t += 1024) {
    const int64_t i = c0 + t;
    uint64_t key = 0;
    if (i < n) {
      if (!keys_in) {
        key = ((uint64_t)ord_of(scores[row * s_stride + i]) << 32) | (uint32_t)~(uint32_t)i;
      } else {
        key = keys_in[row * n + i];
      }
    }
    keys[t] = key;
  }
  __syncthreads();
  bitonic_desc<C>(keys);
  if (values) {  // values re-read by index: the input's exact bits (NaN payloads, signed zeros)
    for (int t = threadIdx.x; t < k; t += 1024) {
      const int64_t idx = (int64_t)(uint32_t)~(uint32_t)keys[t];
      values[row * o_stride + t] = scores[row * s_stride + idx];
      indices[row * o_stride + t] = idx;
    }
  } else {
    const int64_t nout = (int64_t)gridDim.x * k;
    for (int t = threadIdx.x; t < k; t += 1024) keys_out[row * nout + (int64_t)blockIdx.x * k + t] = keys[t];
  }
}

template <int C>
hipError_t run_levels(const TopkArgs& a, hipStream_t s) {
  int64_t n = a.B;
  const uint64_t* in = nullptr;
  uint64_t* bufs[2] = {a.ws, a.ws + topk_ws_keys(a.Nq, a.B, a.k, C) / 2};
  int which = 0;
  bool first = true;
  while (true) {
    const int64_t chunks = (n + C - 1) / C;
    const bool last = chunks == 1;
    if (chunks > 0x7fffffff || a.Nq > 65535) return hipErrorInvalidValue;
    uint64_t* out = last ? nullptr : bufs[which];
    hipLaunchKernelGGL((topk_level_kernel<C>), dim3((unsigned)chunks, (unsigned)a.Nq), dim3(1024), 0, s, a.scores,
                       a.s_stride, first ? nullptr : in, n, a.k, out, last ? a.values : nullptr,
                       last ? a.indices : nullptr, a.o_stride);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || last) return e;
    in = out;
    n = chunks * a.k;
    which ^= 1;
    first = false;
  }
}

}  // namespace

int topk_chunk(int k) { return k <= 512 ? 2048 : 4096; }

// Keys of both ping-pong buffers: level 1 holds ceil(B / C) * k keys per row,
// every later level fewer.
int64_t topk_ws_keys(int64_t Nq, int64_t B, int64_t k, int64_t C) {
  const int64_t chunks = (B + C - 1) / C;
  if (chunks <= 1) return 0;
  return 2 * Nq * chunks * k;
}

hipError_t launch_topk(const TopkArgs& a, hipStream_t s) {
  return topk_chunk(a.k) == 2048 ? run_levels<2048>(a, s) : run_levels<4096>(a, s);
}

}  // namespace fmx
