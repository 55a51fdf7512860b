// Shared device helpers for the gfx950 decode kernels.
//
// bf16 values travel as raw uint16_t bit patterns; arithmetic is fp32 and every rounding
// back to bf16 is an explicit round-to-nearest-even, placed where the reference rounds.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define DF_DEVICE __device__ __forceinline__

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 df_bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float df_f32x4;

namespace df {

constexpr int kWave = 64;

DF_DEVICE float bf2f(uint16_t b) { return __uint_as_float(static_cast<uint32_t>(b) << 16); }

// fp32 -> bf16, round to nearest, ties to even (finite values; NaN stays NaN-shaped).
DF_DEVICE uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// bf16(f) as an fp32 value.
DF_DEVICE float round_bf(float f) { return bf2f(f2bf(f)); }

DF_DEVICE float silu(float x) { return x / (1.0f + expf(-x)); }
DF_DEVICE float sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

// torch.nn.functional.softplus with beta=1, threshold=20.
DF_DEVICE float softplus(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

DF_DEVICE float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

DF_DEVICE float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// Cross-workgroup hand-off without an L2 write-back. On gfx950 each XCD has its own L2, so
// plain stores are not visible to a workgroup on another XCD until a device-scope release
// (buffer_wbl2), which serialises across workgroups (~50 ns each). Hand-off data is instead
// written with system-scope stores (sc0 sc1: write-through to memory) and read with
// system-scope loads (sc0 sc1: miss the caches); `publish_wait` makes the writer's stores
// complete before it signals (the relaxed agent-scope counter RMW that follows).
DF_DEVICE void store_through(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
DF_DEVICE void store_through(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
DF_DEVICE float load_through(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
DF_DEVICE int load_through(const int* p) {
  return __hip_atomic_load(const_cast<int*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
DF_DEVICE void publish_wait() { __builtin_amdgcn_s_waitcnt(0); }
// The "last workgroup merges" count: an agent-scope acquire-release add. The release half
// makes this workgroup's partials (written before the barrier that precedes the call)
// visible device-wide before the count moves; the acquire half, taken by the workgroup
// that sees the final count and passed on to its other threads by the barrier after the
// call, keeps its loads of the other workgroups' partials from returning values older than
// their counts. A relaxed add plus write-through stores is not enough: a partial's store
// can be acknowledged before a load that bypasses the caches sees it, and the merge then
// reads the previous call's value from the reused workspace.
DF_DEVICE int arrive(int* counter) {
  return __hip_atomic_fetch_add(counter, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
}

// Block-wide sum for blockDim.x == 64 * waves; `scratch` holds >= waves floats.
template <int WAVES>
DF_DEVICE float block_sum(float v, float* scratch) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) total += scratch[w];
  return total;
}

}  // namespace df

// Status codes returned by every extern "C" entry point.
enum DfStatus : int {
  DF_OK = 0,
  DF_BAD_ARGUMENT = 1,
  DF_LAUNCH_FAILED = 2,
  DF_WORKSPACE_TOO_SMALL = 3,
};

#define DF_RETURN_LAUNCH_STATUS()                                  \
  do {                                                             \
    hipError_t _e = hipGetLastError();                             \
    return _e == hipSuccess ? DF_OK : DF_LAUNCH_FAILED;            \
  } while (0)
