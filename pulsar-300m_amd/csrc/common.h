// Shared device/host helpers for the gfx950 (CDNA4) Pulsar kernels.
//
// Activations and large weights are either fp32 or bf16 ("T" below). bf16 is stored as
// raw uint16 and converted with round-to-nearest-even, the rounding torch uses for
// .to(torch.bfloat16), so intermediate roundings match the reference op by op.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/pulsar_hip.h"

namespace pulsar {

struct bf16 {
  uint16_t u;
};

__host__ __device__ __forceinline__ float bf2f(bf16 v) {
  return __uint_as_float(static_cast<uint32_t>(v.u) << 16);
}

__host__ __device__ __forceinline__ bf16 f2bf(float f) {
  uint32_t x = __float_as_uint(f);
  bf16 r;
  if ((x & 0x7f800000u) == 0x7f800000u && (x & 0x007fffffu)) {
    r.u = 0x7fc0;  // quiet NaN
    return r;
  }
  x += 0x7fffu + ((x >> 16) & 1u);
  r.u = static_cast<uint16_t>(x >> 16);
  return r;
}

template <typename T>
__device__ __forceinline__ float to_f(T v);
template <>
__device__ __forceinline__ float to_f<float>(float v) { return v; }
template <>
__device__ __forceinline__ float to_f<bf16>(bf16 v) { return bf2f(v); }

template <typename T>
__device__ __forceinline__ T from_f(float v);
template <>
__device__ __forceinline__ float from_f<float>(float v) { return v; }
template <>
__device__ __forceinline__ bf16 from_f<bf16>(float v) { return f2bf(v); }

// Round a float through the storage type T (identity for fp32).
template <typename T>
__device__ __forceinline__ float rnd(float v) { return to_f<T>(from_f<T>(v)); }

constexpr int kWave = 64;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// Block-wide sum for blockDim.x a multiple of 64 (<= 1024). `red` needs 16 floats.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < nw; ++i) t += red[i];
  return t;
}

__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float t = -INFINITY;
  for (int i = 0; i < nw; ++i) t = fmaxf(t, red[i]);
  return t;
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

// ---------------------------------------------------------------------------
// Host-side error state (thread local), surfaced through pulsar_last_error().
// ---------------------------------------------------------------------------
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);

}  // namespace pulsar

#define PULSAR_CHECK_HIP(expr)                                                      \
  do {                                                                              \
    hipError_t _e = (expr);                                                         \
    if (_e != hipSuccess)                                                           \
      return ::pulsar::fail(PULSAR_ERR_HIP, std::string(#expr) + ": " + hipGetErrorString(_e)); \
  } while (0)

#define PULSAR_REQUIRE(cond, msg)                                   \
  do {                                                              \
    if (!(cond)) return ::pulsar::fail(PULSAR_ERR_INVALID, (msg));  \
  } while (0)

#define PULSAR_LAUNCH_CHECK()                                                        \
  do {                                                                               \
    hipError_t _e = hipGetLastError();                                               \
    if (_e != hipSuccess)                                                            \
      return ::pulsar::fail(PULSAR_ERR_HIP, std::string("kernel launch: ") + hipGetErrorString(_e)); \
  } while (0)
