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

// Round to nearest even. On the device this is gfx950's v_cvt_pk_bf16_f32 (no branches);
// the host form is the same rounding in integer arithmetic.
__host__ __device__ __forceinline__ bf16 f2bf(float f) {
  bf16 r;
#if defined(__HIP_DEVICE_COMPILE__)
  r.u = __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
#else
  uint32_t x = __float_as_uint(f);
  if ((x & 0x7f800000u) == 0x7f800000u && (x & 0x007fffffu)) {
    r.u = 0x7fc0;  // quiet NaN
    return r;
  }
  x += 0x7fffu + ((x >> 16) & 1u);
  r.u = static_cast<uint16_t>(x >> 16);
#endif
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

// Lane exchange through DPP (quad permutes and row rotations stay in the VALU).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float swz_xor16(float v) {  // lane ^ 16 within each 32-lane half
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401f));
}
__device__ __forceinline__ float lane_bcast(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Wave64 all-reduce. The partial sums of the 16-lane rows differ in association from lane
// to lane, so the result is taken from lanes 0 and 32 and broadcast: every lane returns
// the identical value.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_mov<0x124>(v);  // row_ror:4
  v += dpp_mov<0x128>(v);  // row_ror:8
  v += swz_xor16(v);
  return lane_bcast(v, 0) + lane_bcast(v, 32);
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_mov<0xB1>(v));
  v = fmaxf(v, dpp_mov<0x4E>(v));
  v = fmaxf(v, dpp_mov<0x124>(v));
  v = fmaxf(v, dpp_mov<0x128>(v));
  v = fmaxf(v, swz_xor16(v));
  return fmaxf(lane_bcast(v, 0), lane_bcast(v, 32));
}

// Sum over the 16 lanes of each DPP row (lanes 16q..16q+15), broadcast from the row's
// first lane.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_mov<0xB1>(v);
  v += dpp_mov<0x4E>(v);
  v += dpp_mov<0x124>(v);
  v += dpp_mov<0x128>(v);
  return __shfl(v, threadIdx.x & 0x30, kWave);
}

// N contiguous elements (N a multiple of 4) to float, with the widest loads that fit.
template <int N>
__device__ __forceinline__ void ldv(const float* p, float* o) {
#pragma unroll
  for (int i = 0; i < N; i += 4) {
    const float4 v = *reinterpret_cast<const float4*>(p + i);
    o[i] = v.x; o[i + 1] = v.y; o[i + 2] = v.z; o[i + 3] = v.w;
  }
}
// 8 bf16 held in 16 bytes to float.
__device__ __forceinline__ void unpack_bf16x8(const uint4& u, float* o) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    o[2 * j] = __uint_as_float(w[j] << 16);
    o[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
  }
}
template <int N>
__device__ __forceinline__ void ldv(const bf16* p, float* o) {
  if constexpr (N % 8 == 0) {
#pragma unroll
    for (int i = 0; i < N; i += 8) {
      const uint4 u = *reinterpret_cast<const uint4*>(p + i);
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        o[i + 2 * j] = __uint_as_float(w[j] << 16);
        o[i + 2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; i += 4) {
      const uint2 u = *reinterpret_cast<const uint2*>(p + i);
      o[i] = __uint_as_float(u.x << 16);
      o[i + 1] = __uint_as_float(u.x & 0xffff0000u);
      o[i + 2] = __uint_as_float(u.y << 16);
      o[i + 3] = __uint_as_float(u.y & 0xffff0000u);
    }
  }
}
// Store N contiguous values (already representable in the storage type).
template <int N>
__device__ __forceinline__ void stv(float* p, const float* v) {
#pragma unroll
  for (int i = 0; i < N; i += 4)
    *reinterpret_cast<float4*>(p + i) = make_float4(v[i], v[i + 1], v[i + 2], v[i + 3]);
}
template <int N>
__device__ __forceinline__ void stv(bf16* p, const float* v) {
  if constexpr (N % 8 == 0) {
#pragma unroll
    for (int i = 0; i < N; i += 8) {
      uint4 u;
      u.x = (uint32_t)f2bf(v[i]).u | ((uint32_t)f2bf(v[i + 1]).u << 16);
      u.y = (uint32_t)f2bf(v[i + 2]).u | ((uint32_t)f2bf(v[i + 3]).u << 16);
      u.z = (uint32_t)f2bf(v[i + 4]).u | ((uint32_t)f2bf(v[i + 5]).u << 16);
      u.w = (uint32_t)f2bf(v[i + 6]).u | ((uint32_t)f2bf(v[i + 7]).u << 16);
      *reinterpret_cast<uint4*>(p + i) = u;
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; i += 4) {
      uint2 u;
      u.x = (uint32_t)f2bf(v[i]).u | ((uint32_t)f2bf(v[i + 1]).u << 16);
      u.y = (uint32_t)f2bf(v[i + 2]).u | ((uint32_t)f2bf(v[i + 3]).u << 16);
      *reinterpret_cast<uint2*>(p + i) = u;
    }
  }
}

// Address-space pointers of the direct global-to-LDS load builtin.
typedef __attribute__((address_space(3))) void* lds_vptr;
typedef __attribute__((address_space(1))) void* glb_vptr;

// s_waitcnt vmcnt(n) alone (expcnt and lgkmcnt left at their maxima), n <= 63.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// 16 bytes per lane from global memory straight into LDS (global_load_lds_dwordx4): lane l's
// bytes land at lds + 16 l; `lds` must be the same for the whole wave. Issued as inline
// assembly so that the compiler neither waits for it before unrelated LDS reads nor counts
// it: the caller waits with wait_vmcnt (these loads count in vmcnt and complete in order)
// and publishes the data to the other waves with lds_barrier.
__device__ __forceinline__ void load_lds16(const void* g, void* lds) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_vptr)lds)));
  // one wait state between the M0 write and the load that reads it
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(m0), "v"(g)
               : "memory", "m0");
}

// Workgroup barrier for data exchanged through LDS only: s_barrier without the release
// fence of __syncthreads (which waits for every outstanding global load, including loads
// still in flight for later steps). The asm statements keep the compiler from moving
// memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Elements of T in 16 bytes (the vector width of the op kernels' loads and stores).
template <typename T>
constexpr int kVec = 16 / (int)sizeof(T);

__host__ __device__ __forceinline__ bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
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

inline unsigned blocks_for(int64_t n, int threads) {
  return (unsigned)((n + threads - 1) / threads);
}

// Runs f(float{}) or f(bf16{}) for the activation dtype.
template <typename F>
int dispatch_dtype(int dtype, F&& f) {
  if (dtype == PULSAR_F32) return f(float{});
  if (dtype == PULSAR_BF16) return f(bf16{});
  return fail(PULSAR_ERR_INVALID, "dtype must be PULSAR_F32 or PULSAR_BF16");
}

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
