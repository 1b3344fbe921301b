// Internal helpers shared by the HIP sources of libnvx_spec.so (gfx950 only).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "nvx_spec.h"

namespace nvx {

// ------------------------------------------------------------------ host side
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Per-entry-point HIP-event timers (enabled by nvx_timing_enable).  Events are
// recorded on the launch stream around the kernel(s) of one entry point.
struct TimerScope {
  int id;
  hipStream_t stream;
  hipEvent_t start = nullptr, stop = nullptr;
  TimerScope(int id, hipStream_t s);
  ~TimerScope();
};

}  // namespace nvx

#define NVX_CHECK(cond, ...)                              \
  do {                                                    \
    if (!(cond)) return nvx::fail(NVX_EINVAL, __VA_ARGS__); \
  } while (0)

#define NVX_HIP(call)                                                          \
  do {                                                                         \
    hipError_t e_ = (call);                                                    \
    if (e_ != hipSuccess)                                                      \
      return nvx::fail(NVX_EHIP, "%s: %s", #call, hipGetErrorString(e_));      \
  } while (0)

#define NVX_LAUNCHED()                                                          \
  do {                                                                          \
    hipError_t e_ = hipGetLastError();                                          \
    if (e_ != hipSuccess)                                                       \
      return nvx::fail(NVX_EHIP, "kernel launch: %s", hipGetErrorString(e_));   \
  } while (0)

// ---------------------------------------------------------------- device side
namespace nvx {

constexpr int kWave = 64;

__device__ __forceinline__ float shfl_xor_f(float v, int off) { return __shfl_xor(v, off, 64); }
__device__ __forceinline__ int shfl_xor_i(int v, int off) { return __shfl_xor(v, off, 64); }
__device__ __forceinline__ float shfl_up_f(float v, int off) { return __shfl_up(v, off, 64); }

// 16-byte load with the non-temporal hint (`global_load_dwordx4 ... nt`), for data a
// kernel streams from HBM exactly once: the softmax statistics pass over [4096, 151936]
// bf16 logits takes 180 us with it against 207 us without, top-k 116 against 123 us.
// Not for inputs the previous kernel has just written (the fused layers after a GEMM
// measured the same or slower with it).
__device__ __forceinline__ uint4 ld_stream(const void* p) {
  typedef uint32_t v4u __attribute__((ext_vector_type(4)));
  const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Unpacking of one 16-byte vector of a row (8 bf16 or 4 fp32 values) to fp32.
template <typename VT>
struct VecTraits;
template <>
struct VecTraits<uint16_t> {  // bf16: 8 values per 16 bytes
  static constexpr int kPer = 8;
  __device__ static void expand(const uint4& w, float (&x)[8]) {
    x[0] = bf16_lo(w.x); x[1] = bf16_hi(w.x); x[2] = bf16_lo(w.y); x[3] = bf16_hi(w.y);
    x[4] = bf16_lo(w.z); x[5] = bf16_hi(w.z); x[6] = bf16_lo(w.w); x[7] = bf16_hi(w.w);
  }
};
template <>
struct VecTraits<float> {  // fp32: 4 values per 16 bytes
  static constexpr int kPer = 4;
  __device__ static void expand(const uint4& w, float (&x)[4]) {
    x[0] = __uint_as_float(w.x); x[1] = __uint_as_float(w.y);
    x[2] = __uint_as_float(w.z); x[3] = __uint_as_float(w.w);
  }
};

// Canonical block sum: xor butterfly inside each wave (offsets 32..1), then an xor
// butterfly over the wave totals (offsets NW/2..1).  Every thread gets the result.
// `red` must hold at least NW floats.  The fp32 association order is part of the
// sampler contract (bit-exact with the CPU restatement).
template <int NT>
__device__ __forceinline__ float block_sum_canonical(float v, float* red) {
  constexpr int NW = NT / kWave;
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = v + shfl_xor_f(v, off);
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float w = red[lane < NW ? lane : 0];
#pragma unroll
  for (int off = NW / 2; off >= 1; off >>= 1) w = w + shfl_xor_f(w, off);
  __syncthreads();
  return __shfl(w, 0, 64);
}

template <int NT>
__device__ __forceinline__ float block_max(float v, float* red) {
  constexpr int NW = NT / kWave;
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, shfl_xor_f(v, off));
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float w = red[lane < NW ? lane : 0];
#pragma unroll
  for (int off = NW / 2; off >= 1; off >>= 1) w = fmaxf(w, shfl_xor_f(w, off));
  __syncthreads();
  return __shfl(w, 0, 64);
}

template <int NT>
__device__ __forceinline__ float block_sum_any(float v, float* red) {
  return block_sum_canonical<NT>(v, red);
}

template <int NT>
__device__ __forceinline__ int block_min_i(int v, int* red) {
  constexpr int NW = NT / kWave;
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = min(v, shfl_xor_i(v, off));
  if (lane == 0) red[wid] = v;
  __syncthreads();
  int w = red[lane < NW ? lane : 0];
#pragma unroll
  for (int off = NW / 2; off >= 1; off >>= 1) w = min(w, shfl_xor_i(w, off));
  __syncthreads();
  return __shfl(w, 0, 64);
}

template <int NT>
__device__ __forceinline__ int block_max_i(int v, int* red) {
  constexpr int NW = NT / kWave;
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = max(v, shfl_xor_i(v, off));
  if (lane == 0) red[wid] = v;
  __syncthreads();
  int w = red[lane < NW ? lane : 0];
#pragma unroll
  for (int off = NW / 2; off >= 1; off >>= 1) w = max(w, shfl_xor_i(w, off));
  __syncthreads();
  return __shfl(w, 0, 64);
}

// Canonical inclusive scan: Kogge-Stone inside each wave (offsets 1..32), then
// Kogge-Stone over the wave totals (offsets 1..NW/2); a thread of wave w > 0 adds
// the inclusive total of waves 0..w-1.  `red` holds >= NW floats.  Returns the
// inclusive prefix; *total receives the block total.
template <int NT>
__device__ __forceinline__ float block_incl_scan_canonical(float v, float* red, float* total) {
  constexpr int NW = NT / kWave;
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    float t = shfl_up_f(v, off);
    if (lane >= off) v = v + t;
  }
  if (lane == kWave - 1) red[wid] = v;
  __syncthreads();
  float w = red[lane < NW ? lane : 0];
#pragma unroll
  for (int off = 1; off < NW; off <<= 1) {
    float t = shfl_up_f(w, off);
    if (lane >= off) w = w + t;
  }
  // lane j of every wave now holds the inclusive total of waves 0..j
  float before = __shfl(w, wid > 0 ? wid - 1 : 0, 64);
  *total = __shfl(w, NW - 1, 64);
  __syncthreads();
  return wid > 0 ? before + v : v;
}

}  // namespace nvx
