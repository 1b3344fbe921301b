// Sampler kernels: temperature softmax and tree / chain rejection sampling.
//
// temperature_softmax: one workgroup per row.  bf16 rows of the Qwen and Llama-3
//   vocabulary sizes are read once into registers (max, sum and write from there);
//   other rows take two streaming passes (online max and sum, then the fp32 write).
//   128-bit accesses when rows are 16-byte aligned.  HBM bound: logits read (a
//   streaming kernel's second pass mostly from the Infinity Cache) and fp32
//   probabilities written once.
//
// rejection_sample_tree: one workgroup (1024 threads) per sequence walks the draft
//   tree from the root.  Per visited node the acceptance tests need two scalars;
//   in stochastic mode each rejection needs one pass over the node's target/draft
//   rows to renormalise the residual (delta mode updates a scalar), and the final
//   draw one inverse-CDF pass.  Only rows on the walk are read.  The fp32 association order of every sum and scan is fixed (see
//   nvx_internal.h) so integer outputs are reproducible bit for bit by the CPU
//   restatement given the same probabilities and uniforms.
#include <float.h>

#include "nvx_internal.h"

#pragma clang fp contract(off)

namespace {

constexpr int kNT = 1024;
constexpr int kNW = kNT / nvx::kWave;
constexpr int kMaxNodes = 64;


__device__ __forceinline__ float load_logit(const void* row, int i, int dtype) {
  if (dtype == NVX_DTYPE_F32) return reinterpret_cast<const float*>(row)[i];
  const uint16_t h = reinterpret_cast<const uint16_t*>(row)[i];
  return __uint_as_float((uint32_t)h << 16);
}

// ------------------------------------------------------- softmax (vectorised)
// One 1024-thread workgroup per row, two streaming passes over the logits: online
// max / sum in log2 units (x * log2(e) / T) with kU (eight for the softmax) 16-byte
// loads in flight per thread, then exp2(fma(x, log2(e)/T, -max)) * (1/sum) written as
// 128-bit stores.
// With at most two rows per CU in flight (~150 MB of rows GPU-wide) the second
// read of a row is served by the Infinity Cache.  1/T folded into the FMA
// keeps the relative error ~1e-6 (contract tolerance 1e-5).
constexpr int kVecNT = 1024;

// Modes of the streaming kernel.  kSoftmax: both passes.  kStatsOnly: the first pass
// only; stores (max in log2 units, 1/sum) for the row in stats[row] (the fused
// rejection walk recomputes each probability it reads).  kFromStats: the second pass
// only, with the row's statistics read from stats[row] (probabilities bit for bit as
// the fused walk computes them).  kU: 16-byte loads in flight per thread.
enum { kSoftmax = 0, kStatsOnly = 1, kFromStats = 2 };
template <typename VT, int kMode = kSoftmax, int kU = 8>
__global__ __launch_bounds__(kVecNT) void softmax_vec_kernel(const VT* __restrict__ logits,
                                                             int64_t stride,
                                                             const float* __restrict__ temps,
                                                             float* __restrict__ probs, int V,
                                                             float2* __restrict__ stats) {
  constexpr int kUnroll = kU;
  using Tr = nvx::VecTraits<VT>;
  constexpr int P = Tr::kPer;
  __shared__ float red[kVecNT / nvx::kWave];
  const int row = blockIdx.x;
  const float T = temps[row];
  const uint4* src = reinterpret_cast<const uint4*>(logits + (int64_t)row * stride);
  float* dst = probs + (int64_t)row * V;
  const int nvec = V / P;
  const int tid = threadIdx.x;
  if (T == 0.f) {  // greedy row: fp32 logits unchanged
    if constexpr (kMode == kStatsOnly) {
      if (tid == 0) stats[row] = make_float2(0.f, 0.f);
      return;
    }
    for (int i = tid; i < nvec; i += kVecNT) {
      float x[P];
      Tr::expand(src[i], x);
#pragma unroll
      for (int e = 0; e < P; e += 4)
        *reinterpret_cast<float4*>(dst + (int64_t)i * P + e) = make_float4(x[e], x[e + 1], x[e + 2], x[e + 3]);
    }
    return;
  }
  const float a = 1.4426950408889634f / T;
  float M, inv;
  int i = tid;
  if constexpr (kMode == kFromStats) {
    M = stats[row].x;
    inv = stats[row].y;
  } else {
    float m = -INFINITY, s = 0.f;
    for (; i + (kUnroll - 1) * kVecNT < nvec; i += kUnroll * kVecNT) {
      uint4 w[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u)
        w[u] = kMode == kStatsOnly ? nvx::ld_stream(src + i + u * kVecNT) : src[i + u * kVecNT];
      float lm = -INFINITY;
      float x[kUnroll][P];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        Tr::expand(w[u], x[u]);
#pragma unroll
        for (int e = 0; e < P; ++e) lm = fmaxf(lm, x[u][e]);
      }
      const float mn = fmaxf(m, lm * a);
      if (mn == -INFINITY) continue;  // every value so far is -inf
      float acc = 0.f;
#pragma unroll
      for (int u = 0; u < kUnroll; ++u)
#pragma unroll
        for (int e = 0; e < P; ++e) acc += __builtin_amdgcn_exp2f(__builtin_fmaf(x[u][e], a, -mn));
      s = (m == -INFINITY ? 0.f : s * __builtin_amdgcn_exp2f(m - mn)) + acc;
      m = mn;
    }
    for (; i < nvec; i += kVecNT) {
      float x[P];
      Tr::expand(src[i], x);
      float lm = -INFINITY;
#pragma unroll
      for (int e = 0; e < P; ++e) lm = fmaxf(lm, x[e]);
      const float mn = fmaxf(m, lm * a);
      if (mn == -INFINITY) continue;
      float acc = 0.f;
#pragma unroll
      for (int e = 0; e < P; ++e) acc += __builtin_amdgcn_exp2f(__builtin_fmaf(x[e], a, -mn));
      s = (m == -INFINITY ? 0.f : s * __builtin_amdgcn_exp2f(m - mn)) + acc;
      m = mn;
    }
    M = nvx::block_max<kVecNT>(m, red);
    const float part = (m == -INFINITY) ? 0.f : s * __builtin_amdgcn_exp2f(m - M);
    inv = 1.f / nvx::block_sum_any<kVecNT>(part, red);
    if constexpr (kMode == kStatsOnly) {
      if (tid == 0) stats[row] = make_float2(M, inv);
      return;
    }
  }
  i = tid;
  for (; i + (kUnroll - 1) * kVecNT < nvec; i += kUnroll * kVecNT) {
    uint4 w[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) w[u] = src[i + u * kVecNT];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      float x[P];
      Tr::expand(w[u], x);
      float* d = dst + (int64_t)(i + u * kVecNT) * P;
#pragma unroll
      for (int e = 0; e < P; e += 4)
        *reinterpret_cast<float4*>(d + e) = make_float4(
            __builtin_amdgcn_exp2f(__builtin_fmaf(x[e], a, -M)) * inv,
            __builtin_amdgcn_exp2f(__builtin_fmaf(x[e + 1], a, -M)) * inv,
            __builtin_amdgcn_exp2f(__builtin_fmaf(x[e + 2], a, -M)) * inv,
            __builtin_amdgcn_exp2f(__builtin_fmaf(x[e + 3], a, -M)) * inv);
    }
  }
  for (; i < nvec; i += kVecNT) {
    float x[P];
    Tr::expand(src[i], x);
    float* d = dst + (int64_t)i * P;
#pragma unroll
    for (int e = 0; e < P; e += 4)
      *reinterpret_cast<float4*>(d + e) = make_float4(
          __builtin_amdgcn_exp2f(__builtin_fmaf(x[e], a, -M)) * inv,
          __builtin_amdgcn_exp2f(__builtin_fmaf(x[e + 1], a, -M)) * inv,
          __builtin_amdgcn_exp2f(__builtin_fmaf(x[e + 2], a, -M)) * inv,
          __builtin_amdgcn_exp2f(__builtin_fmaf(x[e + 3], a, -M)) * inv);
  }
}

// ------------------------------------------------- softmax (row in registers)
// bf16 rows of (NG-1)*8*kRegNT < V <= NG*8*kRegNT logits: each of the 512 threads
// issues its NG 16-byte loads at once, so the row is read from HBM once and held
// packed in registers (4 bytes per two logits); max, sum and the fp32 write then
// work from registers.  Group u of thread t holds logits 8*(u*kRegNT + t) .. +7;
// only the last group reaches past the row (its lanes past the row hold -inf and
// store nothing).  One workgroup per CU (NG*4 + ~15 VGPRs), which alternates load,
// reduce and store; the same math as the streaming kernel with the exact row max
// instead of the online one.  Loads are raw buffer loads (one per-thread offset plus
// a scalar offset per group); stores are global stores from a uniform row base.
constexpr int kRegNT = 512;

template <int NG>
__global__ __launch_bounds__(kRegNT) void softmax_row_kernel(const uint16_t* __restrict__ logits,
                                                             int64_t stride,
                                                             const float* __restrict__ temps,
                                                             float* __restrict__ probs, int V) {
  using Tr = nvx::VecTraits<uint16_t>;
  __shared__ float red[kRegNT / nvx::kWave];
  const int row = blockIdx.x;
  const float T = temps[row];
  const int tid = threadIdx.x;
  const int nvec = V / 8;
  if (T == 0.f) {  // greedy row: fp32 logits unchanged
    const uint4* src = reinterpret_cast<const uint4*>(logits + (int64_t)row * stride);
    float* dst = probs + (int64_t)row * V;
    for (int i = tid; i < nvec; i += kRegNT) {
      float x[8];
      Tr::expand(src[i], x);
      *reinterpret_cast<float4*>(dst + (int64_t)i * 8) = make_float4(x[0], x[1], x[2], x[3]);
      *reinterpret_cast<float4*>(dst + (int64_t)i * 8 + 4) = make_float4(x[4], x[5], x[6], x[7]);
    }
    return;
  }
  constexpr int kRsrcWord3 = 0x00020000;  // gfx9 buffer descriptor word 3 (raw dword access)
  const __amdgpu_buffer_rsrc_t in_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(logits + (int64_t)row * stride), 0, V * 2, kRsrcWord3);
  const int voff = tid * 16;
  const bool tail_ok = tid + (NG - 1) * kRegNT < nvec;
  uint4 w[NG];
#pragma unroll
  for (int u = 0; u < NG - 1; ++u)
    w[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(in_rsrc, voff, u * kRegNT * 16, 0));
  w[NG - 1] = make_uint4(0xFF80FF80u, 0xFF80FF80u, 0xFF80FF80u, 0xFF80FF80u);  // bf16 -inf
  if (tail_ok)
    w[NG - 1] = __builtin_bit_cast(
        uint4, __builtin_amdgcn_raw_buffer_load_b128(in_rsrc, voff, (NG - 1) * kRegNT * 16, 0));
  float* const out_row = probs + (int64_t)row * V;
  auto store = [&](int u, const float (&y)[8]) {
    if (u < NG - 1 || tail_ok) {
      float* d = out_row + (uint32_t)(tid * 8 + u * kRegNT * 8);
      *reinterpret_cast<float4*>(d) = make_float4(y[0], y[1], y[2], y[3]);
      *reinterpret_cast<float4*>(d + 4) = make_float4(y[4], y[5], y[6], y[7]);
    }
  };
  // Each pass re-expands from the packed registers: without this the compiler keeps
  // the expanded fp32 values of the first pass live (8 bytes per two logits).
  auto opaque = [&]() {
#pragma unroll
    for (int u = 0; u < NG; ++u)
      asm volatile("" : "+v"(w[u].x), "+v"(w[u].y), "+v"(w[u].z), "+v"(w[u].w));
  };
  const float a = 1.4426950408889634f / T;
  float lm = -INFINITY;
#pragma unroll
  for (int u = 0; u < NG; ++u) {
    float x[8];
    Tr::expand(w[u], x);
#pragma unroll
    for (int e = 0; e < 8; ++e) lm = fmaxf(lm, x[e]);
  }
  const float M = nvx::block_max<kRegNT>(lm * a, red);
  opaque();
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int u = 0; u < NG; ++u) {
    float x[8];
    Tr::expand(w[u], x);
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      s0 += __builtin_amdgcn_exp2f(__builtin_fmaf(x[e], a, -M));
      s1 += __builtin_amdgcn_exp2f(__builtin_fmaf(x[e + 1], a, -M));
    }
  }
  const float inv = 1.f / nvx::block_sum_any<kRegNT>(s0 + s1, red);
  opaque();
#pragma unroll
  for (int u = 0; u < NG; ++u) {
    float x[8];
    Tr::expand(w[u], x);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(x[e], a, -M)) * inv;
    store(u, x);
  }
}

// Register-resident instantiations: 38 groups cover 151,553..155,648 logits (Qwen's
// 151,936), 32 cover 126,977..131,072 (Llama-3's 128,256).
inline int row_kernel_groups(int vocab) { return (vocab / 8 + kRegNT - 1) / kRegNT; }

// --------------------------------------------------------- softmax (stream)
__global__ __launch_bounds__(kNT) void softmax_stream_kernel(const void* __restrict__ logits,
                                                             int dtype, int64_t stride,
                                                             const float* __restrict__ temps,
                                                             float* __restrict__ probs, int V) {
  __shared__ float red[kNW];
  const int row = blockIdx.x;
  const float T = temps[row];
  const bool greedy = (T == 0.f);
  const int esz = dtype == NVX_DTYPE_F32 ? 4 : 2;
  const void* src = reinterpret_cast<const char*>(logits) + (int64_t)row * stride * esz;
  float* dst = probs + (int64_t)row * V;
  if (greedy) {
    for (int i = threadIdx.x; i < V; i += kNT) dst[i] = load_logit(src, i, dtype);
    return;
  }
  // Online max / sum over the raw logits in log2 units (x * log2(e) / T).
  const float a = 1.4426950408889634f / T;
  float m = -INFINITY, s = 0.f;
  for (int i = threadIdx.x; i < V; i += kNT) {
    const float x = load_logit(src, i, dtype) * a;
    if (x == -INFINITY) continue;
    if (x > m) {
      s = s * __builtin_amdgcn_exp2f(m - x) + 1.f;
      m = x;
    } else {
      s += __builtin_amdgcn_exp2f(x - m);
    }
  }
  const float M = nvx::block_max<kNT>(m, red);
  const float part = (m == -INFINITY) ? 0.f : s * __builtin_amdgcn_exp2f(m - M);
  const float inv = 1.f / nvx::block_sum_any<kNT>(part, red);
  for (int i = threadIdx.x; i < V; i += kNT)
    dst[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(load_logit(src, i, dtype), a, -M)) * inv;
}

// ------------------------------------------------------- rejection sampling
// Current distribution at a node (closed form, see the contract in the oracle):
//   stochastic: cur[y] = max(p[y] - c*q[y], 0) / Z
//   delta:      cur[y] = (y in R ? 0 : p[y]) / Z
struct Residual {
  float c, Z;
  const int* R;  // rejected tokens (LDS), delta mode
  int nR;
  bool delta;
};

__device__ __forceinline__ bool in_set(const int* R, int n, int y) {
  bool hit = false;
  for (int i = 0; i < n; ++i) hit |= (R[i] == y);
  return hit;
}

__device__ __forceinline__ float cur_eval(const Residual& r, float py, float qy, int y) {
  if (r.delta) return (r.nR > 0 && in_set(r.R, r.nR, y) ? 0.f : py) / r.Z;
  return fmaxf(py - r.c * qy, 0.f) / r.Z;
}

__device__ __forceinline__ void load4f(const float* row, int g, int V, bool vec, float out[4]) {
  const int i0 = 4 * g;
  if (vec && i0 + 3 < V) {
    const float4 t = reinterpret_cast<const float4*>(row)[g];
    out[0] = t.x; out[1] = t.y; out[2] = t.z; out[3] = t.w;
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) out[c] = (i0 + c < V) ? row[i0 + c] : 0.f;
  }
}

// Sources of the target distribution read by the walk.  ProbRow: fp32 probability
// rows (the softmax output).  LogitRow: the row's logits with its statistics from
// nvx_softmax_stats; each probability is recomputed as exp2(fma(x, log2(e)/T, -max)) *
// (1/sum), or x itself at temperature 0, the values nvx_softmax_from_stats writes for
// the same statistics.
struct ProbRow {
  const float* row;
  __device__ __forceinline__ void load4(int g, int V, bool vec, float out[4]) const {
    load4f(row, g, V, vec, out);
  }
  __device__ __forceinline__ float at(int y) const { return row[y]; }
};

template <typename VT>
struct LogitRow {
  const VT* row;
  float a, M, inv;
  bool raw;  // temperature 0: the softmax passes the fp32 logits through
  __device__ __forceinline__ float prob(float x) const {
    return raw ? x : __builtin_amdgcn_exp2f(__builtin_fmaf(x, a, -M)) * inv;
  }
  __device__ __forceinline__ static float val(const VT* r, int i) {
    if constexpr (sizeof(VT) == 2) return nvx::bf16_lo((uint32_t)reinterpret_cast<const uint16_t*>(r)[i]);
    else return reinterpret_cast<const float*>(r)[i];
  }
  __device__ __forceinline__ void load4(int g, int V, bool vec, float out[4]) const {
    const int i0 = 4 * g;
    float x[4];
    if (vec && i0 + 3 < V) {
      if constexpr (sizeof(VT) == 2) {
        const uint2 w = reinterpret_cast<const uint2*>(row)[g];
        x[0] = nvx::bf16_lo(w.x); x[1] = nvx::bf16_hi(w.x);
        x[2] = nvx::bf16_lo(w.y); x[3] = nvx::bf16_hi(w.y);
      } else {
        const float4 t = reinterpret_cast<const float4*>(row)[g];
        x[0] = t.x; x[1] = t.y; x[2] = t.z; x[3] = t.w;
      }
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) x[c] = (i0 + c < V) ? val(row, i0 + c) : 0.f;
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) out[c] = (i0 + c < V) ? prob(x[c]) : 0.f;
  }
  __device__ __forceinline__ float at(int y) const { return prob(val(row, y)); }
};

struct ProbSource {
  const float* P;
  int64_t seq_stride;
  int V;
  __device__ __forceinline__ ProbRow row(int b, int cur) const {
    return {P + (int64_t)b * seq_stride + (int64_t)cur * V};
  }
};

template <typename VT>
struct LogitSource {
  const VT* L;
  int64_t row_stride;  // elements between logits rows; sequence b's node i is row b*rows_per_seq + i
  int rows_per_seq;
  const float* temps;   // per logits row
  const float2* stats;  // per logits row: (max in log2 units, 1/sum)
  __device__ __forceinline__ LogitRow<VT> row(int b, int cur) const {
    const int64_t r = (int64_t)b * rows_per_seq + cur;
    const float T = temps[r];
    const float2 st = stats[r];
    return {L + r * row_stride, 1.4426950408889634f / T, st.x, st.y, T == 0.f};
  }
};

// Canonical sum over y of max(p[y] - c*q[y], 0) (the un-normalised stochastic
// residual for multiplier c).  Four groups per lane are loaded before they are
// accumulated (in the same order) to keep more bytes in flight.
template <typename PRow>
__device__ float residual_sum(const PRow& prow, const float* qrow, int V, bool vec, float c,
                              float* red) {
  const int G = (V + 3) / 4;
  float acc = 0.f;
  int g = threadIdx.x;
  for (; g + 3 * kNT < G; g += 4 * kNT) {
    float p[4][4], q[4][4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      prow.load4(g + u * kNT, V, vec, p[u]);
      load4f(qrow, g + u * kNT, V, vec, q[u]);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = acc + fmaxf(p[u][e] - c * q[u][e], 0.f);
  }
  for (; g < G; g += kNT) {
    float p[4], q[4];
    prow.load4(g, V, vec, p);
    load4f(qrow, g, V, vec, q);
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (4 * g + e < V) acc = acc + fmaxf(p[e] - c * q[e], 0.f);
  }
  return nvx::block_sum_canonical<kNT>(acc, red);
}

// Inverse-CDF pick from the current distribution with uniform u (contract in
// oracle/sampler.py: cdf_pick).
template <typename PRow>
__device__ int cdf_pick(const PRow& prow, const float* qrow, int V, bool vec, const Residual& r,
                        float u, float* red, int* redi, float* incl_lds) {
  const int C = 4 * (((V + 3) / 4 + kNT - 1) / kNT);
  const int lo = threadIdx.x * C;
  const int hi = min(lo + C, V);
  // Lane t owns elements [lo, hi); its groups are read four at a time.
  float s = 0.f;
  for (int i = lo; i < hi; i += 16) {
    float p[4][4], q[4][4] = {};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (i + 4 * u < hi) {
        prow.load4(i / 4 + u, V, vec, p[u]);
        if (!r.delta) load4f(qrow, i / 4 + u, V, vec, q[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (i + 4 * u + e < hi) s = s + cur_eval(r, p[u][e], q[u][e], i + 4 * u + e);
  }
  float total;
  const float incl = nvx::block_incl_scan_canonical<kNT>(s, red, &total);
  incl_lds[threadIdx.x] = incl;
  __syncthreads();
  const float tau = u * total;
  float run = threadIdx.x > 0 ? incl_lds[threadIdx.x - 1] : 0.f;
  int first = INT32_MAX, last = -1;
  for (int i = lo; i < hi; i += 16) {
    float p[4][4], q[4][4] = {};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (i + 4 * u < hi) {
        prow.load4(i / 4 + u, V, vec, p[u]);
        if (!r.delta) load4f(qrow, i / 4 + u, V, vec, q[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int y = i + 4 * u + e;
        if (y < hi) {
          const float v = cur_eval(r, p[u][e], q[u][e], y);
          run = run + v;
          if (v > 0.f) {
            last = y;
            if (first == INT32_MAX && run > tau) first = y;
          }
        }
      }
    }
  }
  __syncthreads();
  const int f = nvx::block_min_i<kNT>(first, redi);
  if (f != INT32_MAX) return f;
  return nvx::block_max_i<kNT>(last, redi);
}

// First index of the row maximum.
template <typename PRow>
__device__ int block_argmax(const PRow& row, int V, bool vec, float* red, int* redi) {
  float bv = -INFINITY;
  int bi = INT32_MAX;
  const int G = (V + 3) / 4;
  for (int g0 = threadIdx.x; g0 < G; g0 += 4 * kNT) {
    float p[4][4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (g0 + u * kNT < G) row.load4(g0 + u * kNT, V, vec, p[u]);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int g = g0 + u * kNT;
      if (g >= G) break;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int y = 4 * g + c;
        if (y < V && (p[u][c] > bv || (p[u][c] == bv && y < bi))) {
          bv = p[u][c];
          bi = y;
        }
      }
    }
  }
  const int lane = threadIdx.x & 63, wid = threadIdx.x / 64;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = nvx::shfl_xor_f(bv, off);
    const int oi = nvx::shfl_xor_i(bi, off);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane == 0) {
    red[wid] = bv;
    redi[wid] = bi;
  }
  __syncthreads();
  bv = red[lane < kNW ? lane : 0];
  bi = redi[lane < kNW ? lane : 0];
#pragma unroll
  for (int off = kNW / 2; off >= 1; off >>= 1) {
    const float ov = nvx::shfl_xor_f(bv, off);
    const int oi = nvx::shfl_xor_i(bi, off);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  __syncthreads();
  const int r = __shfl(bi, 0, 64);
  return r == INT32_MAX ? 0 : r;
}

template <typename Src>
__global__ __launch_bounds__(kNT) void rejection_tree_kernel(
    Src src, const float* __restrict__ Q,
    int64_t q_seq_stride, int V, const int32_t* __restrict__ tokens,
    const int32_t* __restrict__ parents, const int32_t* __restrict__ num_nodes, int node_stride,
    const float* __restrict__ U, const float* __restrict__ U_final,
    const uint8_t* __restrict__ greedy_flags, int delta, int32_t* __restrict__ path_out,
    int32_t* __restrict__ acc_out, int32_t* __restrict__ tok_out, int32_t* __restrict__ next_out,
    bool vec) {
  __shared__ float red[kNW];
  __shared__ int redi[kNW];
  __shared__ int s_par[kMaxNodes], s_tok[kMaxNodes], s_path[kMaxNodes];
  __shared__ float s_u[kMaxNodes];
  __shared__ int s_R[kMaxNodes];
  __shared__ float s_incl[kNT];

  const int b = blockIdx.x;
  int T = node_stride;
  if (num_nodes) T = max(1, min(num_nodes[b], node_stride));
  if (threadIdx.x < T) {
    s_par[threadIdx.x] = parents[(int64_t)b * node_stride + threadIdx.x];
    s_tok[threadIdx.x] = tokens[(int64_t)b * node_stride + threadIdx.x];
    s_u[threadIdx.x] = U[(int64_t)b * node_stride + threadIdx.x];
  }
  __syncthreads();
  const bool greedy = greedy_flags ? greedy_flags[b] != 0 : false;
  const float uf = U_final[b];

  int cur = 0, depth = 0, next = 0;
  if (threadIdx.x == 0) s_path[0] = 0;
  while (true) {
    const auto prow = src.row(b, cur);
    const float* qrow = Q ? Q + (int64_t)b * q_seq_stride + (int64_t)cur * V : nullptr;
    int accepted = -1;
    if (greedy) {
      const int a = block_argmax(prow, V, vec, red, redi);
      for (int j = cur + 1; j < T; ++j)
        if (s_par[j] == cur && s_tok[j] == a) {
          accepted = j;
          break;
        }
      if (accepted < 0) {
        next = a;
        break;
      }
    } else {
      Residual res{0.f, 1.f, s_R, 0, delta != 0};
      for (int j = cur + 1; j < T; ++j) {
        if (s_par[j] != cur) continue;
        const int x = s_tok[j];
        const bool valid = x >= 0 && x < V;
        float cx = 0.f, qx = 1.f, px = 0.f;
        if (valid) {
          px = prow.at(x);
          const float qv = res.delta ? 0.f : qrow[x];
          cx = cur_eval(res, px, qv, x);
          if (!res.delta) qx = qv;
        }
        if (s_u[j] * qx <= cx && cx > 0.f) {
          accepted = j;
          break;
        }
        if (res.delta) {
          if (valid && !(res.nR > 0 && in_set(s_R, res.nR, x))) {
            __syncthreads();  // every lane has read s_R
            if (threadIdx.x == 0) s_R[res.nR] = x;
            __syncthreads();
            res.nR += 1;
            res.Z = res.Z - px;
          }
          if (!(res.Z > 0.f)) {
            res.nR = 0;
            res.Z = 1.f;
          }
        } else {
          const float c = res.c + res.Z;
          const float Z = residual_sum(prow, qrow, V, vec, c, red);
          if (Z > 0.f) {
            res.c = c;
            res.Z = Z;
          } else {
            res.c = 0.f;
            res.Z = 1.f;
          }
        }
      }
      if (accepted < 0) {
        next = cdf_pick(prow, qrow, V, vec, res, uf, red, redi, s_incl);
        break;
      }
    }
    cur = accepted;
    depth += 1;
    if (threadIdx.x == 0) s_path[depth] = cur;
  }
  __syncthreads();
  const int64_t ob = (int64_t)b * node_stride;
  for (int i = threadIdx.x; i < node_stride; i += kNT) {
    path_out[ob + i] = (i <= depth) ? s_path[i] : -1;
    int t = -1;
    if (i < depth) t = s_tok[s_path[i + 1]];
    else if (i == depth) t = next;
    tok_out[ob + i] = t;
  }
  if (threadIdx.x == 0) {
    acc_out[b] = depth;
    next_out[b] = next;
  }
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }
// The row statistics are read and written as float2 (max, 1/sum) pairs.
inline bool aligned8(const void* p) { return ((uintptr_t)p & 7) == 0; }

}  // namespace

extern "C" int nvx_temperature_softmax(const void* logits, int32_t logits_dtype,
                                       int64_t logits_row_stride, const float* temperatures,
                                       float* probs, int32_t num_rows, int32_t vocab, void* stream) {
  nvx::clear_error();
  NVX_CHECK(logits_dtype == NVX_DTYPE_F32 || logits_dtype == NVX_DTYPE_BF16,
            "temperature_softmax: logits must be fp32 or bf16 (dtype code %d)", logits_dtype);
  NVX_CHECK(num_rows >= 0 && vocab >= 1 && logits_row_stride >= vocab,
            "temperature_softmax: bad sizes (rows=%d, vocab=%d, stride=%lld)", num_rows, vocab,
            (long long)logits_row_stride);
  if (num_rows == 0) return NVX_OK;
  NVX_CHECK(logits && temperatures && probs, "temperature_softmax: null pointer");
  hipStream_t s = (hipStream_t)stream;
  nvx::TimerScope timer(NVX_TIMER_SOFTMAX, s);
  const int per = logits_dtype == NVX_DTYPE_BF16 ? 8 : 4;
  const bool vec = vocab % per == 0 && logits_row_stride % per == 0 && aligned16(logits) &&
                   aligned16(probs);
  const int groups = row_kernel_groups(vocab);
  if (vec && logits_dtype == NVX_DTYPE_BF16 && (groups == 38 || groups == 32)) {
    hipLaunchKernelGGL(groups == 38 ? softmax_row_kernel<38> : softmax_row_kernel<32>,
                       dim3(num_rows), dim3(kRegNT), 0, s, (const uint16_t*)logits,
                       logits_row_stride, temperatures, probs, vocab);
  } else if (vec && logits_dtype == NVX_DTYPE_BF16) {
    hipLaunchKernelGGL(softmax_vec_kernel<uint16_t>, dim3(num_rows), dim3(kVecNT), 0, s,
                       (const uint16_t*)logits, logits_row_stride, temperatures, probs, vocab,
                       (float2*)nullptr);
  } else if (vec) {
    hipLaunchKernelGGL(softmax_vec_kernel<float>, dim3(num_rows), dim3(kVecNT), 0, s,
                       (const float*)logits, logits_row_stride, temperatures, probs, vocab,
                       (float2*)nullptr);
  } else {
    hipLaunchKernelGGL(softmax_stream_kernel, dim3(num_rows), dim3(kNT), 0, s, logits, logits_dtype,
                       logits_row_stride, temperatures, probs, vocab);
  }
  NVX_LAUNCHED();
  return NVX_OK;
}

extern "C" int nvx_rejection_sample_tree(const float* target_probs, int64_t p_seq_stride,
                                         const float* draft_probs, int64_t q_seq_stride, int32_t vocab,
                                         const int32_t* tokens, const int32_t* parents,
                                         const int32_t* num_nodes, int32_t node_stride,
                                         const float* uniforms, const float* final_uniforms,
                                         const uint8_t* greedy, int32_t draft_mode, int32_t num_seqs,
                                         int32_t* path, int32_t* accepted_len, int32_t* out_tokens,
                                         int32_t* next_token, void* stream) {
  nvx::clear_error();
  NVX_CHECK(num_seqs >= 0 && vocab >= 1, "rejection_sample_tree: bad sizes (seqs=%d, vocab=%d)",
            num_seqs, vocab);
  NVX_CHECK(node_stride >= 1 && node_stride <= kMaxNodes,
            "rejection_sample_tree: node_stride must be in [1, %d] (got %d)", kMaxNodes, node_stride);
  NVX_CHECK(draft_mode == 0 || draft_mode == 1, "rejection_sample_tree: draft_mode must be 0 or 1");
  NVX_CHECK(draft_mode == 1 || draft_probs != nullptr,
            "rejection_sample_tree: draft_probs required in draft_mode 0");
  if (num_seqs == 0) return NVX_OK;
  NVX_CHECK(target_probs && tokens && parents && uniforms && final_uniforms && path &&
                accepted_len && out_tokens && next_token,
            "rejection_sample_tree: null pointer");
  hipStream_t s = (hipStream_t)stream;
  nvx::TimerScope timer(NVX_TIMER_REJECTION, s);
  const bool vec = vocab % 4 == 0 && p_seq_stride % 4 == 0 && aligned16(target_probs) &&
                   (draft_mode == 1 || (q_seq_stride % 4 == 0 && aligned16(draft_probs)));
  hipLaunchKernelGGL(rejection_tree_kernel<ProbSource>, dim3(num_seqs), dim3(kNT), 0, s,
                     ProbSource{target_probs, p_seq_stride, vocab},
                     draft_mode == 1 ? nullptr : draft_probs, q_seq_stride, vocab, tokens, parents,
                     num_nodes, node_stride, uniforms, final_uniforms, greedy, draft_mode, path,
                     accepted_len, out_tokens, next_token, vec);
  NVX_LAUNCHED();
  return NVX_OK;
}

extern "C" int nvx_softmax_stats(const void* logits, int32_t logits_dtype,
                                 int64_t logits_row_stride, const float* temperatures, float* stats,
                                 int32_t num_rows, int32_t vocab, void* stream) {
  nvx::clear_error();
  NVX_CHECK(logits_dtype == NVX_DTYPE_F32 || logits_dtype == NVX_DTYPE_BF16,
            "softmax_stats: logits must be fp32 or bf16 (dtype code %d)", logits_dtype);
  NVX_CHECK(num_rows >= 0 && vocab >= 1 && logits_row_stride >= vocab,
            "softmax_stats: bad sizes (rows=%d, vocab=%d, stride=%lld)", num_rows, vocab,
            (long long)logits_row_stride);
  if (num_rows == 0) return NVX_OK;
  NVX_CHECK(logits && temperatures && stats, "softmax_stats: null pointer");
  NVX_CHECK(aligned8(stats), "softmax_stats: stats must be 8-byte aligned");
  const int per = logits_dtype == NVX_DTYPE_BF16 ? 8 : 4;
  NVX_CHECK(vocab % per == 0 && logits_row_stride % per == 0 && aligned16(logits),
            "softmax_stats: needs 16-byte aligned logits rows with vocab and row stride "
            "multiples of %d", per);
  hipStream_t s = (hipStream_t)stream;
  nvx::TimerScope timer(NVX_TIMER_SOFTMAX, s);
  // One streaming pass (online max and sum) with four 16-byte loads in flight per
  // thread: fewer registers, two workgroups per CU.
  float2* st = reinterpret_cast<float2*>(stats);
  if (logits_dtype == NVX_DTYPE_BF16)
    hipLaunchKernelGGL((softmax_vec_kernel<uint16_t, kStatsOnly, 4>), dim3(num_rows), dim3(kVecNT),
                       0, s, (const uint16_t*)logits, logits_row_stride, temperatures,
                       (float*)nullptr, vocab, st);
  else
    hipLaunchKernelGGL((softmax_vec_kernel<float, kStatsOnly, 4>), dim3(num_rows), dim3(kVecNT), 0,
                       s, (const float*)logits, logits_row_stride, temperatures, (float*)nullptr,
                       vocab, st);
  NVX_LAUNCHED();
  return NVX_OK;
}

extern "C" int nvx_softmax_from_stats(const void* logits, int32_t logits_dtype,
                                      int64_t logits_row_stride, const float* temperatures,
                                      const float* stats, float* probs, int32_t num_rows,
                                      int32_t vocab, void* stream) {
  nvx::clear_error();
  NVX_CHECK(logits_dtype == NVX_DTYPE_F32 || logits_dtype == NVX_DTYPE_BF16,
            "softmax_from_stats: logits must be fp32 or bf16 (dtype code %d)", logits_dtype);
  NVX_CHECK(num_rows >= 0 && vocab >= 1 && logits_row_stride >= vocab,
            "softmax_from_stats: bad sizes (rows=%d, vocab=%d, stride=%lld)", num_rows, vocab,
            (long long)logits_row_stride);
  if (num_rows == 0) return NVX_OK;
  NVX_CHECK(logits && temperatures && stats && probs, "softmax_from_stats: null pointer");
  NVX_CHECK(aligned8(stats), "softmax_from_stats: stats must be 8-byte aligned");
  const int per = logits_dtype == NVX_DTYPE_BF16 ? 8 : 4;
  NVX_CHECK(vocab % per == 0 && logits_row_stride % per == 0 && aligned16(logits) &&
                aligned16(probs),
            "softmax_from_stats: needs 16-byte aligned rows with vocab and row stride multiples "
            "of %d", per);
  hipStream_t s = (hipStream_t)stream;
  nvx::TimerScope timer(NVX_TIMER_SOFTMAX, s);
  float2* st = const_cast<float2*>(reinterpret_cast<const float2*>(stats));
  if (logits_dtype == NVX_DTYPE_BF16)
    hipLaunchKernelGGL((softmax_vec_kernel<uint16_t, kFromStats>), dim3(num_rows), dim3(kVecNT), 0,
                       s, (const uint16_t*)logits, logits_row_stride, temperatures, probs, vocab, st);
  else
    hipLaunchKernelGGL((softmax_vec_kernel<float, kFromStats>), dim3(num_rows), dim3(kVecNT), 0, s,
                       (const float*)logits, logits_row_stride, temperatures, probs, vocab, st);
  NVX_LAUNCHED();
  return NVX_OK;
}

extern "C" int nvx_rejection_sample_tree_logits(
    const void* logits, int32_t logits_dtype, int64_t logits_row_stride,
    const float* temperatures, const float* stats, const float* draft_probs, int64_t q_seq_stride,
    int32_t vocab, const int32_t* tokens, const int32_t* parents, const int32_t* num_nodes,
    int32_t node_stride, const float* uniforms, const float* final_uniforms, const uint8_t* greedy,
    int32_t draft_mode, int32_t num_seqs, int32_t* path, int32_t* accepted_len,
    int32_t* out_tokens, int32_t* next_token, void* stream) {
  nvx::clear_error();
  NVX_CHECK(logits_dtype == NVX_DTYPE_F32 || logits_dtype == NVX_DTYPE_BF16,
            "rejection_sample_tree_logits: logits must be fp32 or bf16 (dtype code %d)",
            logits_dtype);
  NVX_CHECK(num_seqs >= 0 && vocab >= 1 && logits_row_stride >= vocab,
            "rejection_sample_tree_logits: bad sizes (seqs=%d, vocab=%d, stride=%lld)", num_seqs,
            vocab, (long long)logits_row_stride);
  NVX_CHECK(node_stride >= 1 && node_stride <= kMaxNodes,
            "rejection_sample_tree_logits: node_stride must be in [1, %d] (got %d)", kMaxNodes,
            node_stride);
  NVX_CHECK(draft_mode == 0 || draft_mode == 1,
            "rejection_sample_tree_logits: draft_mode must be 0 or 1");
  NVX_CHECK(draft_mode == 1 || draft_probs != nullptr,
            "rejection_sample_tree_logits: draft_probs required in draft_mode 0");
  if (num_seqs == 0) return NVX_OK;
  NVX_CHECK(logits && temperatures && stats && tokens && parents && uniforms && final_uniforms &&
                path && accepted_len && out_tokens && next_token,
            "rejection_sample_tree_logits: null pointer");
  NVX_CHECK(aligned8(stats), "rejection_sample_tree_logits: stats must be 8-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  nvx::TimerScope timer(NVX_TIMER_REJECTION, s);
  const bool bf16 = logits_dtype == NVX_DTYPE_BF16;
  const uintptr_t align = bf16 ? 8 : 16;
  const bool vec = vocab % 4 == 0 && logits_row_stride % 4 == 0 &&
                   ((uintptr_t)logits & (align - 1)) == 0 &&
                   (draft_mode == 1 || (q_seq_stride % 4 == 0 && aligned16(draft_probs)));
  const float2* st = reinterpret_cast<const float2*>(stats);
  const float* q = draft_mode == 1 ? nullptr : draft_probs;
  if (bf16)
    hipLaunchKernelGGL(rejection_tree_kernel<LogitSource<uint16_t>>, dim3(num_seqs), dim3(kNT), 0, s,
                       LogitSource<uint16_t>{(const uint16_t*)logits, logits_row_stride,
                                             node_stride, temperatures, st},
                       q, q_seq_stride, vocab, tokens, parents, num_nodes, node_stride, uniforms,
                       final_uniforms, greedy, draft_mode, path, accepted_len, out_tokens,
                       next_token, vec);
  else
    hipLaunchKernelGGL(rejection_tree_kernel<LogitSource<float>>, dim3(num_seqs), dim3(kNT), 0, s,
                       LogitSource<float>{(const float*)logits, logits_row_stride, node_stride,
                                          temperatures, st},
                       q, q_seq_stride, vocab, tokens, parents, num_nodes, node_stride, uniforms,
                       final_uniforms, greedy, draft_mode, path, accepted_len, out_tokens,
                       next_token, vec);
  NVX_LAUNCHED();
  return NVX_OK;
}
