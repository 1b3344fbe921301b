// Sampler kernels: temperature softmax and tree / chain rejection sampling.
//
// temperature_softmax: one workgroup per row.  bf16 rows of the Qwen and Llama-3
//   vocabulary sizes are read once into registers (max, sum and write from there);
//   other rows take two streaming passes (online max and sum, then the fp32 write).
//   128-bit accesses when rows are 16-byte aligned.  HBM bound: logits read (a
//   streaming kernel's second pass mostly from the Infinity Cache) and fp32
//   probabilities written once.
//
// rejection_sample_tree: K = 16, 8, 4, 2 or 1 workgroups per sequence (64 waves in
//   all up to K = 4 of 16 waves each, then 64 / K waves each) walk the draft tree from
//   the root, each streaming 1/K of every row the walk reads, and exchanging the 64
//   logical-wave totals of each pass through tagged slots in device memory.  Per visited node the acceptance
//   tests need two scalars per child (loaded for every node when the walk starts);
//   in stochastic mode each rejection needs one pass over the node's target/draft
//   rows to renormalise the residual (delta mode updates a scalar).  The final draw
//   reuses the totals of the last pass (one more pass over the target row when the
//   node had no rejection) and re-reads one lane's elements.  Only rows on the walk
//   are read.  The fp32 association order of every sum and scan is fixed (below), the
//   same for every K, so integer outputs are reproducible bit for bit by the CPU
//   restatement given the same probabilities and uniforms.
#include <float.h>

#include <atomic>
#include <type_traits>

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
// The walk's fp32 contract (restated in oracle/sampler.py): a row, padded with
// zeros, is cut into subtiles of kSub = 512 elements; logical wave w (of 64) owns the
// contiguous subtiles [w*R, (w+1)*R), R = ceil(nsub/64), and lane l holds elements
// 8l..8l+7 of each.  A pass adds each lane's values in order into its lane sum L
// (registers only, no cross-lane traffic while the row streams), then chains the 64
// lane sums of a logical wave in lane order (E_l = E_{l-1} + L_l) and the 64 wave
// totals in wave order (W_{w+1} = W_w + E_63); the row total is W_64.  The inverse CDF
// runs over the elements in that order (logical waves, lanes, the lane's elements):
// the pick with uniform u takes the first lane whose end W_w + E_l exceeds u * total
// and resolves the element from one re-read of that lane's elements.  Stochastic
// residuals reuse the pass that computed their normaliser, so the final draw after a
// rejection costs one lane's elements, not a pass.
constexpr int kSub = 512;   // elements per subtile (64 lanes x 8)
constexpr int kBatch = 5;   // subtiles whose loads a wave issues together

enum { kPlain = 0, kResid = 1, kDelta = 2 };  // pass modes: p, max(p - c*q, 0), p with R zeroed

__device__ __forceinline__ bool in_set(const int* R, int n, int y) {
  bool hit = false;
  for (int i = 0; i < n; ++i) hit |= (R[i] == y);
  return hit;
}

// Eight consecutive fp32 values of a row from element y0 (zeros past V).  vec: the
// row allows 16-byte loads at every multiple of 8 elements.
__device__ __forceinline__ void load8f(const float* row, int y0, int V, bool vec, float out[8]) {
  if (vec && y0 + 8 <= V) {
    const float4 a = *reinterpret_cast<const float4*>(row + y0);
    const float4 b = *reinterpret_cast<const float4*>(row + y0 + 4);
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = (y0 + e < V) ? row[y0 + e] : 0.f;
  }
}

// Sources of the target distribution read by the walk.  ProbRow: fp32 probability
// rows (the softmax output).  LogitRow: the row's logits with its statistics from
// nvx_softmax_stats; each probability is recomputed as exp2(fma(x, log2(e)/T, -max)) *
// (1/sum), or x itself at temperature 0, the values nvx_softmax_from_stats writes for
// the same statistics.
struct F32x8 {
  float4 a, b;
};
__device__ __forceinline__ F32x8 raw8f(const float* row, int y0) {
  return {*reinterpret_cast<const float4*>(row + y0), *reinterpret_cast<const float4*>(row + y0 + 4)};
}
__device__ __forceinline__ void unpack8f(const F32x8& r, float out[8]) {
  out[0] = r.a.x; out[1] = r.a.y; out[2] = r.a.z; out[3] = r.a.w;
  out[4] = r.b.x; out[5] = r.b.y; out[6] = r.b.z; out[7] = r.b.w;
}

// Row types: load8 reads 8 values from any y0 (guarded); fetch / values split an
// unguarded 16-byte-aligned read of 8 values into the load and its conversion, so a
// wave can keep several subtiles' loads in flight.
struct ProbRow {
  const float* row;
  using Raw = F32x8;
  __device__ __forceinline__ void load8(int y0, int V, bool vec, float out[8]) const {
    load8f(row, y0, V, vec, out);
  }
  __device__ __forceinline__ Raw fetch(int y0) const { return raw8f(row, y0); }
  __device__ __forceinline__ void values(const Raw& r, float out[8]) const { unpack8f(r, out); }
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
  __device__ __forceinline__ void load8(int y0, int V, bool vec, float out[8]) const {
    float x[8];
    if (vec && y0 + 8 <= V) {
      if constexpr (sizeof(VT) == 2) {
        const uint4 w = *reinterpret_cast<const uint4*>(row + y0);
        nvx::VecTraits<uint16_t>::expand(w, x);
      } else {
        load8f(reinterpret_cast<const float*>(row), y0, V, true, x);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = (y0 + e < V) ? val(row, y0 + e) : 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = (y0 + e < V) ? prob(x[e]) : 0.f;
  }
  using Raw = typename std::conditional<sizeof(VT) == 2, uint4, F32x8>::type;
  __device__ __forceinline__ Raw fetch(int y0) const {
    if constexpr (sizeof(VT) == 2) return *reinterpret_cast<const uint4*>(row + y0);
    else return raw8f(reinterpret_cast<const float*>(row), y0);
  }
  __device__ __forceinline__ void values(const Raw& r, float out[8]) const {
    float x[8];
    if constexpr (sizeof(VT) == 2) nvx::VecTraits<uint16_t>::expand(r, x);
    else unpack8f(r, x);
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = prob(x[e]);
  }
  __device__ __forceinline__ float at(int y) const { return prob(val(row, y)); }
};

struct ProbSource {
  static constexpr bool kLazy = false;
  const float* P;
  int64_t seq_stride;
  int V;
  __device__ __forceinline__ ProbRow row(int b, int cur) const {
    return {P + (int64_t)b * seq_stride + (int64_t)cur * V};
  }
};

template <typename VT>
struct LogitSource {
  static constexpr bool kLazy = false;
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

// Logits whose row statistics the walk computes itself, for the rows it visits only:
// on arriving at a node, the exact row max of the logits (times log2(e)/T) and then
// the canonical-order sum of exp2(fma(x, log2(e)/T, -max)) (the walk's own chain,
// the same bits for every number of workgroups per sequence).  The statistics of each
// visited row are written to stats_out (when given), so nvx_softmax_from_stats can
// rebuild exactly the probabilities the walk used.
template <typename VT>
struct LazyLogitSource {
  static constexpr bool kLazy = true;
  const VT* L;
  int64_t row_stride;
  int rows_per_seq;
  const float* temps;  // per logits row
  float2* stats_out;   // per logits row, written for visited rows (may be null)
  __device__ __forceinline__ int64_t index(int b, int cur) const {
    return (int64_t)b * rows_per_seq + cur;
  }
  __device__ __forceinline__ float scale(int b, int cur) const {
    return 1.4426950408889634f / temps[index(b, cur)];
  }
  // the row's raw logits (for the max)
  __device__ __forceinline__ LogitRow<VT> raw_row(int b, int cur) const {
    return {L + index(b, cur) * row_stride, 0.f, 0.f, 0.f, true};
  }
  __device__ __forceinline__ LogitRow<VT> row(int b, int cur, float M, float inv) const {
    const float T = temps[index(b, cur)];
    return {L + index(b, cur) * row_stride, 1.4426950408889634f / T, M, inv, T == 0.f};
  }
};

// Current residual values of the 8 elements from y0: p (kPlain), max(p - c*q, 0)
// (kResid; separately rounded product and difference), or p with the tokens of R
// zeroed (kDelta).
struct PassSpec {
  int mode;
  float c;
  const int* R;  // LDS
  int nR;
};

template <typename PRow>
__device__ __forceinline__ void residual8(const PRow& prow, const float* qrow, int y0, int V, bool vp,
                                          bool vq, const PassSpec& ps, float v[8]) {
  float p[8];
  prow.load8(y0, V, vp, p);
  if (ps.mode == kResid) {
    float q[8];
    load8f(qrow, y0, V, vq, q);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = fmaxf(p[e] - ps.c * q[e], 0.f);
  } else {
    uint32_t zero = 0;
    if (ps.mode == kDelta)
      for (int i = 0; i < ps.nR; ++i) {
        const uint32_t d = (uint32_t)(ps.R[i] - y0);
        if (d < 8u) zero |= 1u << d;
      }
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = ((zero >> e) & 1u) ? 0.f : p[e];
  }
}

// ------------------------------------------------ walk: layout and exchange
// kLW = 64 logical waves own contiguous runs of R = ceil(nsub / 64) subtiles.  A
// sequence is walked by K = 1, 2, 4, 8 or 16 workgroups of NW = walk_nw(K) waves (K > 1
// only when the whole grid fits on the device at once); real wave j of workgroup k
// holds the M = walk_m(K) logical waves (NW k + j) * M .. + M - 1, so the sums, chains
// and picks are the same bits for every K.
constexpr int kLW = 64;
constexpr int kMaxVocab = kSub * 64 * kLW;   // R <= 64: a lane can hold a subtile index
constexpr int kSlots = 2 * kLW;              // per sequence: two banks of 64 exchange slots
constexpr uint32_t kMaxSpins = 1u << 20;     // bound on a wait for an exchanged value
constexpr uint32_t kFailSkip = 1024;         // > the exchanges of one walk (2 * kMaxNodes + 3)
constexpr int kMaxWidth = 16;                // workgroups per sequence
// K workgroups per sequence: waves per workgroup (16 up to K = 4, then 64 / K) and
// logical waves per real wave (NW * M * K = 64).
constexpr int walk_nw(int K) { return K <= 4 ? 16 : kLW / K; }
constexpr int walk_m(int K) { return kLW / (K * walk_nw(K)); }

struct Layout {
  int nsub, R;
  __device__ __forceinline__ explicit Layout(int V) {
    nsub = max(1, (V + kSub - 1) / kSub);
    R = (nsub + kLW - 1) / kLW;
  }
  __device__ __forceinline__ int lo(int lw) const { return min(lw * R, nsub); }
  __device__ __forceinline__ int hi(int lw) const { return min(lw * R + R, nsub); }
};

// The walk's cross-workgroup state lives in the caller's workspace (zero-filled
// before its first use, then kept by the library), one fixed-size record per
// sequence index at b * kRecWords 64-bit words, so walks of any batch size that
// reuse one workspace see the same record for sequence b:
//  * kSlots 64-bit exchange slots, each holding (exchange number << 32) | value, so a
//    value and the exchange it belongs to are read in one atomic load and no fence
//    or counter orders them; two banks alternate by exchange, so a slot is not
//    rewritten while another workgroup may still wait on it;
//  * then one uint32, the last exchange number used: a walk numbers its exchanges
//    from there, so slots left by earlier walks never match (a walk that timed out
//    moves the base past every number it may have used).
// slots (two 512-byte banks), then the base in a 256-byte tail: a record is 1,280 bytes,
// so every bank starts on a 256-byte boundary and no cache line holds two sequences'
// slots
constexpr int kRecWords = kSlots + 32;
inline size_t walk_workspace_bytes(int num_seqs) {
  const size_t n = num_seqs > 0 ? (size_t)num_seqs : 0;
  return (n * kRecWords * sizeof(uint64_t) + 255) & ~(size_t)255;
}

struct Coop {
  uint64_t* slots;  // this sequence's slots (K > 1)
  uint32_t* base;   // this sequence's exchange base (K > 1)
  int K, k;         // workgroups per sequence, this one's rank
  uint32_t n;       // last exchange number
  int* s_flag;      // LDS: set when a wait timed out
  // All-to-all exchange among the sequence's K workgroups (every workgroup calls it
  // the same number of times): this workgroup's values buf[lo .. lo + cnt) are
  // published, and on return buf[0 .. total) holds every workgroup's values.  buf is
  // in LDS.  Wave 0 publishes and waits, one slot per lane.
  __device__ void exchange(uint32_t* buf, int lo, int cnt, int total) {
    __syncthreads();
    ++n;
    if (threadIdx.x < 64) {
      const int lane = threadIdx.x;
      uint64_t* bank = slots + kLW * (n & 1u);
      const uint64_t tag = (uint64_t)n << 32;
      if (lane < cnt)
        __hip_atomic_store(bank + lo + lane, tag | buf[lo + lane], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      if (lane < total) {
        uint64_t v = 0;
        uint32_t spins = 0;
        while (((v = __hip_atomic_load(bank + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) >>
                32) != (uint64_t)n) {
          if (++spins > kMaxSpins) {
            *s_flag = 1;
            v = 0;
            break;
          }
          __builtin_amdgcn_s_sleep(1);
        }
        buf[lane] = (uint32_t)v;
      }
    }
    __syncthreads();
  }
};

// Residual values from raw loads (full subtiles, MODE fixed at compile time).
template <int MODE, typename PRow>
__device__ __forceinline__ void residual_raw(const PRow& prow, const typename PRow::Raw& pr,
                                             const F32x8& qr, int y0, const PassSpec& ps,
                                             float v[8]) {
  float p[8];
  prow.values(pr, p);
  if constexpr (MODE == kResid) {
    float q[8];
    unpack8f(qr, q);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = fmaxf(p[e] - ps.c * q[e], 0.f);
  } else if constexpr (MODE == kDelta) {
    uint32_t zero = 0;
    for (int i = 0; i < ps.nR; ++i) {
      const uint32_t d = (uint32_t)(ps.R[i] - y0);
      if (d < 8u) zero |= 1u << d;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = ((zero >> e) & 1u) ? 0.f : p[e];
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = p[e];
  }
}

// Lane sum of one logical wave's subtiles [jlo, jhi): the lane's values in order.
// Subtiles wholly inside the row take unguarded 16-byte loads, kBatch in flight;
// the row's last partial subtile (or rows without vector loads) the guarded path.
template <int MODE, typename PRow>
__device__ __forceinline__ float lane_sum(const PRow& prow, const float* qrow, int V, bool vp,
                                          bool vq, const PassSpec& ps, int jlo, int jhi) {
  const int lane = threadIdx.x & 63;
  const bool fast = vp && (MODE != kResid || vq);
  const int jfull = fast ? max(jlo, min(jhi, V / kSub)) : jlo;
  float L = 0.f;
  for (int jb = jlo; jb < jfull; jb += kBatch) {
    typename PRow::Raw pr[kBatch];
    F32x8 qr[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      if (jb + u < jfull) {
        const int y0 = (jb + u) * kSub + lane * 8;
        pr[u] = prow.fetch(y0);
        if constexpr (MODE == kResid) qr[u] = raw8f(qrow, y0);
      }
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      if (jb + u < jfull) {
        float v[8];
        residual_raw<MODE>(prow, pr[u], qr[u], (jb + u) * kSub + lane * 8, ps, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) L = L + v[e];
      }
    }
  }
  for (int j = jfull; j < jhi; ++j) {
    float v[8];
    residual8(prow, qrow, j * kSub + lane * 8, V, vp, vq, ps, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) L = L + v[e];
  }
  return L;
}

// The wave's lane chain E_l = E_{l-1} + L_l in lane order; returns E for this lane
// and leaves the total E_63 in *T (every lane).
__device__ __forceinline__ float lane_chain(float L, float* T) {
  const int lane = threadIdx.x & 63;
  const int Lbits = __float_as_int(L);
  float run = 0.f, E = 0.f;
#pragma unroll
  for (int l = 0; l < 64; ++l) {
    run = run + __int_as_float(__builtin_amdgcn_readlane(Lbits, l));
    E = lane == l ? run : E;
  }
  *T = run;
  return E;
}

// The row chain over the 64 logical wave totals t_lds[0..63], in every wave: returns
// the row total W_64 and leaves in *wpre lane w's exclusive prefix W_w = t_0 + ... +
// t_{w-1} (the same sequential sum from 0).
__device__ __forceinline__ float row_chain(const float* t_lds, float* wpre) {
  const int lane = threadIdx.x & 63;
  const int tbits = __float_as_int(t_lds[lane]);
  float run = 0.f, W = 0.f;
#pragma unroll
  for (int l = 0; l < 64; ++l) {
    W = lane == l ? run : W;
    run = run + __int_as_float(__builtin_amdgcn_readlane(tbits, l));
  }
  *wpre = W;
  return run;
}

// One pass over the row (spec mode MODE).  Fills t_lds[0..63] with the 64 logical
// wave totals (exchanged between the workgroups of the sequence) and returns the
// row total W_64 (every thread); ends[i] is this lane's chain value E_l in the wave's
// i-th logical wave, *wpre the row chain's prefix for logical wave `lane`.
template <int MODE, int NW, int M, typename PRow>
__device__ float chain_pass(const PRow& prow, const float* qrow, int V, bool vp, bool vq,
                            const PassSpec& ps, float* t_lds, float (&ends)[M], float* wpre,
                            Coop& co) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const Layout lay(V);
  const int lw0 = (co.k * NW + wave) * M;
#pragma unroll
  for (int i = 0; i < M; ++i) {
    const float L = lane_sum<MODE>(prow, qrow, V, vp, vq, ps, lay.lo(lw0 + i), lay.hi(lw0 + i));
    float T;
    ends[i] = lane_chain(L, &T);
    if (lane == 0) t_lds[lw0 + i] = T;
  }
  if (NW * M < kLW)
    co.exchange(reinterpret_cast<uint32_t*>(t_lds), co.k * kLW / co.K, kLW / co.K, kLW);
  else
    __syncthreads();
  return row_chain(t_lds, wpre);
}

// Largest y with v(y) > 0 over the sequence's row (-1 if none): the pick's fallback
// when u * total rounds to the total.
template <int MODE, int NW, int M, typename PRow>
__device__ int last_positive(const PRow& prow, const float* qrow, int V, bool vp, bool vq,
                             const PassSpec& ps, int* s_int, uint32_t* s_x, Coop& co) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const Layout lay(V);
  const int lw0 = (co.k * NW + wave) * M;
  int last = -1;
  for (int j = lay.lo(lw0); j < lay.hi(lw0 + M - 1); ++j) {
    float v[8];
    residual8(prow, qrow, j * kSub + lane * 8, V, vp, vq, ps, v);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (v[e] > 0.f) last = j * kSub + lane * 8 + e;
  }
  last = nvx::block_max_i<NW * 64>(last, s_int);
  if (NW * M < kLW) {
    if (threadIdx.x == 0) s_x[co.k] = (uint32_t)last;
    co.exchange(s_x, co.k, 1, co.K);
    for (int r = 0; r < co.K; ++r) last = max(last, (int)s_x[r]);
  }
  return last;
}

// Inverse-CDF pick over the values of the last chain_pass (same spec), whose `ends`
// and row-chain prefix `wpre` are passed in.  Every workgroup of the sequence returns the pick; the
// workgroup that resolved it returns it with *owner = true.  s_int holds NW + 1 ints.
template <int MODE, int NW, int M, typename PRow>
__device__ int chain_pick(const PRow& prow, const float* qrow, int V, bool vp, bool vq,
                          const PassSpec& ps, float wpre, const float (&ends)[M], float total,
                          float u, int* s_int, uint32_t* s_x, Coop& co, bool* owner) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const Layout lay(V);
  const int lw0 = (co.k * NW + wave) * M;
  const float tau = u * total;
  int cand = INT32_MAX;
  float Wi[M];
#pragma unroll
  for (int i = 0; i < M; ++i) {
    Wi[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wpre), lw0 + i));
    const uint64_t m = __ballot((Wi[i] + ends[i]) > tau);
    if (cand == INT32_MAX && m) cand = (lw0 + i) * 64 + __ffsll((unsigned long long)m) - 1;
  }
  int gstar = nvx::block_min_i<NW * 64>(cand, s_int);
  if (NW * M < kLW) {
    if (threadIdx.x == 0) s_x[co.k] = (uint32_t)gstar;
    co.exchange(s_x, co.k, 1, co.K);
    for (int r = 0; r < co.K; ++r) gstar = min(gstar, (int)s_x[r]);
  }
  *owner = false;
  if (gstar == INT32_MAX) {
    const int y = last_positive<MODE, NW, M>(prow, qrow, V, vp, vq, ps, s_int, s_x, co);
    *owner = co.k == 0;
    return y;
  }
  const int lw = gstar / 64, l = gstar % 64;
  const bool mine = lw >= co.k * NW * M && lw < (co.k + 1) * NW * M;
  *owner = mine;
  if (!mine) return -1;
  if (wave == (lw - co.k * NW * M) / M) {  // the owning real wave resolves the element
    const int i = lw - lw0;
    float e_lane = 0.f, w_start = 0.f;
#pragma unroll
    for (int t = 0; t < M; ++t)
      if (t == i) {
        e_lane = ends[t];
        w_start = Wi[t];
      }
    const float e_before = __shfl(e_lane, l > 0 ? l - 1 : 0, 64);
    float run = l > 0 ? w_start + e_before : w_start;
    // lane kk loads lane l's elements of the logical wave's kk-th subtile
    const int jlo = lay.lo(lw), nk = lay.hi(lw) - jlo;
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (lane < nk) residual8(prow, qrow, (jlo + lane) * kSub + l * 8, V, vp, vq, ps, v);
    int first = -1, last = -1;
    for (int kk = 0; kk < nk; ++kk) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[e]), kk));
        run = run + x;
        if (x > 0.f) {
          const int y = (jlo + kk) * kSub + l * 8 + e;
          if (first < 0 && run > tau) first = y;
          last = y;
        }
      }
    }
    if (lane == 0) s_int[NW] = first >= 0 ? first : last;
  }
  __syncthreads();
  const int r = s_int[NW];
  __syncthreads();
  return r;
}

// First index of the row maximum (this workgroup's logical waves, then across the
// sequence's workgroups).
template <int NW, int M, typename PRow>
__device__ int walk_argmax(const PRow& row, int V, bool vec, float* red, int* redi, uint32_t* s_x,
                           Coop& co) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const Layout lay(V);
  float bv = -INFINITY;
  int bi = INT32_MAX;
  const int lw0 = (co.k * NW + wave) * M;
  for (int j = lay.lo(lw0); j < lay.hi(lw0 + M - 1); ++j) {
    const int y0 = j * kSub + lane * 8;
    if (y0 >= V) break;
    float p[8];
    row.load8(y0, V, vec, p);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int y = y0 + e;
      if (y < V && (p[e] > bv || (p[e] == bv && y < bi))) {
        bv = p[e];
        bi = y;
      }
    }
  }
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
    red[wave] = bv;
    redi[wave] = bi;
  }
  __syncthreads();
  bv = red[lane < NW ? lane : 0];
  bi = redi[lane < NW ? lane : 0];
#pragma unroll
  for (int off = NW / 2; off >= 1; off >>= 1) {
    const float ov = nvx::shfl_xor_f(bv, off);
    const int oi = nvx::shfl_xor_i(bi, off);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  __syncthreads();
  bv = __shfl(bv, 0, 64);
  bi = __shfl(bi, 0, 64);
  if (NW * M < kLW) {
    if (threadIdx.x == 0) {
      s_x[2 * co.k] = __float_as_uint(bv);
      s_x[2 * co.k + 1] = (uint32_t)bi;
    }
    co.exchange(s_x, 2 * co.k, 2, 2 * co.K);
    for (int r = 0; r < co.K; ++r) {
      const float ov = __uint_as_float(s_x[2 * r]);
      const int oi = (int)s_x[2 * r + 1];
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
  }
  return bi == INT32_MAX ? 0 : bi;
}

// Largest value of the sequence's row (this workgroup's logical waves, then across
// the sequence's workgroups).  The max is exact in any order.
template <int NW, int M, typename PRow>
__device__ float walk_rowmax(const PRow& row, int V, bool vec, float* red, uint32_t* s_x, Coop& co) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const Layout lay(V);
  float m = -INFINITY;
  const int lw0 = (co.k * NW + wave) * M;
  for (int j = lay.lo(lw0); j < lay.hi(lw0 + M - 1); ++j) {
    const int y0 = j * kSub + lane * 8;
    if (y0 >= V) break;
    float p[8];
    row.load8(y0, V, vec, p);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (y0 + e < V) m = fmaxf(m, p[e]);
  }
  m = nvx::block_max<NW * 64>(m, red);
  if (NW * M < kLW) {
    if (threadIdx.x == 0) s_x[co.k] = __float_as_uint(m);
    co.exchange(s_x, co.k, 1, co.K);
    for (int r = 0; r < co.K; ++r) m = fmaxf(m, __uint_as_float(s_x[r]));
  }
  return m;
}

struct WalkArgs {
  const float* Q;
  int64_t q_seq_stride;
  int V;
  const int32_t* tokens;
  const int32_t* parents;
  const int32_t* num_nodes;
  int node_stride;
  const float* U;
  const float* U_final;
  const uint8_t* greedy_flags;
  int delta;
  int32_t* path_out;
  int32_t* acc_out;
  int32_t* tok_out;
  int32_t* next_out;
  bool vp, vq;
  uint64_t* ex;  // exchange records [num_seqs, kRecWords] (multi-workgroup walks)
};

__device__ void write_walk(const WalkArgs& a, int b, bool failed, int depth, int next,
                           const int* s_path, const int* s_tok) {
  const int64_t ob = (int64_t)b * a.node_stride;
  for (int i = threadIdx.x; i < a.node_stride; i += (int)blockDim.x) {
    a.path_out[ob + i] = (!failed && i <= depth) ? s_path[i] : -1;
    int t = -1;
    if (!failed && i < depth) t = s_tok[s_path[i + 1]];
    else if (!failed && i == depth) t = next;
    a.tok_out[ob + i] = t;
  }
  if (threadIdx.x == 0) {
    a.acc_out[b] = failed ? -1 : depth;
    a.next_out[b] = failed ? -1 : next;
  }
}

// The walk of sequence blockIdx.x / K by K workgroups (see Layout / Coop).  Every
// wave holds the tree in registers, lane j node j: its parent, token and uniform, and
// the two values its acceptance test reads, p(x_j) and q(x_j) on its parent's row,
// loaded once when the walk starts; a node's children (in index order) are a ballot.
template <typename Src, int K>
__global__ __launch_bounds__(walk_nw(K) * 64) __attribute__((amdgpu_waves_per_eu(4)))
void rejection_walk_kernel(Src src, WalkArgs a) {
  constexpr int NW = walk_nw(K), M = walk_m(K);
  __shared__ float red[NW];
  __shared__ int redi[NW + 1];
  __shared__ float t_lds[kLW];
  __shared__ int s_tok[kMaxNodes], s_path[kMaxNodes];
  __shared__ int s_R[kMaxNodes];
  __shared__ int s_flag;
  __shared__ uint32_t s_x[2 * kMaxWidth];  // exchanges of the picks and argmaxes
  __shared__ uint32_t s_fx[kMaxWidth];     // the closing exchange of time-out flags

  const int lane = threadIdx.x & 63;
  const int b = blockIdx.x / K;
  uint64_t* const rec = K > 1 ? a.ex + (size_t)b * kRecWords : nullptr;
  Coop co{rec, K > 1 ? reinterpret_cast<uint32_t*>(rec + kSlots) : nullptr, K,
          (int)(blockIdx.x % K), 0u, &s_flag};
  if (K > 1) co.n = __hip_atomic_load(co.base, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int V = a.V;
  int T = a.node_stride;
  if (a.num_nodes) T = max(1, min(a.num_nodes[b], a.node_stride));
  const bool greedy = a.greedy_flags ? a.greedy_flags[b] != 0 : false;
  const bool dmode = a.delta != 0;
  const float uf = a.U_final[b];
  const bool vp = a.vp, vq = a.vq;
  const int64_t nb = (int64_t)b * a.node_stride;

  int par_l = -1, tok_l = 0;
  float u_l = 0.f, px_l = 0.f, qx_l = 1.f;
  if (lane < T) {
    par_l = a.parents[nb + lane];
    tok_l = a.tokens[nb + lane];
    u_l = a.U[nb + lane];
  }
  // only children of an earlier node are ever tested (the walk moves to higher indices)
  const bool tested =
      !greedy && lane >= 1 && lane < T && par_l >= 0 && par_l < lane && tok_l >= 0 && tok_l < V;
  if (tested) {
    // with lazy statistics p(x) is read when the walk reaches the parent
    if constexpr (!Src::kLazy) px_l = src.row(b, par_l).at(tok_l);
    if (!dmode) qx_l = a.Q[(int64_t)b * a.q_seq_stride + (int64_t)par_l * V + tok_l];
  }
  if (threadIdx.x < T) s_tok[threadIdx.x] = tok_l;
  if (threadIdx.x == 0) {
    s_flag = 0;
    s_path[0] = 0;
  }
  __syncthreads();

  int cur = 0, depth = 0, next = 0;
  bool owner = co.k == 0;
  while (true) {
    const auto prow = [&]() {
      if constexpr (Src::kLazy) {
        // the statistics of this node's row, computed on arrival: the exact max, then
        // the canonical sum of exp2(fma(x, a, -max)); greedy rows pass the logits
        // through and need none
        float Mx = 0.f, inv = 0.f;
        const float sc = src.scale(b, cur);
        if (!greedy && __builtin_isfinite(sc)) {
          Mx = walk_rowmax<NW, M>(src.raw_row(b, cur), V, vp, red, s_x, co) * sc;
          float ends_s[M], wpre_s;
          const PassSpec ps{kPlain, 0.f, nullptr, 0};
          const float sum = chain_pass<kPlain, NW, M>(src.row(b, cur, Mx, 1.f), nullptr, V, vp, vq, ps,
                                                      t_lds, ends_s, &wpre_s, co);
          __syncthreads();  // t_lds read by every thread before it can change
          inv = 1.f / sum;
          if (co.k == 0 && threadIdx.x == 0 && src.stats_out)
            src.stats_out[src.index(b, cur)] = make_float2(Mx, inv);
        }
        const auto r = src.row(b, cur, Mx, inv);
        if (tested && par_l == cur) px_l = r.at(tok_l);
        return r;
      } else {
        return src.row(b, cur);
      }
    }();
    const float* qrow = a.Q ? a.Q + (int64_t)b * a.q_seq_stride + (int64_t)cur * V : nullptr;
    uint64_t kids = __ballot(par_l == cur && lane > cur);
    int accepted = -1;
    if (greedy) {
      const int am = walk_argmax<NW, M>(prow, V, vp, red, redi, s_x, co);
      const uint64_t hit = kids & __ballot(tok_l == am);
      if (hit) {
        accepted = __ffsll((unsigned long long)hit) - 1;
      } else {
        next = am;
        owner = co.k == 0;
        break;
      }
    } else {
      // current distribution cur[y] = v(y) / Z, v per the pass spec; `have` says the
      // last chain_pass (ends, wpre, total) describes the current v
      float c = 0.f, Z = 1.f, total = 0.f, wpre = 0.f;
      float ends[M];
#pragma unroll
      for (int i = 0; i < M; ++i) ends[i] = 0.f;
      int nR = 0;
      bool have = false;
      while (kids) {
        const int j = __ffsll((unsigned long long)kids) - 1;
        kids &= kids - 1;
        const int x = __builtin_amdgcn_readlane(tok_l, j);
        const bool valid = x >= 0 && x < V;
        const float px = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(px_l), j));
        const float uj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(u_l), j));
        float cx = 0.f, qx = 1.f;
        if (valid) {
          if (dmode) {
            cx = (nR > 0 && in_set(s_R, nR, x) ? 0.f : px) / Z;
          } else {
            qx = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(qx_l), j));
            cx = fmaxf(px - c * qx, 0.f) / Z;
          }
        }
        if (uj * qx <= cx && cx > 0.f) {
          accepted = j;
          break;
        }
        if (dmode) {
          if (valid && !(nR > 0 && in_set(s_R, nR, x))) {
            __syncthreads();  // every lane has read s_R
            if (threadIdx.x == 0) s_R[nR] = x;
            __syncthreads();
            nR += 1;
            Z = Z - px;
          }
          if (!(Z > 0.f)) {
            nR = 0;
            Z = 1.f;
          }
        } else {
          const float cn = c + Z;
          const PassSpec ps{kResid, cn, nullptr, 0};
          const float Zn = chain_pass<kResid, NW, M>(prow, qrow, V, vp, vq, ps, t_lds, ends, &wpre, co);
          if (Zn > 0.f) {
            c = cn;
            Z = Zn;
            total = Zn;
            have = true;
          } else {
            c = 0.f;
            Z = 1.f;
            have = false;
          }
          __syncthreads();  // t_lds read by every thread before it can change
        }
        if (s_flag) break;
      }
      if (s_flag) break;
      if (accepted < 0) {
        const PassSpec ps = have ? PassSpec{kResid, c, nullptr, 0}
                                 : PassSpec{dmode && nR > 0 ? kDelta : kPlain, 0.f, s_R, nR};
        if (have) {
          next = chain_pick<kResid, NW, M>(prow, qrow, V, vp, vq, ps, wpre, ends, total, uf, redi, s_x,
                                       co, &owner);
        } else if (ps.mode == kDelta) {
          total = chain_pass<kDelta, NW, M>(prow, qrow, V, vp, vq, ps, t_lds, ends, &wpre, co);
          next = chain_pick<kDelta, NW, M>(prow, qrow, V, vp, vq, ps, wpre, ends, total, uf, redi, s_x,
                                       co, &owner);
        } else {
          total = chain_pass<kPlain, NW, M>(prow, qrow, V, vp, vq, ps, t_lds, ends, &wpre, co);
          next = chain_pick<kPlain, NW, M>(prow, qrow, V, vp, vq, ps, wpre, ends, total, uf, redi, s_x,
                                       co, &owner);
        }
        break;
      }
    }
    if (s_flag) break;
    cur = accepted;
    depth += 1;
    if (threadIdx.x == 0) s_path[depth] = cur;
  }
  // The sequence's workgroups agree whether any wait timed out (the sequence's
  // workgroups failed to meet): then path = tokens = -1, accepted_len = next_token =
  // -1, written by workgroup 0.
  if (K > 1) {
    if (threadIdx.x == 0) s_fx[co.k] = (uint32_t)s_flag;
    co.exchange(s_fx, co.k, 1, K);
    uint32_t any = 0;
    for (int r = 0; r < K; ++r) any |= s_fx[r];
    if (any) {
      __syncthreads();
      if (threadIdx.x == 0) s_flag = 1;
      __syncthreads();
    }
  } else {
    __syncthreads();
  }
  const bool failed = s_flag != 0;
  if (failed) owner = co.k == 0;
  if (owner) write_walk(a, b, failed, depth, next, s_path, s_tok);
  if (K > 1 && co.k == 0 && threadIdx.x == 0)
    __hip_atomic_store(co.base, co.n + (failed ? kFailSkip : 0u), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// Workgroups a device holds at once of rejection_walk_kernel<Src, K> (0 if unknown),
// cached per device.
template <typename Src, int K>
int64_t walk_resident(int dev) {
  static std::atomic<int64_t> cache[64];
  if (dev < 0 || dev >= 64) return 0;
  int64_t r = cache[dev].load(std::memory_order_relaxed);
  if (r > 0) return r;
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &per_cu, reinterpret_cast<const void*>(rejection_walk_kernel<Src, K>), walk_nw(K) * 64,
          0) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  r = (int64_t)cus * per_cu;
  cache[dev].store(r, std::memory_order_relaxed);
  return r;
}

// Upper bound on the workgroups per sequence (nvx_rejection_walk_max_width).
std::atomic<int> g_walk_max_width{kMaxWidth};

// Workgroups per sequence for a walk of num_seqs sequences: the largest of 16, 8, 4
// and 2 (at most the set bound) for which all the walk's workgroups fit on the device
// at once, when the caller gave an exchange workspace and the stream is not being
// captured; else 1.  More workgroups per
// sequence spread one sequence's row passes over more CUs (same total waves), which
// shortens the passes of the sequences that are still walking when the others are
// done.  The K workgroups of a sequence wait for each other, so they must all be
// running together: a grid no larger than what the device holds at once is
// dispatched whole once the device's earlier work drains.  Should a sequence's
// workgroups still fail to meet (a device shared with a kernel that never ends),
// the bounded waits end the walk with the failure outputs rather than a hang.
template <typename Src>
int walk_width(int num_seqs, hipStream_t s, bool have_workspace) {
  if (!have_workspace) return 1;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) {
    (void)hipGetLastError();
    return 1;
  }
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return 1;
  }
  const int wmax = g_walk_max_width.load(std::memory_order_relaxed);
  if (wmax >= 16 && (int64_t)num_seqs * 16 <= walk_resident<Src, 16>(dev)) return 16;
  if (wmax >= 8 && (int64_t)num_seqs * 8 <= walk_resident<Src, 8>(dev)) return 8;
  if (wmax >= 4 && (int64_t)num_seqs * 4 <= walk_resident<Src, 4>(dev)) return 4;
  if (wmax >= 2 && (int64_t)num_seqs * 2 <= walk_resident<Src, 2>(dev)) return 2;
  return 1;
}

template <typename Src>
hipError_t launch_walk(const Src& src, const WalkArgs& a, int num_seqs, hipStream_t s) {
#define NVX_WALK(K)                                                                          \
  hipLaunchKernelGGL((rejection_walk_kernel<Src, K>), dim3(num_seqs * K), dim3(walk_nw(K) * 64), 0, \
                     s, src, a)
  switch (walk_width<Src>(num_seqs, s, a.ex != nullptr)) {
    case 16: NVX_WALK(16); break;
    case 8: NVX_WALK(8); break;
    case 4: NVX_WALK(4); break;
    case 2: NVX_WALK(2); break;
    default: NVX_WALK(1);
  }
#undef NVX_WALK
  return hipGetLastError();
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }
// The row statistics are read and written as float2 (max, 1/sum) pairs.
inline bool aligned8(const void* p) { return ((uintptr_t)p & 7) == 0; }

// The exchange records of a walk in the caller's workspace: NULL means no exchange
// (one workgroup per sequence); otherwise it must hold walk_workspace_bytes(num_seqs)
// and be 8-byte aligned.  Reports a bad workspace and returns false.
bool walk_exchange(const char* who, void* ws, size_t bytes, int num_seqs, uint64_t** ex) {
  *ex = nullptr;
  if (!ws) return true;
  const size_t need = walk_workspace_bytes(num_seqs);
  if (bytes < need) {
    nvx::fail(NVX_EINVAL, "%s: exchange workspace of %zu bytes required for %d sequences (got %zu)",
              who, need, num_seqs, bytes);
    return false;
  }
  if (!aligned8(ws)) {
    nvx::fail(NVX_EINVAL, "%s: the exchange workspace must be 8-byte aligned", who);
    return false;
  }
  *ex = static_cast<uint64_t*>(ws);
  return true;
}

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

extern "C" size_t nvx_rejection_walk_workspace_size(int32_t num_seqs) {
  return walk_workspace_bytes(num_seqs);
}

extern "C" int nvx_rejection_walk_max_width(int32_t max_width) {
  nvx::clear_error();
  NVX_CHECK(max_width >= 1 && max_width <= kMaxWidth,
            "rejection_walk_max_width: %d is outside [1, %d]", max_width, kMaxWidth);
  int w = 1;
  while (w * 2 <= max_width) w *= 2;
  return g_walk_max_width.exchange(w);
}

extern "C" int nvx_rejection_sample_tree(const float* target_probs, int64_t p_seq_stride,
                                         const float* draft_probs, int64_t q_seq_stride, int32_t vocab,
                                         const int32_t* tokens, const int32_t* parents,
                                         const int32_t* num_nodes, int32_t node_stride,
                                         const float* uniforms, const float* final_uniforms,
                                         const uint8_t* greedy, int32_t draft_mode, int32_t num_seqs,
                                         int32_t* path, int32_t* accepted_len, int32_t* out_tokens,
                                         int32_t* next_token, void* workspace,
                                         size_t workspace_bytes, void* stream) {
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
  NVX_CHECK(vocab <= kMaxVocab, "rejection_sample_tree: vocab %d exceeds %d", vocab, kMaxVocab);
  uint64_t* ex = nullptr;
  if (!walk_exchange("rejection_sample_tree", workspace, workspace_bytes, num_seqs, &ex))
    return NVX_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  nvx::TimerScope timer(NVX_TIMER_REJECTION, s);
  const bool vp = vocab % 4 == 0 && p_seq_stride % 4 == 0 && aligned16(target_probs);
  const bool vq = draft_mode == 1 ||
                  (vocab % 4 == 0 && q_seq_stride % 4 == 0 && aligned16(draft_probs));
  const WalkArgs wa{draft_mode == 1 ? nullptr : draft_probs, q_seq_stride, vocab, tokens, parents,
                    num_nodes, node_stride, uniforms, final_uniforms, greedy, draft_mode, path,
                    accepted_len, out_tokens, next_token, vp, vq, ex};
  NVX_HIP(launch_walk(ProbSource{target_probs, p_seq_stride, vocab}, wa, num_seqs, s));
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
    int32_t* out_tokens, int32_t* next_token, void* workspace, size_t workspace_bytes,
    void* stream) {
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
  NVX_CHECK(vocab <= kMaxVocab, "rejection_sample_tree_logits: vocab %d exceeds %d", vocab,
            kMaxVocab);
  uint64_t* ex = nullptr;
  if (!walk_exchange("rejection_sample_tree_logits", workspace, workspace_bytes, num_seqs, &ex))
    return NVX_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  nvx::TimerScope timer(NVX_TIMER_REJECTION, s);
  const bool bf16 = logits_dtype == NVX_DTYPE_BF16;
  const int per = bf16 ? 8 : 4;  // elements per 16 bytes
  const bool vp = vocab % per == 0 && logits_row_stride % per == 0 && aligned16(logits);
  const bool vq = draft_mode == 1 ||
                  (vocab % 4 == 0 && q_seq_stride % 4 == 0 && aligned16(draft_probs));
  const float2* st = reinterpret_cast<const float2*>(stats);
  const WalkArgs wa{draft_mode == 1 ? nullptr : draft_probs, q_seq_stride, vocab, tokens, parents,
                    num_nodes, node_stride, uniforms, final_uniforms, greedy, draft_mode, path,
                    accepted_len, out_tokens, next_token, vp, vq, ex};
  if (bf16)
    NVX_HIP(launch_walk(LogitSource<uint16_t>{(const uint16_t*)logits, logits_row_stride,
                                              node_stride, temperatures, st},
                        wa, num_seqs, s));
  else
    NVX_HIP(launch_walk(LogitSource<float>{(const float*)logits, logits_row_stride, node_stride,
                                           temperatures, st},
                        wa, num_seqs, s));
  return NVX_OK;
}

extern "C" int nvx_rejection_sample_tree_logits_lazy(
    const void* logits, int32_t logits_dtype, int64_t logits_row_stride,
    const float* temperatures, float* stats_out, const float* draft_probs, int64_t q_seq_stride,
    int32_t vocab, const int32_t* tokens, const int32_t* parents, const int32_t* num_nodes,
    int32_t node_stride, const float* uniforms, const float* final_uniforms, const uint8_t* greedy,
    int32_t draft_mode, int32_t num_seqs, int32_t* path, int32_t* accepted_len,
    int32_t* out_tokens, int32_t* next_token, void* workspace, size_t workspace_bytes,
    void* stream) {
  nvx::clear_error();
  NVX_CHECK(logits_dtype == NVX_DTYPE_F32 || logits_dtype == NVX_DTYPE_BF16,
            "rejection_sample_tree_logits_lazy: logits must be fp32 or bf16 (dtype code %d)",
            logits_dtype);
  NVX_CHECK(num_seqs >= 0 && vocab >= 1 && logits_row_stride >= vocab,
            "rejection_sample_tree_logits_lazy: bad sizes (seqs=%d, vocab=%d, stride=%lld)",
            num_seqs, vocab, (long long)logits_row_stride);
  NVX_CHECK(node_stride >= 1 && node_stride <= kMaxNodes,
            "rejection_sample_tree_logits_lazy: node_stride must be in [1, %d] (got %d)", kMaxNodes,
            node_stride);
  NVX_CHECK(draft_mode == 0 || draft_mode == 1,
            "rejection_sample_tree_logits_lazy: draft_mode must be 0 or 1");
  NVX_CHECK(draft_mode == 1 || draft_probs != nullptr,
            "rejection_sample_tree_logits_lazy: draft_probs required in draft_mode 0");
  if (num_seqs == 0) return NVX_OK;
  NVX_CHECK(logits && temperatures && tokens && parents && uniforms && final_uniforms && path &&
                accepted_len && out_tokens && next_token,
            "rejection_sample_tree_logits_lazy: null pointer");
  NVX_CHECK(stats_out == nullptr || aligned8(stats_out),
            "rejection_sample_tree_logits_lazy: stats_out must be 8-byte aligned");
  NVX_CHECK(vocab <= kMaxVocab, "rejection_sample_tree_logits_lazy: vocab %d exceeds %d", vocab,
            kMaxVocab);
  uint64_t* ex = nullptr;
  if (!walk_exchange("rejection_sample_tree_logits_lazy", workspace, workspace_bytes, num_seqs,
                     &ex))
    return NVX_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  nvx::TimerScope timer(NVX_TIMER_REJECTION, s);
  const bool bf16 = logits_dtype == NVX_DTYPE_BF16;
  const int per = bf16 ? 8 : 4;  // elements per 16 bytes
  const bool vp = vocab % per == 0 && logits_row_stride % per == 0 && aligned16(logits);
  const bool vq = draft_mode == 1 ||
                  (vocab % 4 == 0 && q_seq_stride % 4 == 0 && aligned16(draft_probs));
  float2* st = reinterpret_cast<float2*>(stats_out);
  const WalkArgs wa{draft_mode == 1 ? nullptr : draft_probs, q_seq_stride, vocab, tokens, parents,
                    num_nodes, node_stride, uniforms, final_uniforms, greedy, draft_mode, path,
                    accepted_len, out_tokens, next_token, vp, vq, ex};
  if (bf16)
    NVX_HIP(launch_walk(LazyLogitSource<uint16_t>{(const uint16_t*)logits, logits_row_stride,
                                                  node_stride, temperatures, st},
                        wa, num_seqs, s));
  else
    NVX_HIP(launch_walk(LazyLogitSource<float>{(const float*)logits, logits_row_stride,
                                               node_stride, temperatures, st},
                        wa, num_seqs, s));
  return NVX_OK;
}
