// Draft-head top-k: log-softmax and top-k over the vocabulary in one pass over HBM.
//
// EAGLE-2/3 tree expansion (arXiv:2406.16858) needs, for every draft row, the k
// most likely next tokens and their log-probabilities.  One workgroup streams one
// row of logits once (16-byte loads, four in flight per thread):
//  * each lane keeps an online max m and sum s = sum 2^(x*log2e - m*log2e);
//    the workgroup combines them at the end into M and S, and
//    logprob(x) = (x - M) - ln(S);
//  * each wave keeps its best k entries spread over lanes: lane j < k holds the
//    j-th largest 64-bit key  (order-preserving bits of the value) << 32 | ~index,
//    so a larger key ranks first and equal values rank by the lower token id.
//    A value can only enter when it is >= a threshold: the list's k-th value, and
//    from the start the k-th largest of the wave's first-vector lane maxima (k
//    distinct elements, so a lower bound of the row's k-th largest value).  After
//    the first vectors candidates are rare; each is inserted with one lane shift.
//  * the waves' lists meet in LDS, where each key's rank among them (the number
//    of larger keys) is its output slot.
// Rows must be free of NaN.  Outputs per row are ordered by descending
// log-probability, ties to the lower token id.
#include "nvx_internal.h"

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kUnroll = 4;
constexpr int kMaxK = 64;

// Monotone map of fp32 values (no NaN) to uint32: a < b  <=>  ord(a) < ord(b).
__device__ __forceinline__ uint32_t ord_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  return u ^ ((uint32_t)((int32_t)u >> 31) | 0x80000000u);
}
__device__ __forceinline__ float from_ord(uint32_t h) {
  return __uint_as_float(h ^ ((h & 0x80000000u) ? 0x80000000u : 0xffffffffu));
}
__device__ __forceinline__ uint64_t make_key(float x, int idx) {
  return ((uint64_t)ord_bits(x) << 32) | (uint32_t)~(uint32_t)idx;
}
__device__ __forceinline__ uint64_t readlane64(uint64_t v, int lane) {
  const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)v, lane);
  const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), lane);
  return ((uint64_t)hi << 32) | lo;
}

// k-th largest of the 64 lane values (bitonic sort, descending, across the wave).
__device__ __forceinline__ float wave_kth_largest(float v, int k, int lane) {
#pragma unroll
  for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const float o = nvx::shfl_xor_f(v, stride);
      const bool desc = (lane & size) == 0;
      const bool low = (lane & stride) == 0;
      v = (low == desc) ? fmaxf(v, o) : fminf(v, o);
    }
  }
  return __uint_as_float(__builtin_amdgcn_readlane((int)__float_as_uint(v), k - 1));
}

// One wave's top-k list (lanes 0..k-1, descending keys; 0 = empty slot).
struct WaveTopK {
  uint64_t key = 0;   // this lane's entry
  uint64_t kth = 0;   // the list's k-th key (wave uniform)
  float thr0;         // seeded lower bound of the row's k-th largest value
  float thr;          // admission threshold on values (wave uniform)
  int k, lane;

  __device__ void insert(uint64_t c) {
    const uint32_t plo = __shfl_up((uint32_t)key, 1, 64);
    const uint32_t phi = __shfl_up((uint32_t)(key >> 32), 1, 64);
    const uint64_t prev = lane == 0 ? ~0ull : (((uint64_t)phi << 32) | plo);
    const uint64_t nk = prev < c ? prev : (key < c ? c : key);
    if (lane < k) key = nk;
    kth = readlane64(key, k - 1);
    thr = kth ? fmaxf(thr0, from_ord((uint32_t)(kth >> 32))) : thr0;
  }

  // Offer one value per lane (lanes with ok == false offer nothing).  Called with
  // every lane of the wave active: insert() shifts the list across lanes.
  __device__ __forceinline__ void offer(float x, int idx, bool ok = true) {
    uint64_t cm = __ballot(ok && x >= thr);
    while (cm) {
      const int src = __builtin_ctzll(cm);
      cm &= cm - 1;
      const float cx = __uint_as_float(__builtin_amdgcn_readlane((int)__float_as_uint(x), src));
      const int ci = __builtin_amdgcn_readlane(idx, src);
      const uint64_t c = make_key(cx, ci);
      if (c > kth) insert(c);
    }
  }
};

template <typename VT, int NT>
__global__ __launch_bounds__(NT) void topk_logprobs_kernel(const VT* __restrict__ logits,
                                                           int64_t stride, int V, int k,
                                                           int32_t* __restrict__ out_tok,
                                                           float* __restrict__ out_lp) {
  using Tr = nvx::VecTraits<VT>;
  constexpr int P = Tr::kPer;
  constexpr int NW = NT / nvx::kWave;
  __shared__ float red[NW];
  __shared__ uint64_t lists[NW * kMaxK];
  const int row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const uint4* src = reinterpret_cast<const uint4*>(logits + (int64_t)row * stride);
  const int nvec = V / P;

  WaveTopK tk;
  tk.k = k;
  tk.lane = lane;
  {
    float lm = -INFINITY;
    if (tid < nvec) {
      float x[P];
      Tr::expand(src[tid], x);
#pragma unroll
      for (int e = 0; e < P; ++e) lm = fmaxf(lm, x[e]);
    }
    tk.thr0 = wave_kth_largest(lm, k, lane);
    tk.thr = tk.thr0;
  }

  // Lane l of wave w reads vectors w*64 + l + t*NT, t = 0, 1, ...; the loops run on
  // the wave's first vector j so that every lane takes every iteration.
  float m = -INFINITY, m2 = -INFINITY, s = 0.f;
  int j = wid * nvx::kWave;
  for (; j + (nvx::kWave - 1) + (kUnroll - 1) * NT < nvec; j += kUnroll * NT) {
    const int i = j + lane;
    uint4 w[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) w[u] = nvx::ld_stream(src + i + u * NT);
    float x[kUnroll][P];
    float lm = -INFINITY;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      Tr::expand(w[u], x[u]);
#pragma unroll
      for (int e = 0; e < P; ++e) lm = fmaxf(lm, x[u][e]);
    }
    if (lm > m) {
      const float m2n = lm * kLog2e;
      s = (m == -INFINITY) ? 0.f : s * __builtin_amdgcn_exp2f(m2 - m2n);
      m = lm;
      m2 = m2n;
    }
    if (m != -INFINITY) {
      float a0 = 0.f, a1 = 0.f;
#pragma unroll
      for (int u = 0; u < kUnroll; ++u)
#pragma unroll
        for (int e = 0; e < P; e += 2) {
          a0 += __builtin_amdgcn_exp2f(__builtin_fmaf(x[u][e], kLog2e, -m2));
          a1 += __builtin_amdgcn_exp2f(__builtin_fmaf(x[u][e + 1], kLog2e, -m2));
        }
      s += a0 + a1;
    }
    if (__ballot(lm >= tk.thr)) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u)
#pragma unroll
        for (int e = 0; e < P; ++e) tk.offer(x[u][e], (i + u * NT) * P + e);
    }
  }
  for (; j < nvec; j += NT) {  // the rest, one vector per lane per iteration
    const int i = j + lane;
    const bool ok = i < nvec;
    float x[P];
    float lm = -INFINITY;
    if (ok) {
      Tr::expand(src[i], x);
#pragma unroll
      for (int e = 0; e < P; ++e) lm = fmaxf(lm, x[e]);
      if (lm > m) {
        const float m2n = lm * kLog2e;
        s = (m == -INFINITY) ? 0.f : s * __builtin_amdgcn_exp2f(m2 - m2n);
        m = lm;
        m2 = m2n;
      }
      if (m != -INFINITY) {
#pragma unroll
        for (int e = 0; e < P; ++e) s += __builtin_amdgcn_exp2f(__builtin_fmaf(x[e], kLog2e, -m2));
      }
    } else {
#pragma unroll
      for (int e = 0; e < P; ++e) x[e] = -INFINITY;
    }
    if (__ballot(ok && lm >= tk.thr)) {
#pragma unroll
      for (int e = 0; e < P; ++e) tk.offer(x[e], i * P + e, ok);
    }
  }

  const float M = nvx::block_max<NT>(m, red);
  const float part = (m == -INFINITY) ? 0.f : s * __builtin_amdgcn_exp2f(m2 - M * kLog2e);
  const float S = nvx::block_sum_any<NT>(part, red);
  const float lnS = logf(S);

  if (lane < k) lists[wid * k + lane] = tk.key;
  __syncthreads();
  if (tid < NW * k) {
    const uint64_t c = lists[tid];
    if (c != 0) {
      int rank = 0;
      for (int u = 0; u < NW * k; ++u) rank += lists[u] > c ? 1 : 0;
      if (rank < k) {
        out_tok[(int64_t)row * k + rank] = (int32_t)~(uint32_t)c;
        out_lp[(int64_t)row * k + rank] = (from_ord((uint32_t)(c >> 32)) - M) - lnS;
      }
    }
  }
}

template <typename VT>
void launch(const void* logits, int64_t stride, int rows, int V, int k, int32_t* tok, float* lp,
            hipStream_t s) {
  const VT* x = reinterpret_cast<const VT*>(logits);
  // Few rows: wide workgroups keep enough loads in flight per CU; many rows:
  // narrow ones keep the per-wave lists short relative to the row.
  if (rows >= 1024)
    hipLaunchKernelGGL((topk_logprobs_kernel<VT, 256>), dim3(rows), dim3(256), 0, s, x, stride, V,
                       k, tok, lp);
  else
    hipLaunchKernelGGL((topk_logprobs_kernel<VT, 1024>), dim3(rows), dim3(1024), 0, s, x, stride,
                       V, k, tok, lp);
}

}  // namespace

extern "C" int nvx_topk_logprobs(const void* logits, int32_t logits_dtype, int64_t logits_row_stride,
                                 int32_t num_rows, int32_t vocab, int32_t k, int32_t* out_tokens,
                                 float* out_logprobs, void* stream) {
  nvx::clear_error();
  NVX_CHECK(logits_dtype == NVX_DTYPE_BF16 || logits_dtype == NVX_DTYPE_F32,
            "topk_logprobs: logits must be bf16 or fp32 (dtype code %d)", logits_dtype);
  NVX_CHECK(num_rows >= 0 && vocab >= 1, "topk_logprobs: bad sizes (rows %d, vocab %d)", num_rows,
            vocab);
  NVX_CHECK(k >= 1 && k <= kMaxK && k <= vocab, "topk_logprobs: k must be in [1, min(%d, vocab)] (got %d)",
            kMaxK, k);
  const int per = logits_dtype == NVX_DTYPE_BF16 ? 8 : 4;
  NVX_CHECK(vocab % per == 0 && logits_row_stride >= vocab && logits_row_stride % per == 0,
            "topk_logprobs: vocab (%d) and row stride (%lld) must be multiples of %d, stride >= vocab",
            vocab, (long long)logits_row_stride, per);
  if (num_rows == 0) return NVX_OK;
  NVX_CHECK(logits && out_tokens && out_logprobs, "topk_logprobs: null pointer");
  NVX_CHECK(((uintptr_t)logits & 15) == 0, "topk_logprobs: logits must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  nvx::TimerScope timer(NVX_TIMER_TOPK, s);
  if (logits_dtype == NVX_DTYPE_BF16)
    launch<uint16_t>(logits, logits_row_stride, num_rows, vocab, k, out_tokens, out_logprobs, s);
  else
    launch<float>(logits, logits_row_stride, num_rows, vocab, k, out_tokens, out_logprobs, s);
  NVX_LAUNCHED();
  return NVX_OK;
}
