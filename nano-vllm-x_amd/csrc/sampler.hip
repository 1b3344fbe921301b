// Sampler kernels: temperature softmax and tree / chain rejection sampling.
//
// temperature_softmax: one workgroup (1024 threads) per row.  For bf16 rows of up
//   to 1024*8*kRegChunks elements the row is loaded once into registers with
//   128-bit loads (row max, sum of exp, then the fp32 write come from registers);
//   other rows stream twice (online max/sum, then write).  HBM bound: it reads the
//   logits once and writes fp32 probabilities once.
//
// rejection_sample_tree: one workgroup (1024 threads) per sequence walks the draft
//   tree from the root.  Per visited node the acceptance tests need two scalars;
//   each rejection needs one pass over the node's target/draft rows to normalise
//   the residual, and the final draw one inverse-CDF pass.  Only rows on the walk
//   are read.  The fp32 association order of every sum and scan is fixed (see
//   nvx_internal.h) so integer outputs are reproducible bit for bit by the CPU
//   restatement given the same probabilities and uniforms.
#include <float.h>

#include "nvx_internal.h"

#pragma clang fp contract(off)

namespace {

constexpr int kNT = 1024;
constexpr int kNW = kNT / nvx::kWave;
constexpr int kRegChunks = 19;  // 16-byte chunks per thread: V <= 155648 bf16
constexpr int kMaxNodes = 64;

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ float load_logit(const void* row, int i, int dtype) {
  if (dtype == NVX_DTYPE_F32) return reinterpret_cast<const float*>(row)[i];
  const uint16_t h = reinterpret_cast<const uint16_t*>(row)[i];
  return __uint_as_float((uint32_t)h << 16);
}

// ------------------------------------------------------------ softmax (regs)
__global__ __launch_bounds__(kNT) void softmax_bf16_regs_kernel(const uint16_t* __restrict__ logits,
                                                                int64_t stride,
                                                                const float* __restrict__ temps,
                                                                float* __restrict__ probs, int V) {
  __shared__ float red[kNW];
  const int row = blockIdx.x;
  const float T = temps[row];
  const bool greedy = (T == 0.f);
  const uint4* src = reinterpret_cast<const uint4*>(logits + (int64_t)row * stride);
  float4* dst = reinterpret_cast<float4*>(probs + (int64_t)row * V);
  const int nvec = V / 8;

  uint4 buf[kRegChunks];
#pragma unroll
  for (int c = 0; c < kRegChunks; ++c) {
    const int idx = threadIdx.x + c * kNT;
    buf[c] = (idx < nvec) ? src[idx] : make_uint4(0xff80ff80u, 0xff80ff80u, 0xff80ff80u, 0xff80ff80u);
  }
  if (greedy) {
#pragma unroll
    for (int c = 0; c < kRegChunks; ++c) {
      const int idx = threadIdx.x + c * kNT;
      if (idx < nvec) {
        const uint4 w = buf[c];
        dst[2 * idx] = make_float4(bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y));
        dst[2 * idx + 1] = make_float4(bf16_lo(w.z), bf16_hi(w.z), bf16_lo(w.w), bf16_hi(w.w));
      }
    }
    return;
  }
  // max(x / T) == max(x) / T for T > 0 (correctly rounded division is monotone);
  // padding holds -inf.
  float mx = -INFINITY;
#pragma unroll
  for (int c = 0; c < kRegChunks; ++c) {
    const uint4 w = buf[c];
    mx = fmaxf(mx, fmaxf(fmaxf(bf16_lo(w.x), bf16_hi(w.x)), fmaxf(bf16_lo(w.y), bf16_hi(w.y))));
    mx = fmaxf(mx, fmaxf(fmaxf(bf16_lo(w.z), bf16_hi(w.z)), fmaxf(bf16_lo(w.w), bf16_hi(w.w))));
  }
  const float m = nvx::block_max<kNT>(mx, red) / T;
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < kRegChunks; ++c) {
    const int idx = threadIdx.x + c * kNT;
    if (idx < nvec) {
      const uint4 w = buf[c];
      s += __expf(bf16_lo(w.x) / T - m) + __expf(bf16_hi(w.x) / T - m);
      s += __expf(bf16_lo(w.y) / T - m) + __expf(bf16_hi(w.y) / T - m);
      s += __expf(bf16_lo(w.z) / T - m) + __expf(bf16_hi(w.z) / T - m);
      s += __expf(bf16_lo(w.w) / T - m) + __expf(bf16_hi(w.w) / T - m);
    }
  }
  const float inv = 1.f / nvx::block_sum_any<kNT>(s, red);
#pragma unroll
  for (int c = 0; c < kRegChunks; ++c) {
    const int idx = threadIdx.x + c * kNT;
    if (idx < nvec) {
      const uint4 w = buf[c];
      dst[2 * idx] = make_float4(__expf(bf16_lo(w.x) / T - m) * inv, __expf(bf16_hi(w.x) / T - m) * inv,
                                 __expf(bf16_lo(w.y) / T - m) * inv, __expf(bf16_hi(w.y) / T - m) * inv);
      dst[2 * idx + 1] =
          make_float4(__expf(bf16_lo(w.z) / T - m) * inv, __expf(bf16_hi(w.z) / T - m) * inv,
                      __expf(bf16_lo(w.w) / T - m) * inv, __expf(bf16_hi(w.w) / T - m) * inv);
    }
  }
}

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
  float m = -INFINITY, s = 0.f;
  for (int i = threadIdx.x; i < V; i += kNT) {
    const float x = load_logit(src, i, dtype) / T;
    if (x == -INFINITY) continue;
    if (x > m) {
      s = s * __expf(m - x) + 1.f;
      m = x;
    } else {
      s += __expf(x - m);
    }
  }
  const float M = nvx::block_max<kNT>(m, red);
  const float part = (m == -INFINITY) ? 0.f : s * __expf(m - M);
  const float inv = 1.f / nvx::block_sum_any<kNT>(part, red);
  for (int i = threadIdx.x; i < V; i += kNT) dst[i] = __expf(load_logit(src, i, dtype) / T - M) * inv;
}

// ------------------------------------------------------- rejection sampling
struct Chain {
  const float* S;  // normalisers of the residual steps (LDS)
  const int* X;    // rejected token of each step (LDS, delta mode)
  int k;
  bool delta;
};

// cur_k[y] from p[y], q[y] following the residual steps.
__device__ __forceinline__ float chain_eval(const Chain& ch, float py, float qy, int y) {
  float v = py;
  for (int j = 0; j < ch.k; ++j) {
    const float S = ch.S[j];
    if (!(S > 0.f)) {
      v = py;
      continue;
    }
    if (ch.delta)
      v = ((y == ch.X[j]) ? 0.f : v) / S;
    else
      v = fmaxf(v - qy, 0.f) / S;
  }
  return v;
}

__device__ __forceinline__ void load4(const float* row, int g, int V, bool vec, float out[4]) {
  const int i0 = 4 * g;
  if (vec && i0 + 3 < V) {
    const float4 t = reinterpret_cast<const float4*>(row)[g];
    out[0] = t.x; out[1] = t.y; out[2] = t.z; out[3] = t.w;
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) out[c] = (i0 + c < V) ? row[i0 + c] : 0.f;
  }
}

// Canonical sum over y of the residual of the current distribution after also
// rejecting token x: stochastic max(cur - q, 0); delta cur with x zeroed.
__device__ float residual_sum(const float* prow, const float* qrow, int V, bool vec, const Chain& ch,
                              int x, float* red) {
  const int G = (V + 3) / 4;
  float acc = 0.f;
  for (int g = threadIdx.x; g < G; g += kNT) {
    float p[4], q[4] = {0.f, 0.f, 0.f, 0.f};
    load4(prow, g, V, vec, p);
    if (!ch.delta) load4(qrow, g, V, vec, q);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int y = 4 * g + c;
      if (y < V) {
        const float v = chain_eval(ch, p[c], q[c], y);
        const float r = ch.delta ? ((y == x) ? 0.f : v) : fmaxf(v - q[c], 0.f);
        acc = acc + r;
      }
    }
  }
  return nvx::block_sum_canonical<kNT>(acc, red);
}

// Inverse-CDF pick from the current distribution with uniform u (contract in
// oracle/sampler.py: cdf_pick).
__device__ int cdf_pick(const float* prow, const float* qrow, int V, bool vec, const Chain& ch, float u,
                        float* red, int* redi, float* incl_lds) {
  const int C = 4 * (((V + 3) / 4 + kNT - 1) / kNT);
  const int lo = threadIdx.x * C;
  const int hi = min(lo + C, V);
  float s = 0.f;
  for (int i = lo; i < hi; i += 4) {
    float p[4], q[4] = {0.f, 0.f, 0.f, 0.f};
    load4(prow, i / 4, V, vec, p);
    if (!ch.delta) load4(qrow, i / 4, V, vec, q);
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (i + c < hi) s = s + chain_eval(ch, p[c], q[c], i + c);
  }
  float total;
  const float incl = nvx::block_incl_scan_canonical<kNT>(s, red, &total);
  incl_lds[threadIdx.x] = incl;
  __syncthreads();
  const float tau = u * total;
  float run = threadIdx.x > 0 ? incl_lds[threadIdx.x - 1] : 0.f;
  int first = INT32_MAX, last = -1;
  for (int i = lo; i < hi; i += 4) {
    float p[4], q[4] = {0.f, 0.f, 0.f, 0.f};
    load4(prow, i / 4, V, vec, p);
    if (!ch.delta) load4(qrow, i / 4, V, vec, q);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (i + c < hi) {
        const float v = chain_eval(ch, p[c], q[c], i + c);
        run = run + v;
        if (v > 0.f) {
          last = i + c;
          if (first == INT32_MAX && run > tau) first = i + c;
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
__device__ int block_argmax(const float* row, int V, bool vec, float* red, int* redi) {
  float bv = -INFINITY;
  int bi = INT32_MAX;
  const int G = (V + 3) / 4;
  for (int g = threadIdx.x; g < G; g += kNT) {
    float p[4];
    load4(row, g, V, vec, p);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int y = 4 * g + c;
      if (y < V && (p[c] > bv || (p[c] == bv && y < bi))) {
        bv = p[c];
        bi = y;
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

__global__ __launch_bounds__(kNT) void rejection_tree_kernel(
    const float* __restrict__ P, int64_t p_seq_stride, const float* __restrict__ Q,
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
  __shared__ float s_S[kMaxNodes];
  __shared__ int s_X[kMaxNodes];
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
    const float* prow = P + (int64_t)b * p_seq_stride + (int64_t)cur * V;
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
      Chain ch{s_S, s_X, 0, delta != 0};
      for (int j = cur + 1; j < T; ++j) {
        if (s_par[j] != cur) continue;
        const int x = s_tok[j];
        float cx = 0.f, qx = 1.f;
        if (x >= 0 && x < V) {
          const float qv = ch.delta ? 0.f : qrow[x];
          cx = chain_eval(ch, prow[x], qv, x);
          if (!ch.delta) qx = qv;
        }
        if (s_u[j] * qx <= cx && cx > 0.f) {
          accepted = j;
          break;
        }
        const float S = residual_sum(prow, qrow, V, vec, ch, x, red);
        if (threadIdx.x == 0) {
          s_S[ch.k] = S;
          s_X[ch.k] = x;
        }
        __syncthreads();
        ch.k += 1;
      }
      if (accepted < 0) {
        next = cdf_pick(prow, qrow, V, vec, ch, uf, red, redi, s_incl);
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
  const bool regs = logits_dtype == NVX_DTYPE_BF16 && vocab % 8 == 0 &&
                    logits_row_stride % 8 == 0 && vocab <= kNT * 8 * kRegChunks &&
                    aligned16(logits) && aligned16(probs);
  if (regs) {
    hipLaunchKernelGGL(softmax_bf16_regs_kernel, dim3(num_rows), dim3(kNT), 0, s,
                       (const uint16_t*)logits, logits_row_stride, temperatures, probs, vocab);
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
  hipLaunchKernelGGL(rejection_tree_kernel, dim3(num_seqs), dim3(kNT), 0, s, target_probs,
                     p_seq_stride, draft_mode == 1 ? nullptr : draft_probs, q_seq_stride, vocab,
                     tokens, parents, num_nodes, node_stride, uniforms, final_uniforms, greedy,
                     draft_mode, path, accepted_len, out_tokens, next_token, vec);
  NVX_LAUNCHED();
  return NVX_OK;
}
