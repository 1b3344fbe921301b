// KV-cache slot scatter (store_kvcache) and accepted-path compaction.
//
// Both are pure byte movement, bound by HBM.  A cache row (one slot, Hkv*D
// elements) is moved in 16-byte pieces: consecutive threads take consecutive
// pieces of a row so every wave issues fully coalesced 128-bit loads and stores.
#include "nvx_internal.h"

namespace {

constexpr int kNT = 256;
constexpr int kDepthGroup = 8;  // rows gathered into registers before scattering

using vec16 = uint4;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- scatter
__global__ __launch_bounds__(kNT) void store_kv_vec_kernel(
    const char* __restrict__ key, int64_t kstride, const char* __restrict__ value, int64_t vstride,
    char* __restrict__ k_cache, char* __restrict__ v_cache, const int32_t* __restrict__ slots,
    int num_tokens, int vecs_per_row) {
  const int64_t total = (int64_t)num_tokens * vecs_per_row;
  for (int64_t i = (int64_t)blockIdx.x * kNT + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * kNT) {
    const int tok = (int)(i / vecs_per_row);
    const int v = (int)(i - (int64_t)tok * vecs_per_row);
    const int64_t slot = slots[tok];
    if (slot < 0) continue;
    const int64_t row_bytes = (int64_t)vecs_per_row * 16;
    const vec16 kv = *reinterpret_cast<const vec16*>(key + tok * kstride + v * 16);
    const vec16 vv = *reinterpret_cast<const vec16*>(value + tok * vstride + v * 16);
    *reinterpret_cast<vec16*>(k_cache + slot * row_bytes + v * 16) = kv;
    *reinterpret_cast<vec16*>(v_cache + slot * row_bytes + v * 16) = vv;
  }
}

__global__ __launch_bounds__(kNT) void store_kv_byte_kernel(
    const char* __restrict__ key, int64_t kstride, const char* __restrict__ value, int64_t vstride,
    char* __restrict__ k_cache, char* __restrict__ v_cache, const int32_t* __restrict__ slots,
    int num_tokens, int row_bytes) {
  const int64_t total = (int64_t)num_tokens * row_bytes;
  for (int64_t i = (int64_t)blockIdx.x * kNT + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * kNT) {
    const int tok = (int)(i / row_bytes);
    const int c = (int)(i - (int64_t)tok * row_bytes);
    const int64_t slot = slots[tok];
    if (slot < 0) continue;
    k_cache[slot * row_bytes + c] = key[tok * kstride + c];
    v_cache[slot * row_bytes + c] = value[tok * vstride + c];
  }
}

// ------------------------------------------------------------- compaction
// One workgroup per (sequence, layer).  The accepted rows' source and destination
// slots depend only on the sequence, so the workgroup computes them once from
// wave-uniform (scalar) loads of the path and block table.  Each thread then owns a
// 16-byte column of the K or V row: it gathers up to kDepthGroup rows of its column
// into registers, then scatters them.  Groups run in ascending depth; destinations
// ctx+d are always below every later source ctx+path[d'] (path is strictly
// increasing), and columns are disjoint across threads, so no ordering between
// threads is needed.
// Returns -1 for a position outside the block table or an unassigned (-1) entry so a
// malformed path skips the row instead of touching memory outside the cache.
__device__ __forceinline__ int64_t slot_of(const int32_t* bt, int bt_len, int pos, int bs) {
  if (pos < 0 || pos / bs >= bt_len) return -1;
  const int32_t blk = bt[pos / bs];
  return blk < 0 ? -1 : (int64_t)blk * bs + (pos % bs);
}

__global__ __launch_bounds__(kNT) void kv_compact_kernel(
    char* __restrict__ k_cache, char* __restrict__ v_cache, int64_t layer_stride, int num_layers,
    int vecs_per_row, int block_size, const int32_t* __restrict__ block_tables, int bt_stride,
    const int32_t* __restrict__ ctx_lens, const int32_t* __restrict__ path, int path_stride,
    const int32_t* __restrict__ accepted_len) {
  const int b = blockIdx.x / num_layers;
  const int layer = blockIdx.x - b * num_layers;
  const int a = min(accepted_len[b], path_stride - 1);
  if (a <= 0) return;  // uniform over the workgroup
  const int32_t* bt = block_tables + (int64_t)b * bt_stride;
  const int32_t* pth = path + (int64_t)b * path_stride;
  const int ctx = ctx_lens[b];
  const int64_t row_bytes = (int64_t)vecs_per_row * 16;
  char* const kl = k_cache + layer * layer_stride;
  char* const vl = v_cache + layer * layer_stride;
  for (int d0 = 1; d0 <= a; d0 += kDepthGroup) {
    int64_t src[kDepthGroup], dst[kDepthGroup];
#pragma unroll
    for (int j = 0; j < kDepthGroup; ++j) {
      const int d = d0 + j;
      src[j] = d <= a ? slot_of(bt, bt_stride, ctx + pth[d], block_size) : -1;
      dst[j] = d <= a ? slot_of(bt, bt_stride, ctx + d, block_size) : -1;
    }
    for (int col = threadIdx.x; col < 2 * vecs_per_row; col += kNT) {
      char* const base = (col < vecs_per_row ? kl : vl) + (col % vecs_per_row) * 16;
      // Unconditional loads (a row with no valid source reads slot 0 and is not
      // stored) keep the gathered rows in registers with all loads in flight.  The
      // rows are a native 4 x u32 vector type: an array of HIP's uint4 struct here
      // was kept in scratch memory.
      u32x4 rows[kDepthGroup];
#pragma unroll
      for (int j = 0; j < kDepthGroup; ++j)
        rows[j] = __builtin_nontemporal_load(  // each accepted row is read once
            reinterpret_cast<const u32x4*>(base + max(src[j], (int64_t)0) * row_bytes));
#pragma unroll
      for (int j = 0; j < kDepthGroup; ++j)
        if (src[j] >= 0 && dst[j] >= 0) *reinterpret_cast<u32x4*>(base + dst[j] * row_bytes) = rows[j];
    }
  }
}

int grid_for(int64_t work) {
  int64_t g = (work + kNT - 1) / kNT;
  if (g > 65536) g = 65536;
  if (g < 1) g = 1;
  return (int)g;
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

extern "C" int nvx_store_kvcache(const void* key, int64_t key_stride_bytes, const void* value,
                                 int64_t value_stride_bytes, void* k_cache, void* v_cache,
                                 const int32_t* slot_mapping, int32_t num_tokens, int32_t row_bytes,
                                 void* stream) {
  nvx::clear_error();
  NVX_CHECK(num_tokens >= 0 && row_bytes > 0, "store_kvcache: bad sizes (N=%d, row_bytes=%d)",
            num_tokens, row_bytes);
  if (num_tokens == 0) return NVX_OK;
  NVX_CHECK(key && value && k_cache && v_cache && slot_mapping, "store_kvcache: null pointer");
  hipStream_t s = (hipStream_t)stream;
  nvx::TimerScope timer(NVX_TIMER_STORE_KV, s);
  const bool vec = row_bytes % 16 == 0 && key_stride_bytes % 16 == 0 &&
                   value_stride_bytes % 16 == 0 && aligned16(key) && aligned16(value) &&
                   aligned16(k_cache) && aligned16(v_cache);
  if (vec) {
    const int vpr = row_bytes / 16;
    hipLaunchKernelGGL(store_kv_vec_kernel, dim3(grid_for((int64_t)num_tokens * vpr)), dim3(kNT), 0,
                       s, (const char*)key, key_stride_bytes, (const char*)value,
                       value_stride_bytes, (char*)k_cache, (char*)v_cache, slot_mapping, num_tokens,
                       vpr);
  } else {
    hipLaunchKernelGGL(store_kv_byte_kernel, dim3(grid_for((int64_t)num_tokens * row_bytes)),
                       dim3(kNT), 0, s, (const char*)key, key_stride_bytes, (const char*)value,
                       value_stride_bytes, (char*)k_cache, (char*)v_cache, slot_mapping, num_tokens,
                       row_bytes);
  }
  NVX_LAUNCHED();
  return NVX_OK;
}

extern "C" int nvx_kv_compact(void* k_cache, void* v_cache, int64_t layer_stride_bytes,
                              int32_t num_layers, int32_t row_bytes, int32_t block_size,
                              const int32_t* block_tables, int32_t block_table_stride,
                              const int32_t* ctx_lens, const int32_t* path, int32_t path_stride,
                              const int32_t* accepted_len, int32_t num_seqs, void* stream) {
  nvx::clear_error();
  NVX_CHECK(num_seqs >= 0 && num_layers >= 1, "kv_compact: bad sizes (seqs=%d, layers=%d)",
            num_seqs, num_layers);
  NVX_CHECK(row_bytes > 0 && row_bytes % 16 == 0, "kv_compact: row_bytes must be a positive "
            "multiple of 16 (got %d)", row_bytes);
  NVX_CHECK(layer_stride_bytes % 16 == 0 && aligned16(k_cache) && aligned16(v_cache),
            "kv_compact: caches and layer stride must be 16-byte aligned");
  NVX_CHECK(block_size > 0 && path_stride >= 1 && block_table_stride >= 1,
            "kv_compact: bad block_size/path_stride/block_table_stride");
  if (num_seqs == 0) return NVX_OK;
  NVX_CHECK(k_cache && v_cache && block_tables && ctx_lens && path && accepted_len,
            "kv_compact: null pointer");
  hipStream_t s = (hipStream_t)stream;
  nvx::TimerScope timer(NVX_TIMER_KV_COMPACT, s);
  const int vpr = row_bytes / 16;
  const int64_t blocks = (int64_t)num_seqs * num_layers;
  NVX_CHECK(blocks < (1ll << 31), "kv_compact: too many (sequence, layer) pairs");
  hipLaunchKernelGGL(kv_compact_kernel, dim3((unsigned)blocks), dim3(kNT), 0, s, (char*)k_cache,
                     (char*)v_cache, layer_stride_bytes, num_layers, vpr, block_size, block_tables,
                     block_table_stride, ctx_lens, path, path_stride, accepted_len);
  NVX_LAUNCHED();
  return NVX_OK;
}
