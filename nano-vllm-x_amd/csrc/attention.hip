// Paged tree attention for gfx950 (bf16 in, fp32 accumulate, bf16 out).
//
// Work item = (sequence b, KV head hk, q-row chunk, KV split).  The q rows of a
// work item are the G = Hq/Hkv query heads of hk times the sequence's q_len tree
// nodes (row r -> node r / G, head hk*G + r % G), so one staged K/V chunk serves
// the whole GQA group.  Each wave owns 32 q rows.
//
// K and V arrive in LDS by LDS-DMA (global_load_lds_dwordx4) in 64-key chunks.
// Q is scaled by scale*log2(e) when it is loaded (rounded to bf16), and the S chain
// starts from an accumulator holding -m (the row's reference max), so every wave
// computes S^T = K . Q^T - m with v_mfma_f32_32x32x16_bf16 and each probability is
// a single exp2.  Lane l then holds query row l%32 and 16 keys per 32-key tile, so
// the online-softmax row max and row sum are in-lane plus one exchange with lane
// l^32 (the row max only when the reference max is redone; the row sums once, at
// the end).  P^T goes straight from those registers into the B operand of
// O^T += V^T . P^T; the contraction slots are relabelled to the keys the lane
// already holds, and the V^T A operand comes from two ds_read_b64_tr_b16 (gfx950
// LDS transpose reads) per MFMA.
//
// Pipeline: a 2-stage LDS ring (64 KB), one chunk in flight while the other is
// computed, one barrier per chunk.  Waves use < 256 registers, so a CU runs two per
// SIMD: a tree-sized work item of more than 128 rows is one 8-wave workgroup (its K/V
// enters the CU once); smaller items and the q-row chunks of causal prefill are
// 4-wave workgroups, two per CU.  The two waves on
// a SIMD interleave their MFMA and VALU phases.
//
// Masking: keys < context_len - q_len are visible to all rows; key base+m is
// visible to node i iff bit m of its tree mask (or m <= i without a mask).
// With more than one split, partial (o, log2-sum-exp) go to the workspace and a
// second kernel merges them.
#include <mutex>
#include <type_traits>

#include "nvx_internal.h"

namespace {

constexpr int kD = 128;
constexpr int kKC = 64;                         // keys per staged chunk
constexpr int kStages = 2;                      // LDS ring: chunk c computed, c+1 in flight
constexpr int kTileBytes = kKC * kD * 2;        // one K (or V) chunk: 64 rows x 256 B
constexpr int kStageBytes = 2 * kTileBytes;     // K then V
constexpr int kDmaPerChunk = kStageBytes / 1024;  // 1 KB per wave-wide 16-byte-per-lane load
constexpr int kTargetWaves = 256 * 8;           // split-KV target: one round of 8 waves per CU
constexpr int kMaxSplitPages = 512;             // block-table entries one KV split may touch

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

struct AttnParams {
  const uint16_t* q;
  uint16_t* o;
  const uint16_t* k_cache;
  const uint16_t* v_cache;
  const int32_t* block_tables;
  const int32_t* cu_q;
  const int32_t* ctx_lens;
  const uint64_t* tree_mask;
  float* part_o;
  float* part_lse;
  int bt_stride, num_seqs, total_q, Hq, Hkv, G, block_size, nq, nsplit;
  float scale_log2;
};

__device__ __forceinline__ uint16_t f2bf(float x) {
  uint32_t u = __float_as_uint(x);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// LDS rows are 256 B with no padding; the 16-byte slot of logical segment `seg` in
// row `row` is seg ^ swz(row).  swz is a bijection on row % 16 (K reads of 16
// consecutive rows hit 16 different slots) and varies in bits 2-3 over any 4
// consecutive rows (the 4 rows x 4 segments of a transpose read cover 16 slots),
// so both read patterns are bank-conflict free.
__device__ __forceinline__ int swz(int row) { return ((row & 3) << 2) | ((row >> 2) & 3); }

// Cache policy of the K/V loads.  kShared: the K/V of a (sequence, KV head) is read
// by several workgroups (one per q-row chunk), which meet in L2; the loads skip the
// vector L1 (sc1), where nothing is reused.  kStream: every K/V byte is read once
// (one q-row chunk), so the loads are non-temporal (nt) and do not displace what
// other work keeps in the caches.
enum DmaPolicy { kShared = 0, kStream = 1 };

// Wave-wide 16-byte-per-lane load from global memory straight into LDS: lane i's
// data lands at LDS byte address lds_base + 16*i.  Issued from inline asm so the
// compiler does not fence every LDS read behind it; completion is waited for
// explicitly with wait_vm below (each call counts one vector-memory op per wave).
template <int kPolicy>
__device__ __forceinline__ void dma16(const void* sbase, uint32_t voff, uint32_t lds_base) {
  if constexpr (kPolicy == kStream)
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1 nt"
                 :
                 : "v"(voff), "s"(sbase), "s"(lds_base)
                 : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1 sc1"
                 :
                 : "v"(voff), "s"(sbase), "s"(lds_base)
                 : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// Bits [0, n) set, n clamped to [0, 64].
__device__ __forceinline__ uint64_t low_bits64(int n) {
  return n <= 0 ? 0ull : (n >= 64 ? ~0ull : (1ull << n) - 1ull);
}

__device__ __forceinline__ int remap_xcd(int phys, int n) {
  // Blocks are dispatched round-robin over the 8 XCDs; give each XCD a
  // contiguous range of logical ids so the blocks of one (seq, kv head), which
  // read the same K/V, share an L2.
  const int x = phys & 7, slot = phys >> 3;
  const int q = n >> 3, r = n & 7;
  const int start = x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q;
  return start + slot;
}

// Two waves per SIMD (at most 256 VGPR+AGPR each): two 4-wave workgroups per CU.
template <int W, int kPolicy>
__global__ __launch_bounds__(W * 64) __attribute__((amdgpu_waves_per_eu(2)))
void tree_attn_kernel(AttnParams p) {
  constexpr int PER = kDmaPerChunk / W;  // LDS-DMA loads per wave per chunk
  __shared__ __attribute__((aligned(1024))) uint8_t ring[kStages * kStageBytes];
  __shared__ int32_t pages[kMaxSplitPages];

  // Causal launches with several q-row chunks per item (prefill): a later chunk sees
  // more keys, so the heaviest chunks go first, in blockIdx (dispatch) order over all
  // XCDs -- 4 sequences of 2048 prompt tokens at 32/8 heads: 186 us against 225 us with
  // the chunks of an item adjacent.  Otherwise (tree masks: the chunks of an item do
  // equal work) the chunks and splits of an item are adjacent and grouped by XCD, so
  // they meet in one L2 (64-node trees at 64/8 heads: 309 us against 323 us).
  const bool heavy_first = p.nq > 1 && p.tree_mask == nullptr;
  const int logical = heavy_first ? (int)blockIdx.x : remap_xcd(blockIdx.x, gridDim.x);
  const int split = logical % p.nsplit;
  int t = logical / p.nsplit;
  int qc;
  if (heavy_first) {
    const int items = (int)(gridDim.x / ((unsigned)p.nsplit * p.nq));  // (sequence, KV head)
    qc = p.nq - 1 - t / items;
    t %= items;
  } else {
    qc = t % p.nq;
    t /= p.nq;
  }
  const int hk = t % p.Hkv;
  const int b = t / p.Hkv;

  const int q0 = p.cu_q[b];
  const int qlen = p.cu_q[b + 1] - q0;
  const int ctxlen = p.ctx_lens[b];
  const int base = ctxlen - qlen;
  const int rows_total = p.G * qlen;
  const int row0 = qc * W * 32;
  if (row0 >= rows_total || qlen <= 0) return;  // uniform over the block

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, g = lane >> 5, lr = lane & 31;
  const int r = row0 + wave * 32 + lr;  // this lane's q row
  const bool row_ok = r < rows_total;
  const bool wave_active = row0 + wave * 32 < rows_total;
  const int node = row_ok ? r / p.G : 0;
  const int head = hk * p.G + (row_ok ? r % p.G : 0);
  const int token = q0 + node;

  // Q^T fragments (B operand of S^T = K.Q^T): d = 16*s + 8*g + [0..7].
  bf16x8 bq[8];
  {
    const bool ld = row_ok && token < p.total_q;
    const uint16_t* qrow = p.q + ((int64_t)token * p.Hq + head) * kD + 8 * g;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      uint4 v = make_uint4(0, 0, 0, 0);
      if (ld) v = *reinterpret_cast<const uint4*>(qrow + 16 * s);
      bf16x8 x = __builtin_bit_cast(bf16x8, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = (__bf16)((float)x[e] * p.scale_log2);
      bq[s] = x;
    }
  }
  const bool use_tree = p.tree_mask != nullptr;
  // First key that some row of this wave cannot see: the tree start with a tree mask;
  // causal, one past the key of the wave's first node (every row of the wave sees the
  // keys before it).  Chunks wholly before it need no mask -- in causal prefill
  // (base 0) only the chunks on the diagonal of the wave's rows do.
  const int mask_from = use_tree ? base : base + (row0 + wave * 32) / p.G + 1;
  const uint64_t mbits = (use_tree && row_ok && token < p.total_q) ? p.tree_mask[token] : 0ull;

  // Keys beyond the last node of this chunk's rows are masked for every row.
  const int last_node = min(qlen - 1, (row0 + W * 32 - 1) / p.G);
  const int key_end = max(0, min(ctxlen, base + last_node + 1));
  const int nchunks = (key_end + kKC - 1) / kKC;
  const int cps = (nchunks + p.nsplit - 1) / p.nsplit;
  const int c0 = split * cps;
  // A context longer than the max_context_len the launch was sized for would overrun
  // the LDS page table: such keys are dropped rather than written out of bounds.
  const int c1 = min(min(nchunks, c0 + cps), c0 + ((kMaxSplitPages - 1) * p.block_size) / kKC);

  const int32_t* bt = p.block_tables + (int64_t)b * p.bt_stride;
  const int bs = p.block_size;
  const uint32_t ring_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)ring;

  // This split's block-table entries go to LDS once, so the loop reads page ids
  // without touching the vector-memory counter the DMA pipeline waits on.
  const int page0 = (c0 * kKC) / bs;
  const int npages = c1 > c0 ? ((c1 * kKC - 1) / bs - page0 + 1) : 0;
  for (int i = tid; i < npages; i += W * 64)
    pages[i] = (page0 + i < p.bt_stride) ? bt[page0 + i] : -1;
  // Make every prologue global load (Q, mask, pages) complete here, before the
  // first LDS-DMA is queued behind them.
#pragma unroll
  for (int s = 0; s < 8; ++s) asm volatile("" : : "v"(bq[s]));
  asm volatile("" : : "v"(mbits));
  __syncthreads();

  // The PER LDS-DMA loads of this wave for one chunk: load j of wave w fills 4 rows
  // (1 KB) of the K (first 16 loads) or V (last 16) tile; lane i fetches row
  // 4*(ii%16) + i/16, logical segment (i%16)^swz(row), so the tile lands swizzled.
  // The per-lane byte offset within a chunk is loop invariant (lane_full, for chunks
  // wholly before context_len); the chunk's page start is a scalar base.  In the
  // chunk that ends past context_len the missing rows re-read the chunk's first row
  // (finite data; their scores are masked to -inf).
  const int row_stride = p.Hkv * kD * 2;  // bytes between consecutive tokens
  uint32_t lane_off[PER], lane_full[PER];
  int lane_row[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int ii = wave + W * j;
    const int row = 4 * (ii & 15) + (lane >> 4);
    const int seg = (lane & 15) ^ swz(row);
    lane_row[j] = row;
    lane_off[j] = (uint32_t)(hk * kD * 2 + seg * 16);
    lane_full[j] = lane_off[j] + (uint32_t)(row * row_stride);
  }
  // The chunk to issue next, as (page index in the LDS table, key offset in the page),
  // advanced by one chunk per issue (no division in the loop).
  int is_page = 0, is_off = (c0 * kKC) % bs;
  auto issue_chunk = [&](int c, auto stage) {
    constexpr int ST = decltype(stage)::value;
    const int pos0 = c * kKC;
    const int32_t blk = __builtin_amdgcn_readfirstlane(pages[is_page]);
    const int64_t tok0 = blk >= 0 ? (int64_t)blk * bs + is_off : 0;
    is_off += kKC;
    if (is_off == bs) {
      is_off = 0;
      ++is_page;
    }
    const char* kbase = reinterpret_cast<const char*>(p.k_cache) + tok0 * row_stride;
    const char* vbase = reinterpret_cast<const char*>(p.v_cache) + tok0 * row_stride;
    const uint32_t lds0 = ring_base + ST * kStageBytes;
    if (pos0 + kKC <= ctxlen) {
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        const int ii = wave + W * j;
        dma16<kPolicy>(ii >> 4 ? vbase : kbase, lane_full[j],
                       lds0 + (ii >> 4) * kTileBytes + (ii & 15) * 1024);
      }
    } else {
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        const int ii = wave + W * j;
        const int row = pos0 + lane_row[j] < ctxlen ? lane_row[j] : 0;
        dma16<kPolicy>(ii >> 4 ? vbase : kbase, lane_off[j] + (uint32_t)(row * row_stride),
                       lds0 + (ii >> 4) * kTileBytes + (ii & 15) * 1024);
      }
    }
  };

  // m_run: the row's reference max (scaled log2 units).  The S chain starts from
  // cinit = -m_ref (m_ref = m_run, or 0 before the row's first visible key), so the
  // MFMAs deliver c*s - m_ref and each probability is one exp2.  Each of the two S
  // tiles starts from its own copy, so no accumulator is copied per chunk.
  float m_run = -INFINITY, l_run = 0.f;
  f32x16 cinit[2];
#pragma unroll
  for (int j = 0; j < 16; ++j) cinit[0][j] = cinit[1][j] = 0.f;
  f32x16 oacc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int j = 0; j < 16; ++j) oacc[dt][j] = 0.f;

  // LDS byte addresses.  With the swizzle, every read address is a per-lane value
  // (loop invariant, held in registers) plus a constant: the ring stage is a template
  // constant of each unrolled step, so stage and row offsets become immediates.
  //  K fragment (tile kt, d-slice s): row kt*32 + lr, slot (2s + g) ^ swz(lr)
  //    = (k_lane ^ (s << 5)) + stage + kt * 8192
  //  V^T transpose read (group ks, d tile dt, half h): 16-lane group q = lane/16
  //  supplies rows (keys) 16*ks + 8*h + 4*(q/2) + i/4 and d columns
  //  dt*32 + 16*(q%2) + 4*(i%4), i.e.
  //    = (v_lane[h] ^ (dt << 6)) + stage + kTileBytes + ks * 4096
  // (swz depends on row % 16 only, so the row terms 32*kt and 16*ks are plain
  // offsets, and the XORed bits never carry into the row or stage bits.)  The empty
  // asm statements keep the compiler from recomputing the XORs in the loop.
  const uint32_t k_lane = (uint32_t)(lr * 256 + ((g ^ swz(lr)) << 4));
  const int tq = lane >> 4, ti = lane & 15;
  const int tr_key = 4 * (tq >> 1) + (ti >> 2);
  const int tr_d = 16 * (tq & 1) + 4 * (ti & 3);
  const uint32_t v_lane0 = (uint32_t)(tr_key * 256 + ((((tr_d >> 3) ^ swz(tr_key))) << 4) + (tr_d & 7) * 2);
  const uint32_t v_lane1 =
      (uint32_t)((tr_key + 8) * 256 + ((((tr_d >> 3) ^ swz(tr_key + 8))) << 4) + (tr_d & 7) * 2);
  uint32_t k_addr[8], v_addr[2][4];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    k_addr[s] = k_lane ^ (uint32_t)(s << 5);
    asm volatile("" : "+v"(k_addr[s]));
  }
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    v_addr[0][dt] = v_lane0 ^ (uint32_t)(dt << 6);
    v_addr[1][dt] = v_lane1 ^ (uint32_t)(dt << 6);
    asm volatile("" : "+v"(v_addr[0][dt]), "+v"(v_addr[1][dt]));
  }

  // S^T tiles of the chunk in stage ST: sacc[kt] element j holds key
  // kt*32 + (j/4)*8 + 4*g + j%4 of query row lr.  s_pair(s) adds the products over
  // d = 16*s .. 16*s+15.
  auto s_pair = [&](auto stage, int s, f32x16 (&sacc)[2]) {
    constexpr int ST = decltype(stage)::value;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const bf16x8 k = *reinterpret_cast<const bf16x8*>(ring + k_addr[s] + ST * kStageBytes + kt * 8192);
      sacc[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k, bq[s], s == 0 ? cinit[kt] : sacc[kt], 0, 0, 0);
    }
  };
  // O^T += V^T . P^T for key group ks (keys 16*ks .. 16*ks+15).
  auto pv_group = [&](auto stage, int ks, bf16x8 bp) {
    constexpr int ST = decltype(stage)::value;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
          (lds_bf16x4*)(ring + v_addr[0][dt] + ST * kStageBytes + kTileBytes + ks * 4096));
      const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
          (lds_bf16x4*)(ring + v_addr[1][dt] + ST * kStageBytes + kTileBytes + ks * 4096));
      const bf16x8 a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bp, oacc[dt], 0, 0, 0);
    }
  };

  // One step on chunk c (in stage ST): the S MFMAs into sacc, the softmax (VALU),
  // then the P.V MFMAs.
  auto step = [&](int c, auto stage, f32x16 (&sacc)[2]) {
    if (!wave_active) return;

    auto phase_s = [&]() {
#pragma unroll
      for (int s = 0; s < 8; ++s) s_pair(stage, s, sacc);
      // LDS reads run a d-slice ahead of the MFMAs that consume them.
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
      for (int i = 0; i < 6; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    };
    // Probabilities of chunk c against the running reference max m_run, packed to
    // bf16 for the P.V MFMAs; returns this lane's fp32 sum of the probabilities.
    // The sum uses plain fp32 adds in two chains (even and odd elements), each
    // starting from its first term: v_dot2 (the bf16 dot product) executes in the
    // matrix pipe and serialises with the other wave's MFMAs on the SIMD.
    bf16x8 bp[4];
    auto probs = [&]() {
      float e[32];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        // P^T as B operand: slot (g, i) of group ks holds key 16*ks + (i/4)*8 +
        // 4*g + i%4, i.e. element (ks&1)*8 + i of sacc[ks/2].
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          e[ks * 8 + i] = __builtin_amdgcn_exp2f(sacc[ks >> 1][(ks & 1) * 8 + i]);
          bp[ks][i] = (__bf16)e[ks * 8 + i];
        }
      }
      float l0 = e[0], l1 = e[1];
#pragma unroll
      for (int k = 2; k < 32; k += 2) {
        l0 += e[k];
        l1 += e[k + 1];
      }
      return l0 + l1;
    };
    auto phase_softmax = [&]() {
      const int pos0 = c * kKC;
      if (pos0 + kKC > mask_from) {  // keys some row of the wave cannot see
        // Visibility of the chunk's 64 keys for this row as one 64-bit word, cut at
        // context_len.  Tree: keys before the tree, then the row's mask bits (a tree
        // has at most 64 nodes).  Causal: keys up to base + node.  Element j of tile
        // kt is key kt*32 + (j/4)*8 + 4*g + j%4.
        const int off = base - pos0;  // chunk position of the first q-row key
        uint64_t vis64;
        if (use_tree)
          vis64 = (off >= 0 ? (off >= 64 ? 0ull : mbits << off) : (off <= -64 ? 0ull : mbits >> -off)) |
                  low_bits64(off);
        else
          vis64 = low_bits64(off + node + 1);
        vis64 &= low_bits64(ctxlen - pos0);
        const uint64_t v = vis64 >> (4 * g);
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int bit = kt * 32 + (j >> 2) * 8 + (j & 3);
            sacc[kt][j] = ((v >> bit) & 1ull) ? sacc[kt][j] : -INFINITY;
          }
      }
      // Speculative pass against the current reference max (scores stay unscaled;
      // the scale times log2 e is folded into the exponent).  Each lane holds 16
      // keys of its row; as long as their probabilities sum to <= 2^8 the reference
      // stands (every P <= 2^8, exact after the final 1/l).  Otherwise -- a new
      // maximum more than ~4-8 binary orders above the reference, an overflow, or
      // the first visible keys of the row -- the exact row max of this chunk
      // becomes the reference, O and l are rescaled, and P is recomputed.
      float lsum = probs();
      const bool redo = !(lsum <= 256.f) || m_run == -INFINITY;
      if (__any(redo)) {
        // sacc holds c*s - m_ref; the chunk's exact row max becomes the reference.
        const float m_ref = (m_run == -INFINITY) ? 0.f : m_run;
        float mloc = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int j = 0; j < 16; ++j) mloc = fmaxf(mloc, sacc[kt][j]);
        mloc = fmaxf(mloc, nvx::shfl_xor_f(mloc, 32)) + m_ref;
        const float m_new = fmaxf(m_run, mloc);
        const float alpha = (m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
        l_run *= alpha;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
          for (int j = 0; j < 16; ++j) oacc[dt][j] *= alpha;
        m_run = m_new;
        const float m_ref_new = (m_new == -INFINITY) ? 0.f : m_new;
        const float shift = m_ref - m_ref_new;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int j = 0; j < 16; ++j) sacc[kt][j] += shift;
#pragma unroll
        for (int j = 0; j < 16; ++j) cinit[0][j] = cinit[1][j] = -m_ref_new;
        lsum = probs();
      }
      l_run += lsum;  // this lane's half of the row; the halves meet at the end
    };
    // MFMA phases run at raised wave priority: the wave that reaches the matrix
    // core first keeps it for the whole phase while the other wave on the SIMD
    // does its VALU phase.
    __builtin_amdgcn_s_setprio(1);
    phase_s();
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(0);
    phase_softmax();
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) pv_group(stage, ks, bp[ks]);
    // Transpose reads run two MFMAs ahead.
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int i = 0; i < 14; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    __builtin_amdgcn_s_setprio(0);
  };

  // One chunk in flight: wait for chunk c, barrier (every wave is done with chunk
  // c-1, whose stage receives chunk c+1), then compute chunk c.  The loop is unrolled
  // by the two ring stages, so each step's stage is a compile-time constant.
  using Stage0 = std::integral_constant<int, 0>;
  using Stage1 = std::integral_constant<int, 1>;
  f32x16 sacc[2];
  if (c0 < c1) issue_chunk(c0, Stage0{});
  for (int c = c0; c < c1; c += 2) {
    wait_vm<0>();
    __syncthreads();
    if (c + 1 < c1) issue_chunk(c + 1, Stage1{});
    step(c, Stage0{}, sacc);
    if (c + 1 >= c1) break;
    wait_vm<0>();
    __syncthreads();
    if (c + 2 < c1) issue_chunk(c + 2, Stage0{});
    step(c + 1, Stage1{}, sacc);
  }

  l_run += nvx::shfl_xor_f(l_run, 32);  // both halves share m_run
  if (!row_ok || token >= p.total_q) return;
  const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
  if (p.nsplit == 1) {
    uint16_t* orow = p.o + ((int64_t)token * p.Hq + head) * kD;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int jg = 0; jg < 4; ++jg) {
        const int d = dt * 32 + jg * 8 + 4 * g;
        uint2 pk;
        pk.x = (uint32_t)f2bf(oacc[dt][jg * 4 + 0] * inv) | ((uint32_t)f2bf(oacc[dt][jg * 4 + 1] * inv) << 16);
        pk.y = (uint32_t)f2bf(oacc[dt][jg * 4 + 2] * inv) | ((uint32_t)f2bf(oacc[dt][jg * 4 + 3] * inv) << 16);
        *reinterpret_cast<uint2*>(orow + d) = pk;
      }
  } else {
    const int64_t prow = ((int64_t)split * p.total_q + token) * p.Hq + head;
    float* po = p.part_o + prow * kD;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int jg = 0; jg < 4; ++jg) {
        const int d = dt * 32 + jg * 8 + 4 * g;
        *reinterpret_cast<float4*>(po + d) =
            make_float4(oacc[dt][jg * 4 + 0] * inv, oacc[dt][jg * 4 + 1] * inv,
                        oacc[dt][jg * 4 + 2] * inv, oacc[dt][jg * 4 + 3] * inv);
      }
    if (g == 0) p.part_lse[prow] = l_run > 0.f ? m_run + log2f(l_run) : -INFINITY;
  }
}

// Merge split partials: o = sum_s 2^(lse_s - M) o_s / sum_s 2^(lse_s - M).  Eight
// rows per 256-thread workgroup, 32 lanes per row with four elements each (16-byte
// loads of the fp32 partials).
constexpr int kCombineRows = 8;
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ part_o,
                                                      const float* __restrict__ part_lse,
                                                      uint16_t* __restrict__ o, int rows, int nsplit) {
  const int row = blockIdx.x * kCombineRows + (threadIdx.x >> 5);  // token * Hq + head
  if (row >= rows) return;
  const int d = (threadIdx.x & 31) * 4;
  float M = -INFINITY;
  for (int s = 0; s < nsplit; ++s) M = fmaxf(M, part_lse[(int64_t)s * rows + row]);
  float4 num = make_float4(0.f, 0.f, 0.f, 0.f);
  float den = 0.f;
  if (M != -INFINITY) {
    for (int s = 0; s < nsplit; ++s) {
      const float lse = part_lse[(int64_t)s * rows + row];
      if (lse == -INFINITY) continue;
      const float w = exp2f(lse - M);
      const float4 v = *reinterpret_cast<const float4*>(part_o + ((int64_t)s * rows + row) * kD + d);
      den += w;
      num.x += w * v.x;
      num.y += w * v.y;
      num.z += w * v.z;
      num.w += w * v.w;
    }
  }
  uint2 pk;
  if (den > 0.f) {
    pk.x = (uint32_t)f2bf(num.x / den) | ((uint32_t)f2bf(num.y / den) << 16);
    pk.y = (uint32_t)f2bf(num.z / den) | ((uint32_t)f2bf(num.w / den) << 16);
  } else {
    pk.x = pk.y = 0u;
  }
  *reinterpret_cast<uint2*>(o + (int64_t)row * kD + d) = pk;
}

struct Plan {
  int nq, nsplit, waves;
};

// Waves per workgroup.  A tree-sized work item (at most 64 q rows per sequence) of
// more than 128 q rows (a GQA group of four heads over a 64-node tree: 256 rows) gets
// one 8-wave workgroup, so its K/V is streamed into one CU once; the alternative,
// two 4-wave workgroups per item meeting in L2, streams it twice through the CUs'
// load path.  Measured at 64 sequences of 64-node trees over 2k keys (32/8 heads),
// each launch after a 4096 x 4096 x 6144 GEMM: 150-153 us against 160-164 us.  One
// 8-wave workgroup fills a CU (two waves per SIMD).  Longer q (causal prefill) splits
// into many q-row chunks that re-read the same K/V through L2 anyway; there 4-wave
// workgroups, two per CU, let one workgroup's start (Q and first-chunk loads) and end
// overlap the other's chunks: 4 prompts of 2048 tokens at 32/8 heads 155 us against
// 159 us, 16 prompts of 1024 tokens at 16/8 heads 105 us against 115 us.
int waves_for(int rows, int max_q) { return rows > 128 && max_q <= 64 ? 8 : 4; }

// Chunks one KV split may span: its pages (at most ceil(span / block_size) + 1 of
// them) must fit the workgroup's LDS page table.
int max_split_chunks(int block_size) { return ((kMaxSplitPages - 1) * block_size) / kKC; }

// KV splits: enough to fill one round of kTargetWaves waves (at least ~two chunks per
// split), and at least as many as keep every split within the page table, so a long
// context is split further rather than refused.  block_size = kKC gives the most
// splits any allowed page size needs (the workspace size query has no block size).
Plan make_plan(int num_seqs, int max_q, int max_ctx, int Hq, int Hkv, int block_size) {
  const int G = Hq / Hkv;
  const int rows = G * (max_q > 0 ? max_q : 1);
  Plan pl;
  pl.waves = waves_for(rows, max_q);
  pl.nq = (rows + pl.waves * 32 - 1) / (pl.waves * 32);
  const int64_t waves = (int64_t)num_seqs * Hkv * pl.nq * pl.waves;
  int ns = (int)((kTargetWaves + waves - 1) / (waves > 0 ? waves : 1));
  const int max_chunks = (max_ctx + kKC - 1) / kKC;
  const int cap = max(1, max_chunks / 2);
  if (ns > cap) ns = cap;
  const int per_split = max_split_chunks(block_size);
  const int ns_min = (max_chunks + per_split - 1) / per_split;
  if (ns < ns_min) ns = ns_min;
  if (ns < 1) ns = 1;
  pl.nsplit = ns;
  return pl;
}

size_t workspace_bytes_for(const Plan& pl, int total_q, int Hq) {
  if (pl.nsplit <= 1) return 0;
  return (size_t)pl.nsplit * total_q * Hq * (kD + 1) * sizeof(float);
}

}  // namespace

extern "C" size_t nvx_tree_attention_workspace_size(int32_t num_seqs, int32_t total_q,
                                                    int32_t max_seqlen_q, int32_t max_context_len,
                                                    int32_t num_heads, int32_t num_kv_heads,
                                                    int32_t head_dim) {
  if (num_seqs <= 0 || total_q <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0 ||
      head_dim != kD)
    return 0;
  const Plan pl = make_plan(num_seqs, max_seqlen_q, max_context_len, num_heads, num_kv_heads, kKC);
  return workspace_bytes_for(pl, total_q, num_heads);
}

namespace {

// Validation, plan and launches shared by nvx_tree_attention (caller's workspace)
// and nvx_tree_attention_noalloc (the static scratch).  timed: record the optional
// HIP-event timers (they create events, so the no-alloc entry point does not).
int tree_attention_run(const void* q, void* o, const void* k_cache, const void* v_cache,
                       const int32_t* block_tables, int32_t block_table_stride,
                       const int32_t* cu_seqlens_q, const int32_t* context_lens,
                       const uint64_t* tree_mask, int32_t num_seqs, int32_t total_q,
                       int32_t max_seqlen_q, int32_t max_context_len, int32_t num_heads,
                       int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale,
                       void* (*workspace_of)(size_t need, void* arg), void* workspace_arg,
                       size_t workspace_bytes, void* stream, bool timed) {
  NVX_CHECK(head_dim == kD, "tree_attention: head_dim must be %d (got %d)", kD, head_dim);
  NVX_CHECK(num_kv_heads >= 1 && num_heads >= num_kv_heads && num_heads % num_kv_heads == 0,
            "tree_attention: num_heads (%d) must be a multiple of num_kv_heads (%d)", num_heads,
            num_kv_heads);
  NVX_CHECK(block_size >= kKC && block_size % kKC == 0,
            "tree_attention: block_size must be a positive multiple of %d (got %d)", kKC, block_size);
  NVX_CHECK(num_seqs >= 0 && total_q >= 0 && max_seqlen_q >= 0 && max_context_len >= 0,
            "tree_attention: negative size");
  NVX_CHECK(tree_mask == nullptr || max_seqlen_q <= 64,
            "tree_attention: a tree mask allows at most 64 query rows per sequence (got %d)",
            max_seqlen_q);
  NVX_CHECK(block_table_stride >= 1, "tree_attention: block_table_stride must be >= 1");
  if (num_seqs == 0 || total_q == 0) return NVX_OK;
  NVX_CHECK(q && o && k_cache && v_cache && block_tables && cu_seqlens_q && context_lens,
            "tree_attention: null pointer");
  const Plan pl =
      make_plan(num_seqs, max_seqlen_q, max_context_len, num_heads, num_kv_heads, block_size);
  {
    const int chunks = (max_context_len + kKC - 1) / kKC;
    const int cps = (chunks + pl.nsplit - 1) / pl.nsplit;
    NVX_CHECK((cps * kKC + block_size - 1) / block_size + 1 <= kMaxSplitPages,
              "tree_attention: context of %d tokens spans more than %d pages per split",
              max_context_len, kMaxSplitPages);
  }
  const size_t need = workspace_bytes_for(pl, total_q, num_heads);
  NVX_CHECK(workspace_bytes >= need,
            "tree_attention: workspace of %zu bytes required (got %zu)", need, workspace_bytes);
  void* workspace = need ? workspace_of(need, workspace_arg) : nullptr;
  if (need && !workspace) return NVX_EHIP;  // workspace_of reported the failure

  AttnParams p;
  p.q = (const uint16_t*)q;
  p.o = (uint16_t*)o;
  p.k_cache = (const uint16_t*)k_cache;
  p.v_cache = (const uint16_t*)v_cache;
  p.block_tables = block_tables;
  p.cu_q = cu_seqlens_q;
  p.ctx_lens = context_lens;
  p.tree_mask = tree_mask;
  p.part_o = (float*)workspace;
  p.part_lse = pl.nsplit > 1 ? (float*)workspace + (size_t)pl.nsplit * total_q * num_heads * kD : nullptr;
  p.bt_stride = block_table_stride;
  p.num_seqs = num_seqs;
  p.total_q = total_q;
  p.Hq = num_heads;
  p.Hkv = num_kv_heads;
  p.G = num_heads / num_kv_heads;
  p.block_size = block_size;
  p.nq = pl.nq;
  p.nsplit = pl.nsplit;
  p.scale_log2 = scale * 1.4426950408889634f;

  hipStream_t s = (hipStream_t)stream;
  nvx::TimerScope timer(timed ? NVX_TIMER_TREE_ATTENTION : -1, s);
  const int64_t nblocks = (int64_t)num_seqs * num_kv_heads * pl.nq * pl.nsplit;
  NVX_CHECK(nblocks < (1ll << 31), "tree_attention: grid too large");
  const dim3 grid((unsigned)nblocks);
  // One q-row chunk per (sequence, KV head): K/V is streamed once (32 sequences of
  // 32-node trees over 1-4k keys, 16/8 heads: 85 us against 93 us with cached loads;
  // decode of 64 x 2k keys: 89 us against 102 us).  Two or more chunks share K/V
  // through L2, which non-temporal loads would give up (64 sequences of 64-node trees
  // over 2k keys, 32/8 heads, in 4-wave workgroups: 220 us against 202 us with sc1
  // loads).
  if (pl.waves == 8) {
    if (pl.nq == 1)
      hipLaunchKernelGGL((tree_attn_kernel<8, kStream>), grid, dim3(8 * 64), 0, s, p);
    else
      hipLaunchKernelGGL((tree_attn_kernel<8, kShared>), grid, dim3(8 * 64), 0, s, p);
  } else {
    if (pl.nq == 1)
      hipLaunchKernelGGL((tree_attn_kernel<4, kStream>), grid, dim3(4 * 64), 0, s, p);
    else
      hipLaunchKernelGGL((tree_attn_kernel<4, kShared>), grid, dim3(4 * 64), 0, s, p);
  }
  NVX_LAUNCHED();
  if (pl.nsplit > 1) {
    const int rows = total_q * num_heads;
    hipLaunchKernelGGL(combine_kernel, dim3((rows + kCombineRows - 1) / kCombineRows), dim3(256), 0,
                       s, p.part_o, p.part_lse, (uint16_t*)o, rows, pl.nsplit);
    NVX_LAUNCHED();
  }
  return NVX_OK;
}

void* caller_workspace(size_t need, void* ws) {
  if (!ws) nvx::fail(NVX_EINVAL, "tree_attention: workspace of %zu bytes required (got NULL)", need);
  return ws;
}

// ---------------------------------------------------------------- static scratch
// Split-KV partials of nvx_tree_attention_noalloc live in this array instead of a
// caller workspace.  Every GPU the library runs on holds its own copy for the life
// of the process.  In host code `scratch` names a host-side stand-in, not device
// memory: the device address comes from hipGetSymbolAddress, once per device.
constexpr size_t kScratchBytes = size_t(64) << 20;
constexpr int kMaxDevices = 64;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

std::once_flag g_scratch_once[kMaxDevices];
void* g_scratch_ptr[kMaxDevices];
hipError_t g_scratch_err[kMaxDevices];

// The device address of `scratch` on the device current at the call (which must be
// the launch stream's device), looked up on the first call per device.
void* scratch_workspace(size_t need, void* stream) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    nvx::fail(NVX_EHIP, "tree_attention_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    nvx::fail(NVX_EINVAL, "tree_attention_noalloc: device %d beyond the %d supported", dev,
              kMaxDevices);
    return nullptr;
  }
  if (stream) {
    int sdev = -1;
    e = hipStreamGetDevice((hipStream_t)stream, &sdev);
    if (e != hipSuccess || sdev != dev) {
      nvx::fail(NVX_EINVAL, "tree_attention_noalloc: the stream belongs to device %d, the "
                "current device is %d", sdev, dev);
      return nullptr;
    }
  }
  std::call_once(g_scratch_once[dev], [dev] {
    g_scratch_err[dev] = hipGetSymbolAddress(&g_scratch_ptr[dev], HIP_SYMBOL(scratch));
  });
  if (g_scratch_err[dev] != hipSuccess || !g_scratch_ptr[dev]) {
    nvx::fail(NVX_EHIP, "tree_attention_noalloc: hipGetSymbolAddress(scratch): %s",
              hipGetErrorString(g_scratch_err[dev]));
    return nullptr;
  }
  (void)need;  // checked against kScratchBytes by the caller
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" int nvx_tree_attention(const void* q, void* o, const void* k_cache, const void* v_cache,
                                  const int32_t* block_tables, int32_t block_table_stride,
                                  const int32_t* cu_seqlens_q, const int32_t* context_lens,
                                  const uint64_t* tree_mask, int32_t num_seqs, int32_t total_q,
                                  int32_t max_seqlen_q, int32_t max_context_len, int32_t num_heads,
                                  int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                  float scale, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  nvx::clear_error();
  return tree_attention_run(q, o, k_cache, v_cache, block_tables, block_table_stride,
                            cu_seqlens_q, context_lens, tree_mask, num_seqs, total_q,
                            max_seqlen_q, max_context_len, num_heads, num_kv_heads, head_dim,
                            block_size, scale, caller_workspace, workspace, workspace_bytes,
                            stream, true);
}

extern "C" size_t nvx_tree_attention_noalloc_scratch_bytes(void) { return kScratchBytes; }

extern "C" int nvx_tree_attention_noalloc(const void* q, void* o, const void* k_cache,
                                          const void* v_cache, const int32_t* block_tables,
                                          int32_t block_table_stride, const int32_t* cu_seqlens_q,
                                          const int32_t* context_lens, const uint64_t* tree_mask,
                                          int32_t num_seqs, int32_t total_q, int32_t max_seqlen_q,
                                          int32_t max_context_len, int32_t num_heads,
                                          int32_t num_kv_heads, int32_t head_dim,
                                          int32_t block_size, float scale, void* stream) {
  nvx::clear_error();
  // the scratch capacity stands in for the workspace size: a launch whose split-KV
  // partials need more is refused with the size it would need
  const size_t need = nvx_tree_attention_workspace_size(num_seqs, total_q, max_seqlen_q,
                                                        max_context_len, num_heads, num_kv_heads,
                                                        head_dim);
  NVX_CHECK(need <= kScratchBytes,
            "tree_attention_noalloc: split-KV partials need %zu bytes, the static scratch holds "
            "%zu (use nvx_tree_attention with a workspace)", need, kScratchBytes);
  return tree_attention_run(q, o, k_cache, v_cache, block_tables, block_table_stride,
                            cu_seqlens_q, context_lens, tree_mask, num_seqs, total_q,
                            max_seqlen_q, max_context_len, num_heads, num_kv_heads, head_dim,
                            block_size, scale, scratch_workspace, stream, kScratchBytes, stream,
                            false);
}
