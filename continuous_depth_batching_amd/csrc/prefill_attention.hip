// Chunked-prefill (varlen, causal) paged attention on MFMA tiles (CDNA4).
//
// Replaces flash_attn_varlen_func as the reference's prefill path calls it
// after writing the chunk's K/V into the paged cache
// (continuous_batching/prefill_graph.py:265-309, transformers
// integrations/flash_paged.py:62-86): query tokens of sequence s sit at
// positions past[s] .. past[s]+len[s]-1 and attend causally to every cached
// position 0..(own position) of the same cache layer, read through the
// sequence's block table. The chunk's own K/V must already be in the pool
// (cdb_rope_kv_write), so the kernel never touches new keys separately.
//
// Work unit: a tile of 128 query tokens of one sequence and one query head.
//
// bf16 (the serving path): one workgroup of 4 waves per tile, 32 queries per
// wave, on v_mfma_f32_32x32x16_bf16. Keys stream through LDS in blocks of 32:
// a ring of three stages holds each block's K and V in natural [key][head-dim]
// layout (16-byte chunks XOR-swizzled per row), filled by direct-to-LDS block
// loads (global_load_lds_dwordx4) two blocks ahead of the block being
// multiplied, one barrier per block.
//   S^T = K Q^T     A = 32 key rows from LDS, B = the wave's Q^T (registers)
//   O^T += V^T P^T  A = V^T from LDS by transpose loads (ds_read_b64_tr_b16),
//                   B = P^T straight from the S^T accumulators (lane l owns
//                   query l%32 in both)
// Lane l holds 16 of the 32 keys of its query; the other 16 sit in lane l^32,
// so a query's block max is one v_permlane32_swap away. Along the contraction
// the MFMA k-index is bound to keys by the accumulator layout of S^T, and the
// transpose loads read V rows in that order.
// The running max is only raised when a block's max exceeds it by more than
// 2^8 (in exp2 units): until then the probabilities are taken against the
// stale max, which stays exact (the same max divides out of numerator and
// denominator) and only lets them grow to 256, well inside bf16 and fp32
// range; the rescale of the 32x128 accumulator is thus skipped on almost all
// blocks.
// Split tiles (cdb_prefill_attention_split): a long tile's key blocks can be
// spread over several workgroups, each writing an unnormalized partial (O, max,
// row sum) that prefill_merge_kernel combines, so that one long sequence does
// not set the length of the whole launch.
//
// fp32 (reference-precision models and tests): two workgroups of 4 waves per
// tile, 16 queries per wave, on v_mfma_f32_16x16x4f32 with K and V^T staged in
// LDS through registers.

#include "cdb_common.h"
#include "../../include/cdb_amd.h"

namespace cdb {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;

struct PrefillParams {
  const void* q;               // [T, H, D] rotated queries
  const void* k_pool;
  const void* v_pool;
  int64_t layer_stride;
  int32_t layer;
  const int32_t* block_table;  // [table_rows, W]
  const int32_t* table_row;    // [S]
  const int32_t* cu_q;         // [S+1] query-token offsets
  const int32_t* past;         // [S] position of each sequence's first query token
  const int32_t* tile_seq;     // [tiles]
  const int32_t* tile_q0;      // [tiles] first query index (within the sequence) of the tile
  // Split work (bf16 only; null for whole tiles): items [tiles][4] = (sequence,
  // first query, first key block | end key block << 16, partial slot or -1),
  // merges [num_merges][4] = (sequence, first query, first slot, parts).
  const int32_t* items;
  const int32_t* merges;
  float* partials;             // [slots][H][128][D + 2]: unnormalized O, then m and l per query
  void* out;                   // [T, H, D]
  int64_t pool_blocks;
  int32_t num_tiles, num_seqs, num_merges, num_slots;
  int32_t num_heads, num_kv_heads, table_width, block_size_log2;
  float scale_log2;
};

constexpr int kTileQueries = 128;  // queries per tile (the host's tile list uses the same size)
constexpr int kKeys = 32;          // keys per staged block
constexpr int kLdsPages = 1024;    // block ids kept in LDS per workgroup (longer prefixes read the table)
constexpr float kRescaleSlack = 8.f;  // log2 of the largest probability allowed against a stale max

// Where a workgroup's queries and keys live; shared by both kernels.
struct TileGeometry {
  int q_begin, q_len, past, q0, key_end;
  int kvh;
  const int32_t* table;
  bool pages_in_lds;
};

// Reads sequence `s`'s extents. `q0` is the workgroup's first query (within
// the sequence) and `queries` its query count.
CDB_DEVICE TileGeometry tile_geometry(const PrefillParams& P, int s, int q0, int h, int queries) {
  TileGeometry g;
  g.q_begin = P.cu_q[s];
  g.q_len = P.cu_q[s + 1] - g.q_begin;
  g.past = P.past[s];
  g.q0 = q0;
  g.kvh = h / (P.num_heads / P.num_kv_heads);
  g.table = P.block_table + (int64_t)P.table_row[s] * P.table_width;
  // Keys needed by the workgroup: up to its last valid query's position.
  g.key_end = g.past + min(g.q0 + queries, g.q_len);
  const int bs_mask = (1 << P.block_size_log2) - 1;
  g.pages_in_lds = ((g.key_end + bs_mask) >> P.block_size_log2) <= kLdsPages;
  return g;
}

// Copies the prefix's block ids into `page_lds` when they fit; the caller
// issues the barrier.
CDB_DEVICE void fill_page_table(const PrefillParams& P, const TileGeometry& g, int* page_lds) {
  if (!g.pages_in_lds) return;
  const int key_pages = (g.key_end + (1 << P.block_size_log2) - 1) >> P.block_size_log2;
  for (int i = threadIdx.x; i < key_pages; i += blockDim.x) page_lds[i] = i < P.table_width ? g.table[i] : -1;
}

// Pool element offset of key `kp`'s row for the tile's KV head, or -1 when the
// key lies past key_end or its page is unmapped / out of the pool.
CDB_DEVICE int64_t key_offset(const PrefillParams& P, const TileGeometry& g, const int* page_lds, int kp, int D) {
  if (kp >= g.key_end) return -1;
  const int page = kp >> P.block_size_log2;
  const int blk = g.pages_in_lds ? page_lds[page] : (page < P.table_width ? g.table[page] : -1);
  if (blk < 0 || blk >= P.pool_blocks) return -1;
  const int bs_mask = (1 << P.block_size_log2) - 1;
  return ((int64_t)blk * (bs_mask + 1) + (kp & bs_mask)) * ((int64_t)P.num_kv_heads * D) + (int64_t)g.kvh * D;
}

// LDS image of a 32-key block of K or V for the bf16 kernel: row = key, 16-byte
// chunks of head-dim, kRowChunks per row (8 for D <= 64, else 16; D = 96 leaves
// chunks 12..15 empty). Chunk c of row r sits at slot c ^ swizzle(r), with
// swizzle(r) = 2 * sub(r): the 8 rows read together by an S^T operand load and
// the 4 rows x 2 chunks read together by a V transpose load then fall in
// distinct banks.
template <int D> struct BlockLayout {
  static constexpr int kRowChunks = D <= 64 ? 8 : 16;
  static constexpr int kRowBytes = kRowChunks * 16;
  static constexpr int kBytes = kKeys * kRowBytes;
  static constexpr int kChunks = D / 8;                  // chunks holding data
  static constexpr int kWaveLoads = kBytes / (4 * 1024);  // 1 KiB loads per wave per block (K or V)
  static CDB_DEVICE int sub(int row) { return kRowChunks == 16 ? (row & 7) : ((row >> 1) & 3); }
};

typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2_t;

// LDS byte address of a __shared__ object.
CDB_DEVICE uint32_t lds_address(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// The bf16 kernel reads the staged blocks with its own LDS instructions and
// waits for them itself (s_waitcnt lgkmcnt); the compiler does not see these
// reads, so it does not hold them back behind the block loads still in flight
// into the other stages. LDS operations complete in order, so the compiler's
// own lgkmcnt waits stay correct around them.
CDB_DEVICE u32x4_t lds_read_b128(uint32_t addr) {
  u32x4_t v;
  __asm__ volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}
template <int kOffset> CDB_DEVICE u32x2_t lds_read_tr16_b64(uint32_t addr) {
  u32x2_t v;
  __asm__ volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(kOffset));
  return v;
}
CDB_DEVICE int lds_read_i32_now(uint32_t addr) {
  int v;
  __asm__ volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr));
  return v;
}
// A block id from the table in global memory, for prefixes longer than the
// LDS copy; waits for every outstanding load (the block loads included), which
// only such long prefixes pay.
CDB_DEVICE int global_read_i32_now(const int32_t* p) {
  int v;
  __asm__ volatile("global_load_dword %0, %1, off\n\ts_waitcnt vmcnt(0)" : "=v"(v) : "v"(p) : "memory");
  return v;
}
// Waits for every LDS read issued so far; `token` (one of the values read)
// comes out of the wait, and lds_after ties further values to it, so no use of
// them can be scheduled ahead of the wait. Only the wait itself is volatile, so
// the instructions after it remain free to interleave.
template <typename T> CDB_DEVICE void lds_wait(T& token) {
  __asm__ volatile("s_waitcnt lgkmcnt(0)" : "+v"(token)::"memory");
}
template <typename T, typename U> CDB_DEVICE void lds_after(T& v, const U& token) {
  __asm__("" : "+v"(v) : "v"(token));
}
// Waits until the MFMA that produced `acc` (and every MFMA issued before it) has
// finished. The compiler does not know that the LDS reads above write their
// registers only when the data arrives, so it may give them registers that an
// MFMA still in flight is reading; reads issued after a drain cannot overwrite
// a source of an unfinished MFMA.
CDB_DEVICE void mfma_drain(const f32x16_t& acc) {
  float done;
  __asm__ volatile("v_mov_b32 %0, %1" : "=v"(done) : "v"(acc[15]));
  (void)done;
}
// 16 bytes per lane from global memory, not tracked by the compiler: the
// caller waits for it with its own s_waitcnt vmcnt and ties the value to that
// wait (lds_after).
CDB_DEVICE u32x4_t global_load_b128(const void* p) {
  u32x4_t v;
  __asm__ volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(p) : "memory");
  return v;
}
// Block load: 16 bytes per lane from `src` into LDS at lds_base + 16 * lane
// (lds_base uniform over the wave). The compiler sets M0 for it and counts it
// among the vector-memory operations; this kernel reads the staged blocks with
// its own LDS instructions, so the compiler never holds an LDS read back
// behind these loads, and the loop waits for them itself (s_waitcnt vmcnt,
// kDmaPerBlock loads per block).
CDB_DEVICE void block_load_lds(const void* src, uint32_t lds_base) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(uintptr_t)lds_base, 16, 0, 0);
}

template <int D>
__global__ void __launch_bounds__(256) prefill_attention_bf16_kernel(PrefillParams P) {
  using L = BlockLayout<D>;
  constexpr int kStages = 3;               // key blocks resident: computing b, in flight b+1 and b+2
  constexpr int kQSteps = D / 16;          // S^T MFMA k-steps over head_dim
  constexpr int kDTiles = D / 32;          // O^T tiles of 32 head-dim rows
  constexpr int kDmaPerBlock = 2 * L::kWaveLoads;  // vmcnt per wave per issued block
  static_assert(D % 32 == 0 && D <= 128, "head_dim must be 64, 96 or 128");
  static_assert(L::kWaveLoads >= 1 && L::kBytes % (4 * 1024) == 0, "a block is whole 1 KiB loads per wave");

  // Stage s: K image at s * 2 * kBytes, V image right after it.
  __shared__ __attribute__((aligned(1024))) unsigned char ring[kStages * 2 * L::kBytes];
  __shared__ int page_lds[kLdsPages];

  // One workgroup per (tile, head), heads fastest: the host lists the tiles
  // longest prefix first, so the heaviest workgroups of every head start first.
  const int tile = blockIdx.x / P.num_heads;
  const int h = blockIdx.x - tile * P.num_heads;
  if (tile >= P.num_tiles) return;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int col = lane & 31;   // query column of S^T / O^T, or row of an A operand
  const int half = lane >> 5;  // k-slice half of the operands

  // A whole tile, or one part of its key blocks whose unnormalized result goes
  // to a partial slot for prefill_merge_kernel.
  int seq, tile_q0, kv_first = 0, kv_end = 0x7fffffff, slot = -1;
  if (P.items) {
    const int4 it = reinterpret_cast<const int4*>(P.items)[tile];
    seq = it.x;
    tile_q0 = it.y;
    kv_first = it.z & 0xffff;
    kv_end = it.z >> 16;
    slot = it.w;
  } else {
    seq = P.tile_seq[tile];
    tile_q0 = P.tile_q0[tile];
  }
  if (seq < 0 || seq >= P.num_seqs || slot >= P.num_slots) return;  // malformed work list: nothing to write
  const TileGeometry g = tile_geometry(P, seq, tile_q0, h, kTileQueries);
  const bf16_t* k_base = static_cast<const bf16_t*>(P.k_pool) + (int64_t)P.layer * P.layer_stride;
  const bf16_t* v_base = static_cast<const bf16_t*>(P.v_pool) + (int64_t)P.layer * P.layer_stride;

  const int wave_q0 = g.q0 + wave * 32;
  const bool wave_active = wave_q0 < g.q_len;
  const int q_local = wave_q0 + col;
  const bool q_valid = q_local < g.q_len;
  const int q_pos = g.past + q_local;
  const int wave_first_pos = g.past + wave_q0;
  const int wave_key_end = g.past + min(wave_q0 + 32, g.q_len);
  // This workgroup's key blocks: [block0, num_blocks). A part never starts past
  // the tile's first query position, so key `block0 * 32` is visible to every
  // query and the running max is finite from the first block on.
  const int num_blocks = min((g.key_end + kKeys - 1) / kKeys, kv_end);
  const int block0 = kv_first;

  // Q^T operand: k-step c covers head-dim 16c + 8*half .. +7 of query `col`;
  // lanes past the chunk read query 0 and use zeros.
  u32x4_t q_raw[kQSteps];
  bf16x8_t qv[kQSteps];
  {
    const bf16_t* qrow = static_cast<const bf16_t*>(P.q) +
                         ((int64_t)(g.q_begin + (q_valid ? q_local : 0)) * P.num_heads + h) * D;
#pragma unroll
    for (int c = 0; c < kQSteps; ++c) q_raw[c] = global_load_b128(qrow + 16 * c + 8 * half);
  }
  // The block ids' loads overlap Q's; both have landed before the first block
  // load is issued (loads and stores of different kinds need not complete in
  // order, so the block-load waits below count block loads alone).
  fill_page_table(P, g, page_lds);
  __asm__ volatile("s_waitcnt vmcnt(0)" : "+v"(q_raw[0])::"memory");
#pragma unroll
  for (int c = 0; c < kQSteps; ++c) {
    if (c > 0) lds_after(q_raw[c], q_raw[0]);
    const u32x4_t v = q_valid ? q_raw[c] : u32x4_t{0u, 0u, 0u, 0u};
    __builtin_memcpy(&qv[c], &v, 16);
  }

  // Block loads: wave w's load i fills bytes (4i + w) KiB .. +1 KiB of an image;
  // lane l of it fetches the chunk that lands at slot (4i + w) * 64 + l. Keys
  // past key_end fetch the row of key key_end - 1 (always written, so finite:
  // their probabilities are 0 and 0 * V must stay 0).
  const uint32_t ring_lds = lds_address(ring);
  const uint32_t page_base = lds_address(page_lds);
  const int bs_mask = (1 << P.block_size_log2) - 1;
  const int64_t row_elems = (int64_t)P.num_kv_heads * D;
  auto issue_block = [&](int b) {
    if (b >= num_blocks) return;
    const uint32_t k_img = ring_lds + (b % kStages) * 2 * L::kBytes;
    // The lane's rows and chunks are recomputed per block (the volatile asm
    // keeps them from being hoisted into registers held across the loop).
    int ln = lane;
    __asm__ volatile("" : "+v"(ln));
#pragma unroll
    for (int i = 0; i < L::kWaveLoads; ++i) {
      const int slot_index = (4 * i + wave) * 64 + ln;
      const int row = slot_index / L::kRowChunks;
      const int chunk = (slot_index % L::kRowChunks) ^ (2 * L::sub(row));
      const int kp = min(b * kKeys + row, g.key_end - 1);
      const int page = kp >> P.block_size_log2;
      const int blk = g.pages_in_lds ? lds_read_i32_now(page_base + 4 * page)
                                     : (page < P.table_width ? global_read_i32_now(g.table + page) : -1);
      // An unmapped page (a malformed table) reads pool row 0: in bounds, values unspecified.
      const int64_t pool_row = blk >= 0 && blk < P.pool_blocks ? (int64_t)blk * (bs_mask + 1) + (kp & bs_mask) : 0;
      const int64_t off = pool_row * row_elems + g.kvh * D + chunk * 8;
      const uint32_t dst = k_img + (4 * i + wave) * 1024;
      if (chunk < L::kChunks) {
        block_load_lds(k_base + off, dst);
        block_load_lds(v_base + off, dst + L::kBytes);
      }
    }
  };

  // Operand addresses within a stage. S^T: row `col`, logical chunk 2c + half
  // -> byte col * kRowBytes + ((c ^ sub) * 2 + half) * 16. V^T (transpose loads,
  // 4 keys x 16 head-dims per 16 lanes): lane (grp, r, e) = (lane / 16,
  // lane / 4 % 4, lane % 4) reads 8 bytes of key row 16t + 8a + 4(grp / 2) + r at
  // head-dim 32j + 16(grp % 2) + 4e; the swizzle of those rows depends only on
  // (grp / 2, r), so per j one base serves every (t, a) through the offset field.
  const int k_sub = L::sub(col);
  const uint32_t k_read = col * L::kRowBytes + half * 16;
  const int vgrp = lane >> 4, vr = (lane >> 2) & 3, ve = lane & 3;
  const int v_row0 = 4 * (vgrp >> 1) + vr;
  // Tile j's chunk is 4j + c0 with c0 = 2(grp % 2) + e / 2 < 4, so its slot
  // (4j + c0) ^ swizzle = 4j ^ (c0 ^ swizzle): byte (j << 6) ^ v_xor.
  const uint32_t v_base_off = L::kBytes + v_row0 * L::kRowBytes + (ve & 1) * 8;
  const uint32_t v_xor = (uint32_t)((2 * (vgrp & 1) + (ve >> 1)) ^ (2 * L::sub(v_row0))) << 4;

  f32x16_t o[kDTiles];
#pragma unroll
  for (int j = 0; j < kDTiles; ++j) o[j] = f32x16_t{};
  float m_run = -INFINITY;  // the max the probabilities are taken against (exp2 units)
  float l = 0.f;            // this lane's share of the row sum
  // Blocks this wave computes: up to its last query's position.
  const int wave_blocks = wave_active ? min((wave_key_end + kKeys - 1) / kKeys, num_blocks) : 0;

  // S^T of a block: lane holds keys kb + 8*(i/4) + 4*half + i%4 (i = 0..15) of query `col`.
  // The operand addresses are formed afresh for every block (the volatile asm
  // keeps the compiler from hoisting a register per address out of the loop).
  auto read_k = [&](uint32_t img, u32x4_t (&kr)[kQSteps]) {
    uint32_t base = img + k_read, sub32 = (uint32_t)k_sub << 5;
    __asm__ volatile("" : "+v"(base), "+v"(sub32));
#pragma unroll
    for (int c = 0; c < kQSteps; ++c) kr[c] = lds_read_b128(base + (((uint32_t)c << 5) ^ sub32));
  };
  auto scores = [&](u32x4_t (&kr)[kQSteps]) {
    f32x16_t s = f32x16_t{};
#pragma unroll
    for (int c = 0; c < kQSteps; ++c) {
      bf16x8_t kv;
      __builtin_memcpy(&kv, &kr[c], 16);
      s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kv, qv[c], s, 0, 0, 0);
    }
    return s;
  };
  // V^T operands of a block: keys 16t + 4*half + 0..3 (a = 0) and 16t + 8 + 4*half + 0..3
  // (a = 1) at head-dim 32j + col.
  u32x2_t vt[kDTiles][2][2];
  auto read_v = [&](uint32_t img, int j) {
    uint32_t base = img + v_base_off, x = v_xor;
    __asm__ volatile("" : "+v"(base), "+v"(x));
    const uint32_t addr = base + (((uint32_t)j << 6) ^ x);
    vt[j][0][0] = lds_read_tr16_b64<0>(addr);
    vt[j][0][1] = lds_read_tr16_b64<8 * L::kRowBytes>(addr);
    vt[j][1][0] = lds_read_tr16_b64<16 * L::kRowBytes>(addr);
    vt[j][1][1] = lds_read_tr16_b64<24 * L::kRowBytes>(addr);
  };
  // Causal mask, only on blocks that reach past the wave's first query or the last key.
  auto mask = [&](f32x16_t& s, int kb) {
    if (kb + kKeys - 1 > wave_first_pos || kb + kKeys > g.key_end) {
      const int last = min(q_pos, g.key_end - 1) - kb - 4 * half;  // last visible key, relative
#pragma unroll
      for (int i = 0; i < 16; ++i) s[i] = 8 * (i >> 2) + (i & 3) <= last ? s[i] : -INFINITY;
    }
  };
  // Softmax of a block's (masked) scores into bf16 P^T operands, in eight
  // branch-free stages.
  // The running max moves (by a select) only when the block's max exceeds it by
  // more than 2^kRescaleSlack; the accumulator rescale that then follows is the
  // caller's (rare) branch.
  struct Softmax {
    float mx, m_next, alpha, psum;
    float p[16];
  };
  auto softmax_stage = [&](int k, const f32x16_t& s, Softmax& st, bf16x8_t (&pb)[2]) {
    if (k == 0) {
      st.mx = s[0];
#pragma unroll
      for (int i = 1; i < 8; ++i) st.mx = fmaxf(st.mx, s[i]);
    } else if (k == 1) {
#pragma unroll
      for (int i = 8; i < 16; ++i) st.mx = fmaxf(st.mx, s[i]);
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(st.mx), __float_as_uint(st.mx), false, false);
      st.mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
    } else if (k == 2) {
      // Key kb is visible to every query of an active wave from block 0 on, so
      // m_run is finite after the first block; exp2(-inf) = 0 covers the first
      // rescale and every masked key.
      const float m_blk = st.mx * P.scale_log2;
      const bool grow = m_blk > m_run + kRescaleSlack;
      st.m_next = grow ? m_blk : m_run;
      st.alpha = grow ? __builtin_amdgcn_exp2f(m_run - st.m_next) : 1.f;
      m_run = st.m_next;
    } else if (k <= 6) {
#pragma unroll
      for (int i = 4 * (k - 3); i < 4 * (k - 2); ++i)
        st.p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[i], P.scale_log2, -st.m_next));
    } else {
      st.psum = st.p[0];
#pragma unroll
      for (int i = 1; i < 16; ++i) st.psum += st.p[i];
      l = l * st.alpha + st.psum;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int j = 0; j < 8; ++j) pb[t][j] = (__bf16)st.p[8 * t + j];
    }
  };
  auto rescale = [&](float alpha) {
    if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {
#pragma unroll
      for (int j = 0; j < kDTiles; ++j) o[j] *= alpha;
    }
  };
  auto accumulate = [&](const bf16x8_t (&pb)[2], int j) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      bf16x8_t va;
      __builtin_memcpy(&va, &vt[j][t][0], 8);
      __builtin_memcpy(reinterpret_cast<char*>(&va) + 8, &vt[j][t][1], 8);
      o[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb[t], o[j], 0, 0, 0);
    }
  };
  constexpr int kJ0 = 1;  // V^T tiles read during the softmax; the rest after the first P V
  auto stage_lds = [&](int b) { return ring_lds + (b % kStages) * 2 * L::kBytes; };

  lds_barrier();  // page_lds
  for (int i = 0; i < kStages - 1; ++i) issue_block(block0 + i);
  // The first block landed once at most the second block's loads are outstanding.
  if (num_blocks > block0 + 1) {
    __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(kDmaPerBlock) : "memory");
  } else {
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  for (int b = block0; b < num_blocks; ++b) {
    // Block b has landed once at most block b + 1's loads are outstanding.
    if (b > block0) {
      if (b + 1 < num_blocks) {
        __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(kDmaPerBlock) : "memory");
      } else {
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
    }
    lds_barrier();  // every wave's loads of block b are in; stage (b - 1) % 3 is free
    issue_block(b + kStages - 1);
    if (b >= wave_blocks) continue;
    const int kb = b * kKeys;
    const uint32_t img = stage_lds(b);
    mfma_drain(o[kDTiles - 1]);  // the previous block's P V products
    // Scores, then the first V^T operands, read once the score MFMAs are done
    // (into the registers the K operands held) and landing during the softmax.
    f32x16_t s;
    {
      u32x4_t kr[kQSteps];
      read_k(img, kr);
      lds_wait(kr[0]);
#pragma unroll
      for (int c = 1; c < kQSteps; ++c) lds_after(kr[c], kr[0]);
      s = scores(kr);
    }
    mfma_drain(s);
#pragma unroll
    for (int j = 0; j < kJ0; ++j) read_v(img, j);
    bf16x8_t pb[2];
    Softmax st;
    mask(s, kb);
#pragma unroll
    for (int k = 0; k < 8; ++k) softmax_stage(k, s, st, pb);
    rescale(st.alpha);
    lds_wait(vt[kJ0 - 1][1][1]);
#pragma unroll
    for (int j = 0; j < kJ0; ++j)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (j != kJ0 - 1 || t != 3) lds_after(vt[j][t >> 1][t & 1], vt[kJ0 - 1][1][1]);
      }
#pragma unroll
    for (int j = 0; j < kJ0; ++j) accumulate(pb, j);
    if constexpr (kJ0 < kDTiles) {
      mfma_drain(o[kJ0 - 1]);
#pragma unroll
      for (int j = kJ0; j < kDTiles; ++j) read_v(img, j);
      lds_wait(vt[kDTiles - 1][1][1]);
#pragma unroll
      for (int j = kJ0; j < kDTiles; ++j)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          if (j != kDTiles - 1 || t != 3) lds_after(vt[j][t >> 1][t & 1], vt[kDTiles - 1][1][1]);
        }
#pragma unroll
      for (int j = kJ0; j < kDTiles; ++j) accumulate(pb, j);
    }
  }

  // Row sum over both lane halves, normalize, store O (lane: query col,
  // head-dim 32j + 8*(i/4) + 4*half + i%4).
  {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l), __float_as_uint(l), false, false);
    l = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  if (!q_valid) return;
  if (slot >= 0) {
    // Partial: unnormalized O^T, the running max (exp2 units) and the row sum.
    const int qi = wave * 32 + col;
    float* part = P.partials + ((int64_t)slot * P.num_heads + h) * (kTileQueries * (D + 2));
#pragma unroll
    for (int j = 0; j < kDTiles; ++j)
#pragma unroll
      for (int a = 0; a < 4; ++a)
        *reinterpret_cast<float4*>(part + qi * D + 32 * j + 8 * a + 4 * half) =
            make_float4(o[j][4 * a], o[j][4 * a + 1], o[j][4 * a + 2], o[j][4 * a + 3]);
    if (half == 0) {
      part[kTileQueries * D + qi] = m_run;
      part[kTileQueries * D + kTileQueries + qi] = l;
    }
    return;
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  bf16_t* orow = static_cast<bf16_t*>(P.out) + ((int64_t)(g.q_begin + q_local) * P.num_heads + h) * D;
#pragma unroll
  for (int j = 0; j < kDTiles; ++j)
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      Vec<bf16_t, 4> ov;
      ov.set_pair(0, o[j][4 * a] * inv, o[j][4 * a + 1] * inv);
      ov.set_pair(2, o[j][4 * a + 2] * inv, o[j][4 * a + 3] * inv);
      ov.store(orow + 32 * j + 8 * a + 4 * half);
    }
}

// Combines the parts of split tiles: per query, M = max_p m_p and
// O = sum_p 2^(m_p - M) O_p / sum_p 2^(m_p - M) l_p, written as bf16. One
// thread per (query, 4 head-dims), kMergeGroups workgroups per (tile, head),
// so every partial element is read by one thread with all its parts' loads in
// flight together.
constexpr int kMergeGroups = 16;
template <int D>
__global__ void __launch_bounds__(256) prefill_merge_kernel(PrefillParams P) {
  constexpr int kChunks = D / 4;
  constexpr int kPart = kTileQueries * (D + 2);
  constexpr int kMaxParts = 8;  // parts combined per pass of the loop below
  static_assert(kTileQueries * kChunks <= kMergeGroups * 256, "one thread per (query, 4 head-dims)");
  const int group = blockIdx.x % kMergeGroups;
  const int mh = blockIdx.x / kMergeGroups;
  const int merge = mh / P.num_heads;
  const int h = mh - merge * P.num_heads;
  if (merge >= P.num_merges) return;
  const int4 mg = reinterpret_cast<const int4*>(P.merges)[merge];
  if (mg.x < 0 || mg.x >= P.num_seqs || mg.z < 0 || mg.w <= 0 || mg.z + mg.w > P.num_slots) return;
  const int q_begin = P.cu_q[mg.x];
  const int queries = min(kTileQueries, P.cu_q[mg.x + 1] - q_begin - mg.y);
  const int idx = group * 256 + threadIdx.x;
  if (idx >= queries * kChunks) return;
  const int qi = idx / kChunks;
  const int c = idx - qi * kChunks;
  const float* base = P.partials + ((int64_t)mg.z * P.num_heads + h) * kPart;
  const int64_t part_stride = (int64_t)P.num_heads * kPart;
  float m = -INFINITY;
  for (int p = 0; p < mg.w; ++p) m = fmaxf(m, base[p * part_stride + kTileQueries * D + qi]);
  float lsum = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int p0 = 0; p0 < mg.w; p0 += kMaxParts) {
    float w[kMaxParts], lp[kMaxParts];
    float4 op[kMaxParts];
#pragma unroll
    for (int k = 0; k < kMaxParts; ++k) {
      if (p0 + k < mg.w) {
        const float* part = base + (p0 + k) * part_stride;
        w[k] = part[kTileQueries * D + qi];
        lp[k] = part[kTileQueries * D + kTileQueries + qi];
        op[k] = *reinterpret_cast<const float4*>(part + qi * D + 4 * c);
      }
    }
#pragma unroll
    for (int k = 0; k < kMaxParts; ++k) {
      if (p0 + k < mg.w) {
        const float wk = __builtin_amdgcn_exp2f(w[k] - m);
        lsum += wk * lp[k];
        acc.x += wk * op[k].x;
        acc.y += wk * op[k].y;
        acc.z += wk * op[k].z;
        acc.w += wk * op[k].w;
      }
    }
  }
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  Vec<bf16_t, 4> ov;
  ov.set(0, acc.x * inv);
  ov.set(1, acc.y * inv);
  ov.set(2, acc.z * inv);
  ov.set(3, acc.w * inv);
  ov.store(static_cast<bf16_t*>(P.out) + ((int64_t)(q_begin + mg.y + qi) * P.num_heads + h) * D + 4 * c);
}

template <int D>
__global__ void __launch_bounds__(256) prefill_attention_f32_kernel(PrefillParams P) {
  constexpr int kQueries = 64;              // per workgroup: half a tile, 16 per wave
  constexpr int kChunks = D / 16;           // 16-byte vectors per lane across D
  constexpr int kDTiles = D / 16;           // output tiles of 16 head-dim rows
  constexpr int kKRow = D + 4;              // padding against bank conflicts
  // V^T rows of 36 elements: the transposed stores below (8 bytes per key pair,
  // 16 pairs x 4 d-chunks per wave) then land in distinct banks.
  constexpr int kVRow = kKeys + 4;
  static_assert(D % 16 == 0, "head_dim must split into 4 lane groups of 16-byte vectors");

  __shared__ __attribute__((aligned(16))) float k_lds[2][kKeys][kKRow];
  __shared__ __attribute__((aligned(16))) float vt_lds[2][D][kVRow];
  __shared__ int page_lds[kLdsPages];

  // Two workgroups per (tile, head): blockIdx = (tile * 2 + half) * heads + head.
  const int h = blockIdx.x % P.num_heads;
  const int tile = blockIdx.x / P.num_heads / 2;
  const int sub = (blockIdx.x / P.num_heads) & 1;
  if (tile >= P.num_tiles) return;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int col = lane & 15;   // query (S^T/O^T column) or key/d row for A operands
  const int grp = lane >> 4;   // k-group

  const int seq = P.tile_seq[tile];
  if (seq < 0 || seq >= P.num_seqs) return;  // malformed tile list: nothing to write
  const TileGeometry g = tile_geometry(P, seq, P.tile_q0[tile] + sub * kQueries, h, kQueries);
  fill_page_table(P, g, page_lds);
  if (g.q0 >= g.q_len) return;  // the whole workgroup: this half of the tile is empty
  const float* k_base = static_cast<const float*>(P.k_pool) + (int64_t)P.layer * P.layer_stride;
  const float* v_base = static_cast<const float*>(P.v_pool) + (int64_t)P.layer * P.layer_stride;

  const int q_local = g.q0 + wave * 16 + col;
  const bool q_valid = q_local < g.q_len;
  const int q_pos = g.past + q_local;
  const int wave_first_pos = g.past + g.q0 + wave * 16;
  const int wave_key_end = g.past + min(g.q0 + wave * 16 + 16, g.q_len);

  // Q^T operand: lane holds query `col`, vector chunk c covers d in [16c + 4grp, +4).
  Vec<float, 4> qv[kChunks];
  {
    const float* qrow = static_cast<const float*>(P.q) +
                        ((int64_t)(g.q_begin + (q_valid ? q_local : 0)) * P.num_heads + h) * D;
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      if (q_valid) {
        qv[c].load(qrow + 16 * c + 4 * grp);
      } else {
#pragma unroll
        for (int w = 0; w < 4; ++w) qv[c].w[w] = 0u;
      }
    }
  }

  f32x4_t o[kDTiles];
#pragma unroll
  for (int j = 0; j < kDTiles; ++j) o[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;

  // Staging work: (16-byte d-chunk, key pair); a thread loads both keys of its
  // pair so it can store V^T one key pair per 8 bytes.
  constexpr int kChunksPerKey = D / 4;
  constexpr int kPairs = kKeys / 2;
  constexpr int kCombos = kChunksPerKey * kPairs;
  constexpr int kCombosPerThread = (kCombos + 255) / 256;
  Vec<float, 4> kreg[2 * kCombosPerThread], vreg[2 * kCombosPerThread];
  auto load_block = [&](int kb) {
#pragma unroll
    for (int r = 0; r < kCombosPerThread; ++r) {
      const int combo = tid + r * 256;
      const int c = combo / kPairs;
      const int pair = combo - c * kPairs;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int64_t off = combo < kCombos ? key_offset(P, g, page_lds, kb + 2 * pair + e, D) : -1;
        Vec<float, 4>& kr = kreg[2 * r + e];
        Vec<float, 4>& vr = vreg[2 * r + e];
        if (off >= 0) {
          kr.load(k_base + off + c * 4);
          vr.load(v_base + off + c * 4);
        } else {
#pragma unroll
          for (int w = 0; w < 4; ++w) kr.w[w] = vr.w[w] = 0u;
        }
      }
    }
  };
  auto store_block = [&](int buf) {
#pragma unroll
    for (int r = 0; r < kCombosPerThread; ++r) {
      const int combo = tid + r * 256;
      if (combo >= kCombos) continue;
      const int c = combo / kPairs;
      const int pair = combo - c * kPairs;
      kreg[2 * r].store(&k_lds[buf][2 * pair][c * 4]);
      kreg[2 * r + 1].store(&k_lds[buf][2 * pair + 1][c * 4]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<uint2*>(&vt_lds[buf][c * 4 + i][2 * pair]) = make_uint2(vreg[2 * r].w[i], vreg[2 * r + 1].w[i]);
    }
  };

  __syncthreads();  // page_lds
  if (g.key_end > 0) {
    load_block(0);
    store_block(0);
  }
  __syncthreads();

  int buf = 0;
  for (int kb = 0; kb < g.key_end; kb += kKeys, buf ^= 1) {
    const bool has_next = kb + kKeys < g.key_end;
    if (has_next) load_block(kb + kKeys);

    if (kb < wave_key_end) {
      // S^T for key tiles 0 (keys kb..kb+15) and 1 (kb+16..kb+31): lane holds keys 4*grp+i.
      f32x4_t st[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        st[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < kChunks; ++c) {
          Vec<float, 4> kv;
          kv.load(&k_lds[buf][t * 16 + col][16 * c + 4 * grp]);
#pragma unroll
          for (int i = 0; i < 4; ++i) st[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.get(i), qv[c].get(i), st[t], 0, 0, 0);
        }
      }
      const bool masked = kb + kKeys - 1 > wave_first_pos || kb + kKeys > g.key_end;
      float sv[2][4];
      float mloc = -INFINITY;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int kp = kb + t * 16 + grp * 4 + i;
          const float x = st[t][i] * P.scale_log2;
          sv[t][i] = !masked || (kp <= q_pos && kp < g.key_end) ? x : -INFINITY;
          mloc = fmaxf(mloc, sv[t][i]);
        }
      mloc = fmaxf(mloc, shfl_xor_f32(mloc, 16));
      mloc = fmaxf(mloc, shfl_xor_f32(mloc, 32));
      // Key 0 is visible to every query, so from the first block on m_new is
      // finite: exp2(-inf) = 0 covers the first rescale and every masked key.
      const float m_new = fmaxf(m, mloc);
      const float alpha = __builtin_amdgcn_exp2f(m - m_new);
      float psum = 0.f;
      float p[2][4];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p[t][i] = __builtin_amdgcn_exp2f(sv[t][i] - m_new);
          psum += p[t][i];
        }
      l = l * alpha + psum;
      m = m_new;
#pragma unroll
      for (int j = 0; j < kDTiles; ++j) o[j] *= alpha;
      // Per key tile t, MFMA i uses k-slice grp <-> key 16t + 4grp + i.
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int j = 0; j < kDTiles; ++j) {
          Vec<float, 4> va;
          va.load(&vt_lds[buf][j * 16 + col][16 * t + 4 * grp]);
#pragma unroll
          for (int i = 0; i < 4; ++i) o[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(va.get(i), p[t][i], o[j], 0, 0, 0);
        }
    }
    if (has_next) store_block(buf ^ 1);
    __syncthreads();
  }

  // Total row sum over the 4 key groups, normalize, store O (lane: query col, d = 16j + 4*grp + i).
  l += shfl_xor_f32(l, 16);
  l += shfl_xor_f32(l, 32);
  if (!q_valid) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  float* orow = static_cast<float*>(P.out) + ((int64_t)(g.q_begin + q_local) * P.num_heads + h) * D;
#pragma unroll
  for (int j = 0; j < kDTiles; ++j) {
    Vec<float, 4> ov;
#pragma unroll
    for (int i = 0; i < 4; ++i) ov.set(i, o[j][i] * inv);
    ov.store(orow + j * 16 + 4 * grp);
  }
}

}  // namespace cdb

using namespace cdb;

namespace {

// Shared argument checks of the two entry points; fills everything in P but the
// work lists.
int prefill_setup(PrefillParams& P, const void* q, const void* k_pool, const void* v_pool, int64_t layer_stride,
                  int32_t layer, int32_t num_cache_layers, int64_t pool_blocks, const int32_t* block_table,
                  const int32_t* table_row, int32_t table_width, const int32_t* cu_q, const int32_t* past,
                  int32_t num_seqs, void* out, int32_t num_heads, int32_t num_kv_heads, int32_t block_size,
                  float scale) {
  if (!q || !k_pool || !v_pool || !block_table || !table_row || !cu_q || !past || !out) return CDB_ERR_NULL;
  if (num_seqs <= 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads || table_width <= 0 ||
      layer < 0 || layer >= num_cache_layers || pool_blocks <= 0)
    return CDB_ERR_SHAPE;
  // The softmax takes maxima of unscaled scores: the scale must be a positive number.
  if (!(scale > 0.f) || !__builtin_isfinite(scale)) return CDB_ERR_SHAPE;
  int bs_log2 = 0;
  while ((1 << bs_log2) < block_size) ++bs_log2;
  if (block_size <= 0 || (1 << bs_log2) != block_size) return CDB_ERR_SHAPE;
  P = PrefillParams{};
  P.q = q;
  P.k_pool = k_pool;
  P.v_pool = v_pool;
  P.layer_stride = layer_stride;
  P.layer = layer;
  P.block_table = block_table;
  P.table_row = table_row;
  P.cu_q = cu_q;
  P.past = past;
  P.out = out;
  P.pool_blocks = pool_blocks;
  P.num_seqs = num_seqs;
  P.num_heads = num_heads;
  P.num_kv_heads = num_kv_heads;
  P.table_width = table_width;
  P.block_size_log2 = bs_log2;
  P.scale_log2 = scale * 1.4426950408889634f;
  return CDB_OK;
}

int launch(const void* kernel, int64_t groups, const PrefillParams& P, hipStream_t stream) {
  if (groups > 0x7fffffff) return CDB_ERR_SHAPE;
  if (groups == 0) return CDB_OK;
  void* args[] = {const_cast<PrefillParams*>(&P)};
  if (hipLaunchKernel(kernel, dim3((unsigned)groups), dim3(256), args, 0, stream) != hipSuccess) return CDB_ERR_HIP;
  return hipGetLastError() == hipSuccess ? CDB_OK : CDB_ERR_HIP;
}

template <int D> const void* bf16_kernel() { return reinterpret_cast<const void*>(&prefill_attention_bf16_kernel<D>); }
template <int D> const void* f32_kernel() { return reinterpret_cast<const void*>(&prefill_attention_f32_kernel<D>); }
template <int D> const void* merge_kernel() { return reinterpret_cast<const void*>(&prefill_merge_kernel<D>); }

}  // namespace

extern "C" {

int cdb_prefill_attention(const void* q, const void* k_pool, const void* v_pool, int64_t layer_stride, int32_t layer,
                          int32_t num_cache_layers, int64_t pool_blocks, const int32_t* block_table, const int32_t* table_row,
                          int32_t table_width, const int32_t* cu_q, const int32_t* past, int32_t num_seqs,
                          const int32_t* tile_seq, const int32_t* tile_q0, int32_t num_tiles, void* out,
                          int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale,
                          int32_t dtype, hipStream_t stream) {
  if (num_tiles == 0) return CDB_OK;
  if (!tile_seq || !tile_q0) return CDB_ERR_NULL;
  if (num_tiles < 0) return CDB_ERR_SHAPE;
  PrefillParams P;
  const int rc = prefill_setup(P, q, k_pool, v_pool, layer_stride, layer, num_cache_layers, pool_blocks, block_table,
                               table_row, table_width, cu_q, past, num_seqs, out, num_heads, num_kv_heads, block_size,
                               scale);
  if (rc != CDB_OK) return rc;
  P.tile_seq = tile_seq;
  P.tile_q0 = tile_q0;
  P.num_tiles = num_tiles;
  if (dtype == CDB_DTYPE_BF16) {
    const int64_t groups = (int64_t)num_tiles * num_heads;
    switch (head_dim) {
      case 64: return launch(bf16_kernel<64>(), groups, P, stream);
      case 96: return launch(bf16_kernel<96>(), groups, P, stream);
      case 128: return launch(bf16_kernel<128>(), groups, P, stream);
      default: return CDB_ERR_UNSUPPORTED;
    }
  }
  if (dtype == CDB_DTYPE_F32) {
    const int64_t groups = (int64_t)num_tiles * num_heads * 2;
    switch (head_dim) {
      case 64: return launch(f32_kernel<64>(), groups, P, stream);
      case 96: return launch(f32_kernel<96>(), groups, P, stream);
      case 128: return launch(f32_kernel<128>(), groups, P, stream);
      default: return CDB_ERR_UNSUPPORTED;
    }
  }
  return CDB_ERR_UNSUPPORTED;
}

int64_t cdb_prefill_partial_bytes(int32_t num_slots, int32_t num_heads, int32_t head_dim) {
  if (num_slots < 0 || num_heads <= 0 || head_dim <= 0) return -1;
  return (int64_t)num_slots * num_heads * kTileQueries * (head_dim + 2) * (int64_t)sizeof(float);
}

int cdb_prefill_attention_split(const void* q, const void* k_pool, const void* v_pool, int64_t layer_stride,
                                int32_t layer, int32_t num_cache_layers, int64_t pool_blocks,
                                const int32_t* block_table, const int32_t* table_row, int32_t table_width,
                                const int32_t* cu_q, const int32_t* past, int32_t num_seqs, const int32_t* items,
                                int32_t num_items, const int32_t* merges, int32_t num_merges, int32_t num_slots,
                                void* partials, int64_t partials_bytes, void* out, int32_t num_heads,
                                int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale,
                                int32_t dtype, hipStream_t stream) {
  if (num_items == 0) return CDB_OK;
  if (num_items < 0 || num_merges < 0 || num_slots < 0) return CDB_ERR_SHAPE;
  if (!items || (num_merges > 0 && !merges) || (num_slots > 0 && !partials)) return CDB_ERR_NULL;
  if (dtype != CDB_DTYPE_BF16 || (head_dim != 64 && head_dim != 96 && head_dim != 128)) return CDB_ERR_UNSUPPORTED;
  PrefillParams P;
  const int rc = prefill_setup(P, q, k_pool, v_pool, layer_stride, layer, num_cache_layers, pool_blocks, block_table,
                               table_row, table_width, cu_q, past, num_seqs, out, num_heads, num_kv_heads, block_size,
                               scale);
  if (rc != CDB_OK) return rc;
  if (partials_bytes < cdb_prefill_partial_bytes(num_slots, num_heads, head_dim)) return CDB_ERR_CAPACITY;
  P.items = items;
  P.num_tiles = num_items;
  P.merges = merges;
  P.num_merges = num_merges;
  P.num_slots = num_slots;
  P.partials = static_cast<float*>(partials);
  const int64_t groups = (int64_t)num_items * num_heads;
  const int64_t merge_groups = (int64_t)num_merges * num_heads * kMergeGroups;
  int code = CDB_ERR_UNSUPPORTED;
  switch (head_dim) {
    case 64:
      code = launch(bf16_kernel<64>(), groups, P, stream);
      return code == CDB_OK ? launch(merge_kernel<64>(), merge_groups, P, stream) : code;
    case 96:
      code = launch(bf16_kernel<96>(), groups, P, stream);
      return code == CDB_OK ? launch(merge_kernel<96>(), merge_groups, P, stream) : code;
    case 128:
      code = launch(bf16_kernel<128>(), groups, P, stream);
      return code == CDB_OK ? launch(merge_kernel<128>(), merge_groups, P, stream) : code;
  }
  return code;
}

}  // extern "C"
