// Mixed-depth paged decode attention with fused RoPE and KV append (CDNA4).
//
// One launch serves a recurrent-stage batch in which every row may sit at a
// different loop step: row b reads and writes the KV pages of its own cache
// layer (slot * num_layers + layer). For each row the kernel
//   1. rotates the row's new query and key (split-half or interleaved RoPE),
//   2. appends the rotated key and the value at position p_b = seqlens[b]
//      through the row's block table,
//   3. attends causally over positions 0..p_b with scale `scale`.
// This is the contract of flash_attn_with_kvcache as the reference's paged
// decode branch calls it (transformers integrations/flash_paged.py:100-147),
// with RoPE (ouro/modeling_ouro.py:179-204, huginn/modeling_huginn.py:155-196)
// folded in.
//
// Kernels on one stream:
//   * decode_plan_kernel (one workgroup) cuts every row's context into chunks
//     of a fixed number of pages and lists the chunks longest first: all full
//     chunks, then the rows' last chunks by decreasing length. Each chunk gets
//     a 64-byte descriptor and its own partial slot. The plan depends only on
//     the rows' positions, table rows and cache-layer offsets, so a caller that
//     runs the same rows through several layers plans once and attends per
//     layer (cdb_paged_decode_attention_staged).
//   * one decode kernel. A work item is (chunk, query head) and belongs to one
//     wave of a persistent grid, which takes items in the plan's order, so the
//     longest items go first and every wave ends on short ones.
//     - paged_decode_fast_kernel (16-token pages, 8-page chunks: the engine's
//       shape; more than kDeepRowsOf<D> rows): while a wave streams one item it
//       already holds the next item's descriptor and loads its query and new
//       token, and the next item's first K/V step is issued into the buffer the
//       current item's last step frees; the launch's tail goes to whichever
//       wave asks first, from its XCD's queue.
//     - paged_decode_deep_kernel (the same shape, at most kDeepRowsOf<D> rows): each
//       wave keeps three K/V steps in flight, and the wave that stores a row's
//       last chunk merges the row (arrival counters, agent-coherent partials).
//     - paged_decode_kernel: any page size and chunk length.
//   * decode_merge_kernel (after the fast and general forms) combines the
//     partials of rows with several chunks, in chunk order, and fills the
//     output of rows without work.
// A chunk's tokens, and therefore its partial, do not depend on which other
// rows share the launch, every form computes a chunk the same way, and the
// merge order is fixed: a row's output is bit-identical in any batch
// composition (unless the workspace is too small for the launch's chunks, when
// the plan lengthens them).
// Inside a wave, lane = 16 * slot + chunk: the 16 lanes of a DPP row split the
// head dimension into 16-byte chunks and the 4 slots take interleaved tokens,
// each with its own online-softmax state, merged across slots at the end. A
// wave step is 16 tokens (4 per slot).
//
// Workspace, each part 256-byte aligned: int32 header [chunk_tokens,
// chunk_prefix[0..B]], the tail queue counters (kQueues lines of 128 bytes),
// one int32 arrival counter per (row, head); then int32 descriptors
// [capacity][16], then fp32 partials [capacity, H, D + 2] (unnormalized
// accumulator, running max, running sum).

#include <algorithm>
#include <mutex>
#include <utility>
#include <vector>

#include "cdb_common.h"
#include "../../include/cdb_amd.h"

namespace cdb {

constexpr int kMaxRowsLds = 2048;
// Descriptor words: b | last flag, t_begin, t_end, p, partial slot, chunks in row, trow, layer,
// then the block ids of the chunk's first kChunkPagesFast pages (-1 past the table).
constexpr int kDescInts = 16;
constexpr int kChunkPagesFast = 8;
constexpr int kDescBytes = kDescInts * 4;
constexpr int kLastChunk = 1 << 30;    // flag in descriptor word 0
constexpr int kPlanThreads = 1024;
constexpr int kLengthKeys = 64;        // last chunks are ordered by ceil(tokens / 32), capped here
constexpr int kQueues = 8;             // one item queue per XCD (workgroups are dealt to XCDs round-robin)
constexpr int kCounterStride = 32;     // ints between queue counters: one 128-byte line each

struct DecodeParams {
  const void* q;            // [B, H, D], rows q_stride elements apart
  const void* k_new;        // [B, Hkv, D], rows kv_stride elements apart
  const void* v_new;        // [B, Hkv, D], rows kv_stride elements apart
  void* k_pool;             // cache layer l keys at k_pool + l * layer_stride, rows x [Hkv, D]
  void* v_pool;
  const int32_t* block_table;   // [num_table_rows, table_width]
  const int32_t* table_row;     // [B] or null (row b uses table row b)
  const int32_t* seqlens;       // [B]: position of the new token; < 0 marks a padding row
  const int32_t* cache_layer;   // [B] per-row offset added to cache_layer0, or null
  const float* rope_cos;        // [max_positions, D/2] or null
  const float* rope_sin;
  const void* q_bias;           // [H, D] or null, added to q before rotation
  const void* k_bias;           // [Hkv, D] or null
  void* out;                    // [B, H, D]
  int32_t* header;              // [B + 2]: chunk tokens, then the chunk prefix over rows
  int32_t* counters;            // [kQueues * kCounterStride]: per-XCD item queues of the fast form
  int32_t* arrivals;            // [B * H]: chunks of each (row, head) finished in the current deep-form call
  int32_t* desc;                // [capacity][kDescInts]
  float* partial;               // [capacity, H, D + 2]
  int64_t layer_stride;         // elements between cache layers
  int64_t q_stride, kv_stride;  // elements between consecutive rows of q and of k_new/v_new
  int32_t cache_layer0;
  int32_t num_rows, num_heads, num_kv_heads;
  int32_t table_width, block_size_log2, chunk_pages;
  int32_t rope_style;           // 0 none, 1 split-half, 2 interleaved pairs
  int32_t max_positions;
  int32_t num_cache_layers;     // valid cache layers are [0, num_cache_layers)
  int64_t pool_blocks;          // valid block ids are [0, pool_blocks)
  int64_t capacity;             // chunks the workspace holds (descriptors and partials)
  float scale_log2;             // softmax scale * log2(e)
};

template <int D> struct Layout {
  static constexpr int kChunk = D / 16;  // elements per lane
  static_assert(D % 16 == 0, "head_dim must be a multiple of 16");
};

// A row gets chunks when its new-token position fits the block table and the
// RoPE table; its cache layer is checked per call (it depends on cache_layer0).
CDB_DEVICE bool position_in_range(const DecodeParams& P, int p) {
  if (p < 0) return false;
  if ((int64_t)p >= ((int64_t)P.table_width << P.block_size_log2)) return false;
  return P.rope_cos == nullptr || p < P.max_positions;
}

CDB_DEVICE bool layer_in_range(const DecodeParams& P, int layer_offset) {
  const int layer = P.cache_layer0 + layer_offset;
  return layer >= 0 && layer < P.num_cache_layers;
}

// ---------------------------------------------------------------------------
// Plan
// ---------------------------------------------------------------------------

// Sum of v over the workgroup, returned to every thread.
template <int NT>
CDB_DEVICE int64_t block_sum(int64_t v, int64_t* scratch) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  int64_t total = 0;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) total += scratch[w];
  __syncthreads();
  return total;
}

// In-place exclusive prefix of two count arrays at once: on entry a[b + 1] and
// c[b + 1] hold row b's counts (a[0] = c[0] = 0); on exit they hold the sums
// over rows before b + 1. Each thread owns a contiguous run of rows; a
// wave-level scan of the run totals and the wave totals in LDS give every run
// its offset.
template <int NT>
CDB_DEVICE void block_prefix2(int* a, int* c, int B, int* wave_tot) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int kWaves = NT / 64;
  const int per = (B + NT - 1) / NT;
  const int lo = min(tid * per, B), hi = min(lo + per, B);
  int sa = 0, sc = 0;
  for (int b = lo; b < hi; ++b) {
    sa += a[b + 1];
    sc += c[b + 1];
  }
  int ia = sa, ic = sc;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int na = __shfl_up(ia, off, 64), nc = __shfl_up(ic, off, 64);
    if (lane >= off) {
      ia += na;
      ic += nc;
    }
  }
  if (lane == 63) {
    wave_tot[wave] = ia;
    wave_tot[kWaves + wave] = ic;
  }
  __syncthreads();
  int ra = ia - sa, rc = ic - sc;
  for (int w = 0; w < wave; ++w) {
    ra += wave_tot[w];
    rc += wave_tot[kWaves + w];
  }
  for (int b = lo; b < hi; ++b) {
    ra += a[b + 1];
    rc += c[b + 1];
    a[b + 1] = ra;
    c[b + 1] = rc;
  }
  __syncthreads();
}

CDB_DEVICE int length_key(int tokens) { return min((tokens + 31) >> 5, kLengthKeys - 1); }

__global__ void __launch_bounds__(kPlanThreads) decode_plan_kernel(DecodeParams P) {
  __shared__ int row_pos[kMaxRowsLds];           // position, or -1 for a row without chunks
  __shared__ int row_trow[kMaxRowsLds];          // block-table row
  __shared__ int row_layer[kMaxRowsLds];         // cache-layer offset
  __shared__ int chunk_prefix[kMaxRowsLds + 1];  // chunks of rows before b (partial slots)
  __shared__ int full_prefix[kMaxRowsLds + 1];   // full chunks of rows before b
  __shared__ int key_next[kLengthKeys];          // next free descriptor of each last-chunk length
  __shared__ int wave_tot[2 * (kPlanThreads / 64)];
  __shared__ int64_t sum_scratch[kPlanThreads / 64];

  const int tid = threadIdx.x;
  const int B = P.num_rows;
  for (int b = tid; b < B; b += kPlanThreads) {
    const int p = P.seqlens[b];
    const int trow = P.table_row ? P.table_row[b] : b;
    row_pos[b] = position_in_range(P, p) && trow >= 0 ? p : -1;
    row_trow[b] = trow;
    row_layer[b] = P.cache_layer ? P.cache_layer[b] : 0;
  }
  if (tid < kLengthKeys) key_next[tid] = 0;
  __syncthreads();

  // Chunks of chunk_pages pages; lengthened only when the workspace cannot hold them (one chunk
  // per row always fits: the host checks capacity >= B).
  int64_t ct = (int64_t)P.chunk_pages << P.block_size_log2;
  for (;;) {
    int64_t n = 0;
    for (int b = tid; b < B; b += kPlanThreads) n += row_pos[b] >= 0 ? (row_pos[b] + ct) / ct : 0;
    if (block_sum<kPlanThreads>(n, sum_scratch) <= P.capacity || ct >= (1 << 29)) break;
    ct <<= 1;
  }
  const int chunk_tokens = (int)ct;

  for (int b = tid; b < B; b += kPlanThreads) {
    const int p = row_pos[b];
    const int n = p >= 0 ? (p + chunk_tokens) / chunk_tokens : 0;
    chunk_prefix[b + 1] = n;
    full_prefix[b + 1] = n > 0 ? n - 1 : 0;
    if (n > 0) atomicAdd(&key_next[length_key(p + 1 - (n - 1) * chunk_tokens)], 1);
  }
  if (tid == 0) chunk_prefix[0] = full_prefix[0] = 0;
  __syncthreads();
  block_prefix2<kPlanThreads>(chunk_prefix, full_prefix, B, wave_tot);
  if (tid == 0) {
    // Last chunks follow the full ones, longest first.
    int at = full_prefix[B];
    for (int k = kLengthKeys - 1; k >= 0; --k) {
      const int count = key_next[k];
      key_next[k] = at;
      at += count;
    }
  }
  __syncthreads();

  for (int b = tid; b <= B; b += kPlanThreads) P.header[1 + b] = chunk_prefix[b];
  if (tid == 0) P.header[0] = chunk_tokens;
  if (tid < kQueues) P.counters[tid * kCounterStride] = 0;
  for (int i = tid; i < B * P.num_heads; i += kPlanThreads) P.arrivals[i] = 0;
  // One thread per chunk (in partial-slot order): a long row's descriptors are written in parallel.
  const int total_chunks = chunk_prefix[B];
  for (int ci = tid; ci < total_chunks; ci += kPlanThreads) {
    int lo = 0, hi = B - 1;  // the row owning chunk ci: the largest b with chunk_prefix[b] <= ci
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (chunk_prefix[mid] <= ci) lo = mid; else hi = mid - 1;
    }
    const int b = lo;
    const int p = row_pos[b];
    const int n = chunk_prefix[b + 1] - chunk_prefix[b];
    const int trow = row_trow[b];
    const int layer = row_layer[b];
    {
      const int c = ci - chunk_prefix[b];
      const bool last = c == n - 1;
      const int t_begin = c * chunk_tokens;
      const int at = last ? atomicAdd(&key_next[length_key(p + 1 - t_begin)], 1) : full_prefix[b] + c;
      if (at >= P.capacity) continue;  // only when positions near 2^29 outgrow even the longest chunks
      int4* d = reinterpret_cast<int4*>(P.desc + (int64_t)at * kDescInts);
      d[0] = make_int4(b | (last ? kLastChunk : 0), t_begin, last ? p : t_begin + chunk_tokens, p);
      d[1] = make_int4(chunk_prefix[b] + c, n, trow, layer);
      const int32_t* row_table = P.block_table + (int64_t)trow * P.table_width;
      const int page0 = t_begin >> P.block_size_log2;
      int ids[kChunkPagesFast];
#pragma unroll
      for (int j = 0; j < kChunkPagesFast; ++j) ids[j] = page0 + j < P.table_width ? row_table[page0 + j] : -1;
      d[2] = make_int4(ids[0], ids[1], ids[2], ids[3]);
      d[3] = make_int4(ids[4], ids[5], ids[6], ids[7]);
    }
  }
}

// ---------------------------------------------------------------------------
// Decode
// ---------------------------------------------------------------------------

// One work item: a chunk of one row for one query head. Pointers are derived
// at use so that two items (the current and the next) stay cheap to hold.
struct Item {
  int b, h, t_begin, t_end, p, partial, trow, layer;
  int nsplit;               // chunks of the row (0 for a descriptor no plan could have written)
  bool last, single, live;  // live: the row's cache layer exists in this call
};

// The descriptor and header words are read-only while the decode kernel runs
// and their addresses are wave-uniform: they are read through the constant
// address space, i.e. with scalar loads into SGPRs.
typedef int int4_v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(4))) const int4_v const_int4_v;
typedef __attribute__((address_space(4))) const int32_t const_int32;

struct RawDesc {
  int4_v a, b;
};

CDB_DEVICE RawDesc load_desc(const DecodeParams& P, int ci) {
  const const_int4_v* d = (const const_int4_v*)(P.desc + (int64_t)ci * kDescInts);
  return RawDesc{d[0], d[1]};
}

CDB_DEVICE int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

CDB_DEVICE Item make_item(const DecodeParams& P, const RawDesc& r, int h) {
  Item it;
  const int w0 = r.a.x;
  it.b = w0 & (kLastChunk - 1);
  it.last = (w0 & kLastChunk) != 0;
  it.t_begin = r.a.y;
  it.p = r.a.w;
  it.partial = r.b.x;
  const int nsplit = r.b.y;
  it.nsplit = nsplit;
  it.single = nsplit == 1;
  it.h = h;
  const int layer_offset = r.b.w;
  const int t_end = r.a.z;
  it.trow = r.b.z;
  // A descriptor that no plan of these rows could have written reads row 0 and
  // writes nothing; a row whose cache layer does not exist reads no KV, appends
  // nothing and gets a NaN output.
  const bool sane = it.b < P.num_rows && it.trow >= 0 && it.t_begin >= 0 && it.t_begin <= t_end &&
                    t_end <= it.p && position_in_range(P, it.p) && nsplit > 0 && it.partial >= 0 &&
                    it.partial < P.capacity;
  it.live = sane && layer_in_range(P, layer_offset);
  if (!sane) {
    it.b = it.p = it.partial = it.nsplit = 0;
    it.single = it.last = false;
  }
  it.t_end = it.live ? t_end : it.t_begin;
  it.layer = it.live ? P.cache_layer0 + layer_offset : 0;
  if (!it.live) it.trow = 0;
  return it;
}

template <typename T>
CDB_DEVICE T* pool_layer(void* pool, const DecodeParams& P, const Item& it) {
  return static_cast<T*>(pool) + (int64_t)it.layer * P.layer_stride;
}

CDB_DEVICE const int32_t* table_of(const DecodeParams& P, const Item& it) {
  return P.block_table + (int64_t)it.trow * P.table_width;
}

// RoPE angles of this lane's chunk at one position, loaded ahead of the
// rotation: split-half style uses C consecutive entries, interleaved style C/2.
template <int D>
struct Angles {
  Vec<float, D / 16> c, s;
};

template <int D, int R>
CDB_DEVICE void load_angles(const DecodeParams& P, int pos, int chunk, Angles<D>& a) {
  constexpr int C = Layout<D>::kChunk;
  if constexpr (R == 0) return;
  const int half = D / 2;
  const float* cos_row = P.rope_cos + (int64_t)pos * half;
  const float* sin_row = P.rope_sin + (int64_t)pos * half;
  if constexpr (R == 1) {
    const int f0 = (chunk * C) % half;
    a.c.load(cos_row + f0);
    a.s.load(sin_row + f0);
  } else {
    Vec<float, C / 2> c, s;
    c.load(cos_row + chunk * C / 2);
    s.load(sin_row + chunk * C / 2);
#pragma unroll
    for (int i = 0; i < C / 2; ++i) {
      a.c.w[i] = c.w[i];
      a.s.w[i] = s.w[i];
    }
  }
}

// Rotate this lane's chunk of a head vector. `own`/`partner` are the lane's
// chunk and (for split-half) the chunk D/2 away; values are returned rounded to
// the storage type the way the reference's torch ops round them.
template <typename T, int D, int R>
CDB_DEVICE void rope_chunk(const Angles<D>& ang, int chunk, const float* own, const float* partner, float* out) {
  constexpr int C = Layout<D>::kChunk;
  if constexpr (R == 0) {
#pragma unroll
    for (int i = 0; i < C; ++i) out[i] = own[i];
    return;
  } else if constexpr (R == 1) {
    // q*cos + rotate_half(q)*sin with cos/sin = cat(f, f); each op rounded. A
    // chunk lies inside one half, so its angles are C consecutive table entries.
    const bool first_half = chunk * C < D / 2;
#pragma unroll
    for (int i = 0; i < C; ++i) {
      const float rot = first_half ? -partner[i] : partner[i];
      const float a = Elem<T>::round(mul_rn(own[i], __uint_as_float(ang.c.w[i])));
      const float b = Elem<T>::round(mul_rn(rot, __uint_as_float(ang.s.w[i])));
      out[i] = Elem<T>::round(add_rn(a, b));
    }
  } else {
    // Interleaved (even, odd) pairs rotated in fp32, rounded once at the end.
#pragma unroll
    for (int i = 0; i < C; i += 2) {
      const float c = __uint_as_float(ang.c.w[i / 2]), s = __uint_as_float(ang.s.w[i / 2]);
      const float x0 = own[i], x1 = own[i + 1];
      out[i] = Elem<T>::round(sub_rn(mul_rn(x0, c), mul_rn(x1, s)));
      out[i + 1] = Elem<T>::round(add_rn(mul_rn(x1, c), mul_rn(x0, s)));
    }
  }
}

// This lane's chunk of one head vector as loaded (rotation happens later so the
// loads can be issued early).
template <typename T, int D>
struct RawChunk {
  Vec<T, D / 16> own;
};

template <typename T, int D, int R>
CDB_DEVICE void load_raw(const T* base, int chunk, RawChunk<T, D>& r) {
  r.own.load(base + chunk * Layout<D>::kChunk);
}

// Add an optional per-head bias to a loaded chunk and rotate it. Split-half
// rotation pairs chunk c with chunk c ^ 8, which is the lane 8 places along the
// same 16-lane DPP row: the partner values come from a row rotate by 8.
template <typename T, int D, int R>
CDB_DEVICE void rotate_raw(const RawChunk<T, D>& r, const Angles<D>& ang, const T* bias, int chunk, float* out) {
  constexpr int C = Layout<D>::kChunk;
  float own[C], partner[C];
#pragma unroll
  for (int i = 0; i < C; ++i) own[i] = r.own.get(i);
  if (bias != nullptr) {
    Vec<T, C> bv;
    bv.load(bias + chunk * C);
#pragma unroll
    for (int i = 0; i < C; ++i) own[i] = Elem<T>::round(add_rn(own[i], bv.get(i)));
  }
  if constexpr (R == 1) {
#pragma unroll
    for (int i = 0; i < C; ++i) partner[i] = dpp_f32<kRowRor8>(own[i]);
  }
  rope_chunk<T, D, R>(ang, chunk, own, partner, out);
}

// The block ids of 64 consecutive pages starting at `base`, one per lane
// (-1 past the table's width). Loaded once per 64 pages so that K/V addresses
// never wait on a block-table load inside the streaming loop.
CDB_DEVICE int load_page_window(const int32_t* table, int base, int table_width, int lane) {
  const int page = base + lane;
  return page < table_width ? table[page] : -1;
}

// Block id of `page` from the window (`page - base` must be in [0, 64)).
CDB_DEVICE int window_block(int window, int base, int page) {
  return __builtin_amdgcn_ds_bpermute((page - base) << 2, window);
}

// Load one wave step (16 tokens: 4 per slot) of K and V for this lane's chunk.
// t0 is a multiple of 16 and the step's pages lie in the window. Tokens at or
// past t_end, or with an out-of-range block id, are masked: they load the
// layer's first row instead (always a valid address) and attend_step gives
// them zero weight and zero values. The loads are unconditional: a branch that
// zeroes the registers of a masked token would have to wait for every load in
// flight before writing them.
template <typename T, int D>
CDB_DEVICE void load_step(const DecodeParams& P, int window, int win_base, const T* k_base, const T* v_base,
                          int t0, int t_end, int slot, int chunk, int kvh, int bs_log2, int64_t row_elems,
                          Vec<T, D / 16> (&kv)[4], Vec<T, D / 16> (&vv)[4], bool (&valid)[4]) {
  constexpr int C = D / 16;
  // With pages of >= 16 tokens the whole step sits in one page: one wave-uniform lookup.
  const bool one_page = bs_log2 >= 4;
  const int step_blk = one_page ? __builtin_amdgcn_readlane(window, (t0 >> bs_log2) - win_base) : -1;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int t = t0 + 4 * u + slot;
    const int blk_any = one_page ? step_blk : window_block(window, win_base, t >> bs_log2);
    const int blk = t < t_end ? blk_any : -1;
    valid[u] = blk >= 0 && blk < P.pool_blocks;
    const int64_t row = valid[u] ? ((int64_t)blk << bs_log2) + (t & ((1 << bs_log2) - 1)) : 0;
    const int64_t off = row * row_elems + (int64_t)kvh * D + chunk * C;
    kv[u].load(k_base + off);
    vv[u].load(v_base + off);
  }
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// a.x * b.x + a.y * b.y + c over packed bf16 pairs, fp32 accumulate (v_dot2c_f32_bf16).
CDB_DEVICE float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c,
                                         false);
}

// The query in the form the step loop consumes: for bf16 pools the rotated
// query's bf16 pairs (exact: RoPE output is rounded to bf16) with the scale
// applied to each score; for fp32 pools fp32 pre-scaled by scale*log2(e).
template <typename T, int D>
struct QueryReg {
  static constexpr bool kBf16 = sizeof(T) == 2;
  float f[kBf16 ? 1 : D / 16];
  uint32_t p[kBf16 ? D / 32 : 1];
};

template <typename T, int D>
CDB_DEVICE void make_query(const DecodeParams& P, const float* rotated, QueryReg<T, D>& q) {
  constexpr int C = D / 16;
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int w = 0; w < C / 2; ++w) q.p[w] = pack_bf16x2(rotated[2 * w], rotated[2 * w + 1]);
  } else {
#pragma unroll
    for (int i = 0; i < C; ++i) q.f[i] = rotated[i] * P.scale_log2;
  }
}

// Score of one key chunk (this lane's part, summed over the DPP row), in log2 units.
template <typename T, int D>
CDB_DEVICE float score(const QueryReg<T, D>& q, float scale_log2, const Vec<T, D / 16>& k) {
  constexpr int C = D / 16;
  float dot = 0.f;
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int w = 0; w < C / 2; ++w) dot = dot2_bf16(q.p[w], k.w[w], dot);
    return row16_sum(dot) * scale_log2;
  } else {
#pragma unroll
    for (int i = 0; i < C; ++i) dot = fmaf(q.f[i], k.get(i), dot);
    return row16_sum(dot);
  }
}

// Online-softmax update of one slot's state with its 4 tokens of a wave step.
// bf16: P.V pairs two tokens' probabilities, rounded to bf16 as flash-attention
// feeds P to its PV product, against the two tokens' values interleaved with
// v_perm.
template <typename T, int D>
CDB_DEVICE void attend_step(const QueryReg<T, D>& q, float scale_log2, const Vec<T, D / 16> (&kv)[4],
                            Vec<T, D / 16> (&vv)[4], const bool (&valid)[4], float& m, float& l, float* acc) {
  constexpr int C = D / 16;
  constexpr bool kBf16 = sizeof(T) == 2;
  float sc[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const float dot = score<T, D>(q, scale_log2, kv[u]);
    sc[u] = valid[u] ? dot : -INFINITY;
  }
  const float m_new = fmaxf(m, fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])));
  if (m_new == -INFINITY) return;
  // A masked token's value words are zeroed (in place: the buffer is consumed
  // here), so its zero weight never meets a NaN.
#pragma unroll
  for (int u = 0; u < 4; ++u) {
#pragma unroll
    for (int w = 0; w < Vec<T, C>::kWords; ++w) vv[u].w[w] = valid[u] ? vv[u].w[w] : 0u;
  }
  const float alpha = exp2f(m - m_new);
  l *= alpha;
#pragma unroll
  for (int i = 0; i < C; ++i) acc[i] *= alpha;
  if constexpr (kBf16) {
#pragma unroll
    for (int u = 0; u < 4; u += 2) {
      const float p0 = exp2f(sc[u] - m_new), p1 = exp2f(sc[u + 1] - m_new);
      l += p0 + p1;
      const uint32_t pk = pack_bf16x2(p0, p1);
#pragma unroll
      for (int w = 0; w < C / 2; ++w) {
        const uint32_t a = vv[u].w[w], b = vv[u + 1].w[w];
        acc[2 * w] = dot2_bf16(pk, __builtin_amdgcn_perm(b, a, 0x05040100u), acc[2 * w]);       // (a.lo, b.lo)
        acc[2 * w + 1] = dot2_bf16(pk, __builtin_amdgcn_perm(b, a, 0x07060302u), acc[2 * w + 1]);  // (a.hi, b.hi)
      }
    }
  } else {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float pu = exp2f(sc[u] - m_new);
      l += pu;
#pragma unroll
      for (int i = 0; i < C; ++i) acc[i] = fmaf(pu, __uint_as_float(vv[u].w[i]), acc[i]);
    }
  }
  m = m_new;
}

// An item's query and new-token key/value as loaded ahead of use. The RoPE
// angles of the item's position (shared by the query and the key) are read
// when the item is rotated: they come from a small table that stays in L2.
template <typename T, int D>
struct Pending {
  RawChunk<T, D> q, k;
  Vec<T, D / 16> v;
};

// Rotated new keys and new values of a wave's items wait in LDS from the item
// before until the item's end: two slots per wave (current item, next item), each
// [2][words][64 lanes], so they hold no registers while the K/V stream runs.
template <typename T, int D>
struct Stash {
  static constexpr int kWords = Vec<T, D / 16>::kWords;
  static constexpr int kPerSlot = 2 * kWords * 64;
  static constexpr int kPerWorkgroup = 2 * 4 * kPerSlot;
};

template <typename T, int D>
CDB_DEVICE uint32_t* stash_slot(uint32_t* stash, int parity, int wave) {
  return stash + (parity * 4 + wave) * Stash<T, D>::kPerSlot;
}

template <typename T, int D>
CDB_DEVICE void stash_put(uint32_t* slot, int which, const Vec<T, D / 16>& v, int lane) {
#pragma unroll
  for (int w = 0; w < Stash<T, D>::kWords; ++w) slot[(which * Stash<T, D>::kWords + w) * 64 + lane] = v.w[w];
}

template <typename T, int D>
CDB_DEVICE void stash_get(const uint32_t* slot, int which, Vec<T, D / 16>& v, int lane) {
#pragma unroll
  for (int w = 0; w < Stash<T, D>::kWords; ++w) v.w[w] = slot[(which * Stash<T, D>::kWords + w) * 64 + lane];
}

template <typename T, int D, int R>
CDB_DEVICE void issue_pending(const DecodeParams& P, const Item& it, int chunk, Pending<T, D>& pend) {
  constexpr int C = D / 16;
  const int kvh = it.h / (P.num_heads / P.num_kv_heads);
  load_raw<T, D, R>(static_cast<const T*>(P.q) + (int64_t)it.b * P.q_stride + (int64_t)it.h * D, chunk, pend.q);
  if (it.last && it.live) {
    const int64_t off = (int64_t)it.b * P.kv_stride + (int64_t)kvh * D;
    load_raw<T, D, R>(static_cast<const T*>(P.k_new) + off, chunk, pend.k);
    pend.v.load(static_cast<const T*>(P.v_new) + off + chunk * C);
  }
}

// Rotates an item's query into q and, for a row's last chunk, its new key into
// the stash slot (with the new value beside it).
template <typename T, int D, int R>
CDB_DEVICE void finish_pending(const DecodeParams& P, const Item& it, int chunk, int lane, const Pending<T, D>& pend,
                               QueryReg<T, D>& q, uint32_t* slot) {
  constexpr int C = D / 16;
  const T* q_bias = static_cast<const T*>(P.q_bias);
  const T* k_bias = static_cast<const T*>(P.k_bias);
  Angles<D> ang;
  load_angles<D, R>(P, it.p, chunk, ang);
  float rot[C];
  rotate_raw<T, D, R>(pend.q, ang, q_bias ? q_bias + (int64_t)it.h * D : nullptr, chunk, rot);
  make_query<T, D>(P, rot, q);
  if (it.last && it.live) {
    const int kvh = it.h / (P.num_heads / P.num_kv_heads);
    rotate_raw<T, D, R>(pend.k, ang, k_bias ? k_bias + (int64_t)kvh * D : nullptr, chunk, rot);
    Vec<T, C> k;
#pragma unroll
    for (int i = 0; i < C; i += 2) k.set_pair(i, rot[i], rot[i + 1]);
    stash_put<T, D>(slot, 0, k, lane);
    stash_put<T, D>(slot, 1, pend.v, lane);
  }
}

// The general form: any page size and chunk length (block ids through a 64-page
// window of the block table, reloaded as a long chunk streams past it).
template <typename T, int D, int R>
__global__ void __launch_bounds__(256, 3) paged_decode_kernel(DecodeParams P) {
  constexpr int C = Layout<D>::kChunk;
  const int lane = threadIdx.x & 63;
  const int slot = lane >> 4;
  const int chunk = lane & 15;
  const int H = P.num_heads;
  const int nwaves = gridDim.x * 4;
  const int bs_log2 = P.block_size_log2;
  const int kv_group = H / P.num_kv_heads;
  const int64_t row_elems = (int64_t)P.num_kv_heads * D;  // one cached token, all kv heads
  const int wave = threadIdx.x >> 6;
  __shared__ uint32_t stash[Stash<T, D>::kPerWorkgroup];
  int parity = 0;

  // Descriptor slots past the plan's chunks hold stale words; they are read
  // (inside the workspace) but never used.
  const int64_t cap_items = P.capacity * H;
  int item = uniform(blockIdx.x * 4 + wave);
  const auto desc_of = [&](int it) { return load_desc(P, it < cap_items ? it / H : 0); };
  RawDesc d_next = desc_of(item);
  const int chunks = *(const const_int32*)(P.header + 1 + P.num_rows);
  const int n_items = (int)min((int64_t)chunks, P.capacity) * H;
  if (item >= n_items) return;

  // The first item's window, first K/V step, query and new token are loaded
  // here; every later item's are prefetched during the item before it.
  Item cur = make_item(P, d_next, item % H);
  d_next = desc_of(item + nwaves);
  int win_base = cur.t_begin >> bs_log2;
  int window = load_page_window(table_of(P, cur), win_base, P.table_width, lane);
  Vec<T, C> ka[4], va[4], kb[4], vb[4];
  bool vla[4], vlb[4];
  load_step<T, D>(P, window, win_base, pool_layer<T>(P.k_pool, P, cur), pool_layer<T>(P.v_pool, P, cur),
                  cur.t_begin, cur.t_end, slot, chunk, cur.h / kv_group, bs_log2, row_elems, ka, va, vla);
  QueryReg<T, D> q;
  {
    Pending<T, D> pend;
    issue_pending<T, D, R>(P, cur, chunk, pend);
    finish_pending<T, D, R>(P, cur, chunk, lane, pend, q, stash_slot<T, D>(stash, parity, wave));
  }

  for (;;) {
    const int next = item + nwaves;
    const bool has_next = next < n_items;
    const int kvh = cur.h / kv_group;
    T* const k_base = pool_layer<T>(P.k_pool, P, cur);
    T* const v_base = pool_layer<T>(P.v_pool, P, cur);
    const int32_t* const table = table_of(P, cur);

    // The next item: its descriptor arrived during this item's predecessor; its
    // window, query and new token are requested now, and the descriptor after
    // it too.
    const Item nxt = make_item(P, d_next, next % H);
    d_next = desc_of(next + nwaves);
    const int nwin_base = nxt.t_begin >> bs_log2;
    const int nwindow = has_next ? load_page_window(table_of(P, nxt), nwin_base, P.table_width, lane) : -1;
    Pending<T, D> pend;
    if (has_next) issue_pending<T, D, R>(P, nxt, chunk, pend);

    float m = -INFINITY, l = 0.f;
    float acc[C];
#pragma unroll
    for (int i = 0; i < C; ++i) acc[i] = 0.f;

    // Keeps the pages of the step starting at t0 inside the current window (wave-uniform).
    auto cover = [&](int t0) {
      if (((t0 + 15) >> bs_log2) - win_base >= 64) {
        win_base = t0 >> bs_log2;
        window = load_page_window(table, win_base, P.table_width, lane);
      }
    };
    auto prefetch_next_first = [&]() {
      if (has_next)
        load_step<T, D>(P, nwindow, nwin_base, pool_layer<T>(P.k_pool, P, nxt), pool_layer<T>(P.v_pool, P, nxt),
                        nxt.t_begin, nxt.t_end, slot, chunk, nxt.h / kv_group, bs_log2, row_elems, ka, va, vla);
    };
    // One pair of wave steps: the step in buffer a (already loaded) and the one
    // after it in buffer b. The step after the pair goes into a, or, after the
    // item's last pair, the next item's first step. Returns whether the item
    // continues.
    auto pair = [&](int t0) {
      const bool second = t0 + 16 < cur.t_end;
      if (second) {
        cover(t0 + 16);
        load_step<T, D>(P, window, win_base, k_base, v_base, t0 + 16, cur.t_end, slot, chunk, kvh, bs_log2,
                        row_elems, kb, vb, vlb);
      }
      attend_step<T, D>(q, P.scale_log2, ka, va, vla, m, l, acc);
      const bool more = t0 + 32 < cur.t_end;
      if (more) {
        cover(t0 + 32);
        load_step<T, D>(P, window, win_base, k_base, v_base, t0 + 32, cur.t_end, slot, chunk, kvh, bs_log2,
                        row_elems, ka, va, vla);
      } else {
        prefetch_next_first();
      }
      if (second) attend_step<T, D>(q, P.scale_log2, kb, vb, vlb, m, l, acc);
      return more;
    };

    // The next item's query and new key are rotated after this item's first
    // pair, by when their loads have arrived; only their rotated forms stay live.
    QueryReg<T, D> qn;
    uint32_t* const next_slot = stash_slot<T, D>(stash, parity ^ 1, wave);
    if (cur.t_begin < cur.t_end) {
      int t0 = cur.t_begin;
      bool more = pair(t0);
      if (has_next) finish_pending<T, D, R>(P, nxt, chunk, lane, pend, qn, next_slot);
      while (more) {
        t0 += 32;
        more = pair(t0);
      }
    } else {
      prefetch_next_first();
      if (has_next) finish_pending<T, D, R>(P, nxt, chunk, lane, pend, qn, next_slot);
    }

    if (cur.last && cur.live) {
      // The new token: append its rotated key and its value, then attend to it from registers.
      const int p = cur.p;
      const int p_page = p >> bs_log2;
      const int new_blk = p_page - win_base >= 0 && p_page - win_base < 64
                              ? __builtin_amdgcn_readlane(window, p_page - win_base)
                              : table[p_page];
      Vec<T, C> kn, vn;
      const uint32_t* cur_slot = stash_slot<T, D>(stash, parity, wave);
      stash_get<T, D>(cur_slot, 0, kn, lane);
      stash_get<T, D>(cur_slot, 1, vn, lane);
      if (slot == 0 && cur.h % kv_group == 0 && new_blk >= 0 && new_blk < P.pool_blocks) {
        const int64_t row = ((int64_t)new_blk << bs_log2) + (p & ((1 << bs_log2) - 1));
        const int64_t off = row * row_elems + (int64_t)kvh * D + chunk * C;
        kn.store(k_base + off);
        vn.store(v_base + off);
      }
      const float dot = score<T, D>(q, P.scale_log2, kn);
      if (slot == 0) {
        const float m_new = fmaxf(m, dot);
        const float alpha = exp2f(m - m_new);
        const float pn = exp2f(dot - m_new);
        l = l * alpha + pn;
#pragma unroll
        for (int i = 0; i < C; ++i) acc[i] = fmaf(pn, vn.get(i), acc[i] * alpha);
        m = m_new;
      }
    }

    // Merge the four slots of the wave (lanes 16 apart hold the same chunk).
    float m_all = fmaxf(m, shfl_xor_f32(m, 16));
    m_all = fmaxf(m_all, shfl_xor_f32(m_all, 32));
    const float f = (m == -INFINITY) ? 0.f : exp2f(m - m_all);
    l *= f;
#pragma unroll
    for (int i = 0; i < C; ++i) acc[i] *= f;
    l += shfl_xor_f32(l, 16);
    l += shfl_xor_f32(l, 32);
#pragma unroll
    for (int i = 0; i < C; ++i) {
      acc[i] += shfl_xor_f32(acc[i], 16);
      acc[i] += shfl_xor_f32(acc[i], 32);
    }

    if (slot == 0) {
      if (cur.single) {
        // A single-chunk row stores its normalized output (NaN when its cache layer is missing).
        T* out_row = static_cast<T*>(P.out) + ((int64_t)cur.b * H + cur.h) * D;
        const float inv = cur.live ? 1.f / l : __builtin_nanf("");
        Vec<T, C> o;
#pragma unroll
        for (int i = 0; i < C; i += 2) o.set_pair(i, acc[i] * inv, acc[i + 1] * inv);
        o.store(out_row + chunk * C);
      } else if (cur.live) {
        float* part = P.partial + ((int64_t)cur.partial * H + cur.h) * (D + 2);
#pragma unroll
        for (int i = 0; i < C; ++i) part[chunk * C + i] = acc[i];
        if (chunk == 0) {
          part[D] = m_all;
          part[D + 1] = l;
        }
      }
    }

    if (!has_next) break;
    item = next;
    cur = nxt;
    window = nwindow;
    win_base = nwin_base;
    q = qn;
    parity ^= 1;
  }
}

// ---------------------------------------------------------------------------
// Fast form: pages of 16 tokens and chunks of kChunkPagesFast pages (128 tokens,
// 8 wave steps). A chunk's block ids come with its descriptor, in SGPRs, so the
// stream needs no block-table window; the 4 step pairs are unrolled and every
// path through a pair issues the same 16 loads, so each wait leaves exactly the
// other buffer's loads in flight.
// ---------------------------------------------------------------------------

struct FastItem {
  Item it;
  int blk[kChunkPagesFast];
};

struct RawFastDesc {
  int4_v a, b, c, d;
};

CDB_DEVICE RawFastDesc load_fast_desc(const DecodeParams& P, int ci) {
  const const_int4_v* d = (const const_int4_v*)(P.desc + (int64_t)ci * kDescInts);
  return RawFastDesc{d[0], d[1], d[2], d[3]};
}

CDB_DEVICE FastItem make_fast_item(const DecodeParams& P, const RawFastDesc& r, int h) {
  FastItem f;
  f.it = make_item(P, RawDesc{r.a, r.b}, h);
  f.blk[0] = r.c.x; f.blk[1] = r.c.y; f.blk[2] = r.c.z; f.blk[3] = r.c.w;
  f.blk[4] = r.d.x; f.blk[5] = r.d.y; f.blk[6] = r.d.z; f.blk[7] = r.d.w;
#pragma unroll
  for (int j = 0; j < kChunkPagesFast; ++j)
    if (!f.it.live || f.blk[j] < 0 || f.blk[j] >= P.pool_blocks) f.blk[j] = -1;
  return f;
}

// Wave step s (16 tokens of page s of the chunk) of K and V. The lane's byte
// offsets inside a page, one per token u, are loop-invariant; a masked page
// reads page 0 of the layer (any valid address) and every token of a masked
// page or at/after t_end gets zero weight. The pages are read once per layer,
// so the loads carry the nontemporal hint (the deep form measured 4-7% faster
// with it, the persistent form 1-2%, and the headline decode run 3%).
template <typename T, int D>
CDB_DEVICE void load_fast_step(const DecodeParams& P, const FastItem& f, int s, const uint32_t (&lane_off)[4],
                               int slot, Vec<T, D / 16> (&kv)[4], Vec<T, D / 16> (&vv)[4], bool (&valid)[4]) {
  const int blk = f.blk[s];
  const int64_t page_bytes = (int64_t)(blk < 0 ? 0 : blk) * (16 * P.num_kv_heads * D * (int64_t)sizeof(T));
  const char* kp = reinterpret_cast<const char*>(pool_layer<T>(P.k_pool, P, f.it)) + page_bytes;
  const char* vp = reinterpret_cast<const char*>(pool_layer<T>(P.v_pool, P, f.it)) + page_bytes;
  const int t0 = f.it.t_begin + 16 * s;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    valid[u] = blk >= 0 && t0 + 4 * u + slot < f.it.t_end;
    kv[u].load_nt(reinterpret_cast<const T*>(kp + lane_off[u]));
    vv[u].load_nt(reinterpret_cast<const T*>(vp + lane_off[u]));
  }
}

template <typename T, int D>
CDB_DEVICE void fast_lane_offsets(const DecodeParams& P, int kvh, int slot, int chunk, uint32_t (&lane_off)[4]) {
  const uint32_t row_bytes = P.num_kv_heads * D * (uint32_t)sizeof(T);
#pragma unroll
  for (int u = 0; u < 4; ++u)
    lane_off[u] = (uint32_t)(4 * u + slot) * row_bytes + (uint32_t)(kvh * D + chunk * (D / 16)) * (uint32_t)sizeof(T);
}

template <typename T, int D, int R>
__global__ void __launch_bounds__(256, 3) paged_decode_fast_kernel(DecodeParams P) {
  constexpr int C = Layout<D>::kChunk;
  const int lane = threadIdx.x & 63;
  const int slot = lane >> 4;
  const int chunk = lane & 15;
  const int H = P.num_heads;
  const int kv_group = H / P.num_kv_heads;
  const int wave = threadIdx.x >> 6;
  __shared__ uint32_t stash[Stash<T, D>::kPerWorkgroup];
  int parity = 0;

  // Items in the plan's longest-first order: wave w takes items w, w + W, ...
  // for its static rounds (no coordination); the remaining items, the tail of
  // the launch, go to whichever wave asks first, from the queue of
  // its workgroup's XCD (queue x of n holds tail items x, x + n, ...). A wave asks
  // when it starts its last static item, so the request's round trip overlaps
  // that item's stream, and waves that stream faster take more of the tail.
  const int nwaves = gridDim.x * 4;
  // A grid of fewer than kQueues workgroups uses only as many queues as it has
  // workgroups, so every queue that holds tail items is drained.
  const int nqueues = min((int)gridDim.x, kQueues);
  const int queue = blockIdx.x % nqueues;
  int32_t* const counter = P.counters + queue * kCounterStride;
  const auto grab = [&]() {
    int k = 0;
    if (lane == 0) k = atomicAdd(counter, 1);
    return k;  // lane 0 holds the ticket; read it with uniform() once it is needed
  };
  const int chunks = *(const const_int32*)(P.header + 1 + P.num_rows);
  const int n_items = (int)min((int64_t)chunks, P.capacity) * H;
  // The tail covers half a round to one and a half rounds of items: a longer
  // tail pays more queue round trips, a shorter one balances less (at 128 rows
  // of 16 heads, 2 static rounds and a 0.56-round tail take 90 us against 97 us
  // with 1 static round). The first round is always static; a launch with at
  // most one item per wave has no tail.
  const int static_rounds = (int)max((2 * (int64_t)n_items - nwaves) / (2 * (int64_t)nwaves), (int64_t)1);
  const int tail_base = min(static_rounds * nwaves, n_items);
  const bool has_tail = tail_base < n_items;
  const int wave_id = uniform(blockIdx.x * 4 + wave);
  int round = 0;
  int item = wave_id;
  if (item >= n_items) return;

  FastItem cur = make_fast_item(P, load_fast_desc(P, item / H), item % H);
  uint32_t lane_off[4];
  fast_lane_offsets<T, D>(P, cur.it.h / kv_group, slot, chunk, lane_off);
  Vec<T, C> ka[4], va[4], kb[4], vb[4];
  bool vla[4], vlb[4];
  load_fast_step<T, D>(P, cur, 0, lane_off, slot, ka, va, vla);
  QueryReg<T, D> q;
  {
    Pending<T, D> pend;
    issue_pending<T, D, R>(P, cur.it, chunk, pend);
    finish_pending<T, D, R>(P, cur.it, chunk, lane, pend, q, stash_slot<T, D>(stash, parity, wave));
  }

  for (;;) {
    // The next item: the next static round, or a tail ticket requested now.
    ++round;
    const bool static_next = round < static_rounds;
    const int ticket = !static_next && has_tail ? grab() : 0;
    int next = n_items;
    bool has_next = false;
    RawFastDesc d_next;
    bool next_known = false;
    // The next item's index and descriptor, once this item's first pair has run.
    auto know_next = [&]() {
      if (next_known) return;
      next_known = true;
      // A negative ticket (queue counters that no plan reset) selects no item.
      const int t = static_next || !has_tail ? -1 : uniform(ticket);
      next = static_next ? wave_id + round * nwaves : t >= 0 ? tail_base + t * nqueues + queue : n_items;
      has_next = next >= 0 && next < n_items;
      d_next = load_fast_desc(P, has_next ? next / H : 0);
    };
    const Item& c = cur.it;
    const int kvh = c.h / kv_group;
    const int steps = (c.t_end - c.t_begin + 15) >> 4;  // wave steps of cached tokens, 0..8

    float m = -INFINITY, l = 0.f;
    float acc[C];
#pragma unroll
    for (int i = 0; i < C; ++i) acc[i] = 0.f;

    FastItem nxt;
    bool nxt_ready = false;
    uint32_t next_off[4];
    Pending<T, D> pend;
    QueryReg<T, D> qn;
    uint32_t* const next_slot = stash_slot<T, D>(stash, parity ^ 1, wave);
    // The next item: its fields (and its query, key and value loads) once its
    // descriptor is needed, its first step when this item's stream ends.
    auto ready_next = [&]() {
      if (nxt_ready) return;
      nxt_ready = true;
      know_next();
      nxt = make_fast_item(P, d_next, next % H);
      if (!has_next) nxt.it.t_end = nxt.it.t_begin;  // a fully masked dummy step
      fast_lane_offsets<T, D>(P, nxt.it.h / kv_group, slot, chunk, next_off);
      if (has_next) issue_pending<T, D, R>(P, nxt.it, chunk, pend);
    };
    auto first_of_next = [&]() {
      ready_next();
      load_fast_step<T, D>(P, nxt, 0, next_off, slot, ka, va, vla);
    };

    if (steps == 0) {
      first_of_next();
    } else {
#pragma unroll
      for (int pr = 0; pr < kChunkPagesFast / 2; ++pr) {
        const int s0 = 2 * pr;
        if (s0 >= steps) break;
        load_fast_step<T, D>(P, cur, s0 + 1, lane_off, slot, kb, vb, vlb);
        attend_step<T, D>(q, P.scale_log2, ka, va, vla, m, l, acc);
        if (s0 + 2 < steps)
          load_fast_step<T, D>(P, cur, s0 + 2, lane_off, slot, ka, va, vla);
        else
          first_of_next();
        attend_step<T, D>(q, P.scale_log2, kb, vb, vlb, m, l, acc);
        if (pr == 0) know_next();
        if (pr == 1) ready_next();
      }
    }
    ready_next();
    if (has_next) finish_pending<T, D, R>(P, nxt.it, chunk, lane, pend, qn, next_slot);

    if (c.last && c.live) {
      // The new token: append its rotated key and its value, then attend to it from registers.
      const int p = c.p;
      const int rel = (p >> 4) - (c.t_begin >> 4);  // page of p inside the chunk, 0..7
      int new_blk = -1;
#pragma unroll
      for (int j = 0; j < kChunkPagesFast; ++j)
        if (j == rel) new_blk = cur.blk[j];
      Vec<T, C> kn, vn;
      const uint32_t* cur_slot = stash_slot<T, D>(stash, parity, wave);
      stash_get<T, D>(cur_slot, 0, kn, lane);
      stash_get<T, D>(cur_slot, 1, vn, lane);
      if (slot == 0 && c.h % kv_group == 0 && new_blk >= 0) {
        const int64_t off = (((int64_t)new_blk << 4) + (p & 15)) * ((int64_t)P.num_kv_heads * D) +
                            (int64_t)kvh * D + chunk * C;
        kn.store(pool_layer<T>(P.k_pool, P, c) + off);
        vn.store(pool_layer<T>(P.v_pool, P, c) + off);
      }
      const float dot = score<T, D>(q, P.scale_log2, kn);
      if (slot == 0) {
        const float m_new = fmaxf(m, dot);
        const float alpha = exp2f(m - m_new);
        const float pn = exp2f(dot - m_new);
        l = l * alpha + pn;
#pragma unroll
        for (int i = 0; i < C; ++i) acc[i] = fmaf(pn, vn.get(i), acc[i] * alpha);
        m = m_new;
      }
    }

    // Merge the four slots of the wave (lanes 16 apart hold the same chunk).
    float m_all = fmaxf(m, shfl_xor_f32(m, 16));
    m_all = fmaxf(m_all, shfl_xor_f32(m_all, 32));
    const float f = (m == -INFINITY) ? 0.f : exp2f(m - m_all);
    l *= f;
#pragma unroll
    for (int i = 0; i < C; ++i) acc[i] *= f;
    l += shfl_xor_f32(l, 16);
    l += shfl_xor_f32(l, 32);
#pragma unroll
    for (int i = 0; i < C; ++i) {
      acc[i] += shfl_xor_f32(acc[i], 16);
      acc[i] += shfl_xor_f32(acc[i], 32);
    }

    if (slot == 0) {
      if (c.single) {
        T* out_row = static_cast<T*>(P.out) + ((int64_t)c.b * H + c.h) * D;
        const float inv = c.live ? 1.f / l : __builtin_nanf("");
        Vec<T, C> o;
#pragma unroll
        for (int i = 0; i < C; i += 2) o.set_pair(i, acc[i] * inv, acc[i + 1] * inv);
        o.store(out_row + chunk * C);
      } else if (c.live) {
        float* part = P.partial + ((int64_t)c.partial * H + c.h) * (D + 2);
#pragma unroll
        for (int i = 0; i < C; ++i) part[chunk * C + i] = acc[i];
        if (chunk == 0) {
          part[D] = m_all;
          part[D + 1] = l;
        }
      }
    }

    if (!has_next) break;
    item = next;
    cur = nxt;
#pragma unroll
    for (int u = 0; u < 4; ++u) lane_off[u] = next_off[u];
    q = qn;
    parity ^= 1;
  }
}

// The fast form for launches of up to kDeepRowsOf<D> rows: such a launch gives a
// wave a few items, so latency matters more than occupancy. Each wave keeps kDeepSteps - 1 steps of K/V in
// flight (four register buffers, 2 waves per SIMD) instead of one, and takes
// its items without cross-item prefetch. A chunk is computed exactly as in
// paged_decode_fast_kernel (same steps in the same order, same masking, same
// new-token and slot merge), so a row's result does not depend on the form.
// The limit is where the deep form stops measuring faster than the persistent
// one: 256 rows for 128-wide heads (with the nontemporal K/V loads, 4-8% faster
// from 128 to 256 rows, no merge launch; 120 rows before them), 120 rows for the
// other head sizes, where it was measured with cached loads.
template <int D> constexpr int kDeepRowsOf = D == 128 ? 256 : 120;
constexpr int kDeepSteps = 4;

template <typename T, int D, bool kCoherent = false>
CDB_DEVICE void merge_chunks(const float* part, int64_t stride, int nsplit, int lane, T* out_row);

// Agent-coherent float loads: the eight XCDs' L2s do not share dirty lines, and these read at the
// point where all of them agree (sc1), without invalidating a whole L2.
CDB_DEVICE float load_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One item's partial (D accumulator floats, then the max and the sum): slot 0's values, the ones
// the merge and the single-chunk output use (the other slots' sums can differ in the last bit,
// since each lane may fuse its own product into its add). Lane (slot s, chunk q) fetches slot 0's
// pair 2s of chunk q and writes it as one 8-byte store (elements 8q + 2s and 8q + 2s + 1 at
// D = 128; the first C/2 slots in general), so a wave's store covers the accumulator contiguously.
// The stores are agent-coherent, for the in-kernel merge. They go out as pairs because each
// coherent store is written through on its own: one 4-byte store per float moved eight times the
// partial's bytes.
template <int D>
CDB_DEVICE void store_partial(float* part, const float* acc, float m_all, float l, int slot, int chunk) {
  constexpr int C = D / 16;
  static_assert(C % 2 == 0, "pairs of accumulator floats");
  float lo = 0.f, hi = 0.f;
#pragma unroll
  for (int k = 0; k < C / 2; ++k) {
    const float a = __int_as_float(__builtin_amdgcn_ds_bpermute(chunk << 2, __float_as_int(acc[2 * k])));
    const float b = __int_as_float(__builtin_amdgcn_ds_bpermute(chunk << 2, __float_as_int(acc[2 * k + 1])));
    lo = slot == k ? a : lo;
    hi = slot == k ? b : hi;
  }
  if (slot < C / 2) {
    uint64_t* dst = reinterpret_cast<uint64_t*>(part + chunk * C + 2 * slot);
    const uint64_t pair = (uint64_t)__float_as_uint(lo) | ((uint64_t)__float_as_uint(hi) << 32);
    __hip_atomic_store(dst, pair, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (slot == 0 && chunk == 0) {
    uint64_t* dst = reinterpret_cast<uint64_t*>(part + D);
    const uint64_t pair = (uint64_t)__float_as_uint(m_all) | ((uint64_t)__float_as_uint(l) << 32);
    __hip_atomic_store(dst, pair, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// The deep form merges without a launch of its own. Every item of a multi-chunk row stores its
// partial with agent-coherent stores, waits until they are performed, and counts itself in its
// (row, head)'s arrival counter (a vector atomic, coherent across the XCDs). The wave that arrives
// last reads the row's partials with agent-coherent loads, merges them in chunk order with the
// merge launch's own arithmetic (so a row's output does not depend on the form), and resets the
// counter for the next call.
template <typename T, int D>
CDB_DEVICE void finish_row_head(const DecodeParams& P, const Item& c, int lane) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's partial stores are performed
  int32_t* const counter = P.arrivals + (int64_t)c.b * P.num_heads + c.h;
  int ticket = 0;
  if (lane == 0) ticket = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (uniform(ticket) != c.nsplit - 1) return;
  asm volatile("" ::: "memory");  // no partial load moves above the arrival count
  T* out_row = static_cast<T*>(P.out) + ((int64_t)c.b * P.num_heads + c.h) * D;
  const int first = P.header[1 + c.b];
  if (c.live && first >= 0 && first + (int64_t)c.nsplit <= P.capacity) {
    const int64_t stride = (int64_t)P.num_heads * (D + 2);
    merge_chunks<T, D, true>(P.partial + (int64_t)first * stride + (int64_t)c.h * (D + 2), stride, c.nsplit,
                             lane, out_row);
  } else {
    for (int d = lane; d < D; d += 64) Elem<T>::store(out_row + d, __builtin_nanf(""));
  }
  if (lane == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Output of the rows that have no chunks, which the merge launch fills in the other forms: zeros
// for padding rows, NaN for rows whose position is out of range. Wave w takes (row, head) pairs
// w, w + W, ...
template <typename T, int D>
CDB_DEVICE void fill_chunkless_rows(const DecodeParams& P, int wave_id, int nwaves, int lane) {
  const int H = P.num_heads;
  for (int pr = wave_id; pr < P.num_rows * H; pr += nwaves) {
    const int b = pr / H;
    if (P.header[2 + b] != P.header[1 + b]) continue;
    const float fill = P.seqlens[b] < 0 ? 0.f : __builtin_nanf("");
    T* out_row = static_cast<T*>(P.out) + (int64_t)pr * D;
    for (int d = lane; d < D; d += 64) Elem<T>::store(out_row + d, fill);
  }
}

template <typename T, int D, int R>
__global__ void __launch_bounds__(256, 2) paged_decode_deep_kernel(DecodeParams P) {
  constexpr int C = Layout<D>::kChunk;
  const int lane = threadIdx.x & 63;
  const int slot = lane >> 4;
  const int chunk = lane & 15;
  const int H = P.num_heads;
  const int kv_group = H / P.num_kv_heads;
  const int nwaves = gridDim.x * 4;
  const int chunks = *(const const_int32*)(P.header + 1 + P.num_rows);
  const int n_items = (int)min((int64_t)chunks, P.capacity) * H;
  const int wave_id = uniform(blockIdx.x * 4 + (threadIdx.x >> 6));
  for (int item = wave_id; item < n_items; item += nwaves) {
    const FastItem cur = make_fast_item(P, load_fast_desc(P, item / H), item % H);
    const Item& c = cur.it;
    const int kvh = c.h / kv_group;
    const int steps = (c.t_end - c.t_begin + 15) >> 4;  // wave steps of cached tokens, 0..8
    const bool append = c.last && c.live;
    uint32_t lane_off[4];
    fast_lane_offsets<T, D>(P, kvh, slot, chunk, lane_off);

    // Query, new token and angles first; then the first steps, all in flight together.
    Pending<T, D> pend;
    issue_pending<T, D, R>(P, c, chunk, pend);
    Angles<D> ang;
    load_angles<D, R>(P, c.p, chunk, ang);
    Vec<T, C> kbuf[kDeepSteps][4], vbuf[kDeepSteps][4];
    bool vl[kDeepSteps][4];
#pragma unroll
    for (int st = 0; st < kDeepSteps - 1; ++st) load_fast_step<T, D>(P, cur, st, lane_off, slot, kbuf[st], vbuf[st], vl[st]);

    QueryReg<T, D> q;
    Vec<T, C> kn, vn;
    {
      const T* q_bias = static_cast<const T*>(P.q_bias);
      const T* k_bias = static_cast<const T*>(P.k_bias);
      float rot[C];
      rotate_raw<T, D, R>(pend.q, ang, q_bias ? q_bias + (int64_t)c.h * D : nullptr, chunk, rot);
      make_query<T, D>(P, rot, q);
      if (append) {
        rotate_raw<T, D, R>(pend.k, ang, k_bias ? k_bias + (int64_t)kvh * D : nullptr, chunk, rot);
#pragma unroll
        for (int i = 0; i < C; i += 2) kn.set_pair(i, rot[i], rot[i + 1]);
        vn = pend.v;
      }
    }

    float m = -INFINITY, l = 0.f;
    float acc[C];
#pragma unroll
    for (int i = 0; i < C; ++i) acc[i] = 0.f;
#pragma unroll
    for (int st = 0; st < kChunkPagesFast; ++st) {
      if (st >= steps) break;
      const int ahead = st + kDeepSteps - 1;
      if (ahead < kChunkPagesFast)
        load_fast_step<T, D>(P, cur, ahead, lane_off, slot, kbuf[ahead % kDeepSteps], vbuf[ahead % kDeepSteps],
                             vl[ahead % kDeepSteps]);
      attend_step<T, D>(q, P.scale_log2, kbuf[st % kDeepSteps], vbuf[st % kDeepSteps], vl[st % kDeepSteps], m, l,
                        acc);
    }

    if (append) {
      // The new token: append its rotated key and its value, then attend to it from registers.
      const int p = c.p;
      const int rel = (p >> 4) - (c.t_begin >> 4);  // page of p inside the chunk, 0..7
      int new_blk = -1;
#pragma unroll
      for (int j = 0; j < kChunkPagesFast; ++j)
        if (j == rel) new_blk = cur.blk[j];
      if (slot == 0 && c.h % kv_group == 0 && new_blk >= 0) {
        const int64_t off = (((int64_t)new_blk << 4) + (p & 15)) * ((int64_t)P.num_kv_heads * D) +
                            (int64_t)kvh * D + chunk * C;
        kn.store(pool_layer<T>(P.k_pool, P, c) + off);
        vn.store(pool_layer<T>(P.v_pool, P, c) + off);
      }
      const float dot = score<T, D>(q, P.scale_log2, kn);
      if (slot == 0) {
        const float m_new = fmaxf(m, dot);
        const float alpha = exp2f(m - m_new);
        const float pn = exp2f(dot - m_new);
        l = l * alpha + pn;
#pragma unroll
        for (int i = 0; i < C; ++i) acc[i] = fmaf(pn, vn.get(i), acc[i] * alpha);
        m = m_new;
      }
    }

    // Merge the four slots of the wave (lanes 16 apart hold the same chunk).
    float m_all = fmaxf(m, shfl_xor_f32(m, 16));
    m_all = fmaxf(m_all, shfl_xor_f32(m_all, 32));
    const float f = (m == -INFINITY) ? 0.f : exp2f(m - m_all);
    l *= f;
#pragma unroll
    for (int i = 0; i < C; ++i) acc[i] *= f;
    l += shfl_xor_f32(l, 16);
    l += shfl_xor_f32(l, 32);
#pragma unroll
    for (int i = 0; i < C; ++i) {
      acc[i] += shfl_xor_f32(acc[i], 16);
      acc[i] += shfl_xor_f32(acc[i], 32);
    }
    if (slot == 0) {
      if (c.single) {
        T* out_row = static_cast<T*>(P.out) + ((int64_t)c.b * H + c.h) * D;
        const float inv = c.live ? 1.f / l : __builtin_nanf("");
        Vec<T, C> o;
#pragma unroll
        for (int i = 0; i < C; i += 2) o.set_pair(i, acc[i] * inv, acc[i + 1] * inv);
        o.store(out_row + chunk * C);
      }
    }
    if (!c.single && c.live)
      store_partial<D>(P.partial + ((int64_t)c.partial * H + c.h) * (D + 2), acc, m_all, l, slot, chunk);
    if (!c.single && c.nsplit > 1) finish_row_head<T, D>(P, c, lane);
  }
  fill_chunkless_rows<T, D>(P, wave_id, nwaves, lane);
}

// The merge of one (row, head): chunk c's partial (unnormalized accumulator of
// D floats, then its max and sum) starts at part + c * stride. Lane s holds
// chunk s's (max, sum) so the global max and the denominator are wave
// reductions; the accumulators are read eight chunks at a time so their loads
// are in flight together.
template <typename T, int D, bool kCoherent>
CDB_DEVICE void merge_chunks(const float* part, int64_t stride, int nsplit, int lane, T* out_row) {
  const auto ld = [](const float* p) { return kCoherent ? load_coherent(p) : *p; };
  const int d0 = lane, d1 = lane + 64;
  float run_m = -INFINITY, den = 0.f, num0 = 0.f, num1 = 0.f;
  for (int base = 0; base < nsplit; base += 64) {
    const int cnt = min(64, nsplit - base);
    const float* chunk_part = part + (int64_t)base * stride;
    float a0[8], a1[8];
    auto load_group = [&](int s0) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const bool ok = s0 + j < cnt;
        const float* ps = chunk_part + (int64_t)(s0 + j) * stride;
        a0[j] = ok && d0 < D ? ld(ps + d0) : 0.f;
        a1[j] = ok && d1 < D ? ld(ps + d1) : 0.f;
      }
    };
    // The first eight chunks' accumulators are read with the (max, sum) pairs, so
    // their loads overlap instead of waiting for the wave reductions.
    load_group(0);
    float ms = -INFINITY, ls = 0.f;
    if (lane < cnt) {
      ms = ld(chunk_part + lane * stride + D);
      ls = ld(chunk_part + lane * stride + D + 1);
    }
    const float new_m = fmaxf(run_m, wave_max(ms));
    const float keep = run_m == -INFINITY ? 0.f : exp2f(run_m - new_m);
    num0 *= keep;
    num1 *= keep;
    den *= keep;
    const float ws = ms == -INFINITY ? 0.f : exp2f(ms - new_m);
    den += wave_sum(ws * ls);
    for (int s0 = 0; s0 < cnt; s0 += 8) {
      if (s0 > 0) load_group(s0);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        // Lanes at or past cnt hold a zero weight.
        const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ws), min(s0 + j, 63)));
        num0 = fmaf(wj, a0[j], num0);
        num1 = fmaf(wj, a1[j], num1);
      }
    }
    run_m = new_m;
  }
  const float inv = 1.f / den;
  if (d0 < D) Elem<T>::store(out_row + d0, num0 * inv);
  if (d1 < D) Elem<T>::store(out_row + d1, num1 * inv);
}

// Merge the chunk partials of every (row, head) whose row has more than one
// chunk, in chunk order; one wave per (row, head). Rows without chunks get zeros
// (padding rows) or NaN (rows out of range), and multi-chunk rows whose cache
// layer is missing get NaN.
template <typename T, int D>
__global__ void __launch_bounds__(256) decode_merge_kernel(DecodeParams P) {
  const int lane = threadIdx.x & 63;
  const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
  // The decode kernel before this one has drained the item queues: reset them for the next call.
  if (blockIdx.x == 0 && threadIdx.x < kQueues) P.counters[threadIdx.x * kCounterStride] = 0;
  if (w >= P.num_rows * P.num_heads) return;
  const int b = w / P.num_heads;
  const int h = w - b * P.num_heads;
  const int first = P.header[1 + b];
  const int nsplit = P.header[2 + b] - first;
  if (nsplit == 1) return;  // stored by the decode kernel
  T* out_row = static_cast<T*>(P.out) + ((int64_t)b * P.num_heads + h) * D;
  const bool live = nsplit > 1 && first >= 0 && first + (int64_t)nsplit <= P.capacity &&
                    layer_in_range(P, P.cache_layer ? P.cache_layer[b] : 0);
  if (!live) {
    const float fill = nsplit == 0 && P.seqlens[b] < 0 ? 0.f : __builtin_nanf("");
    for (int d = lane; d < D; d += 64) Elem<T>::store(out_row + d, fill);
    return;
  }
  const int64_t stride = (int64_t)P.num_heads * (D + 2);
  merge_chunks<T, D>(P.partial + (int64_t)first * stride + (int64_t)h * (D + 2), stride, nsplit, lane, out_row);
}

}  // namespace cdb

using namespace cdb;

// The fixed scratch of cdb_paged_decode_attention_noalloc: a file-scope device array, one copy per
// GPU, alive until the process ends. Host code never passes the array's name to a kernel (on the
// host it is only a stand-in symbol); scratch_address() resolves each device's own address once,
// with that device current, and the launches use that address.
static __device__ __align__(256) unsigned char scratch[CDB_DECODE_SCRATCH_BYTES];

namespace {

int g_num_cus = 0;

// Resident workgroups per CU for a kernel, cached per kernel. The persistent
// decode kernels assign items by wave stride, so a grid must not exceed what is
// resident at once.
typedef void (*DecodeKernel)(DecodeParams);
std::mutex g_occupancy_mutex;
std::vector<std::pair<DecodeKernel, int>> g_occupancy;

int resident_blocks_per_cu(DecodeKernel kernel) {
  std::lock_guard<std::mutex> lock(g_occupancy_mutex);
  for (const auto& entry : g_occupancy)
    if (entry.first == kernel) return entry.second;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, 256, 0) != hipSuccess || n <= 0) n = 1;
  g_occupancy.emplace_back(kernel, n);
  return n;
}

int ilog2_exact(int x) {
  if (x <= 0 || (x & (x - 1))) return -1;
  int r = 0;
  while ((1 << r) < x) ++r;
  return r;
}

// Workspace: the header (chunk tokens, chunk prefix over rows), the queue counters, the
// arrival counters (one per row and head), each 256-byte aligned; then descriptors and partials.
int64_t counters_offset(int64_t num_rows) { return ((num_rows + 2) * 4 + 255) / 256 * 256; }
int64_t arrivals_offset(int64_t num_rows) { return counters_offset(num_rows) + kQueues * kCounterStride * 4; }
int64_t header_bytes(int64_t num_rows, int64_t num_heads) {
  return arrivals_offset(num_rows) + (num_rows * num_heads * 4 + 255) / 256 * 256;
}

int64_t bytes_per_chunk(int64_t num_heads, int64_t head_dim) {
  return kDescBytes + num_heads * (head_dim + 2) * (int64_t)sizeof(float);
}

// The persistent grid is at most what is resident at once, and no larger than
// the launch can have items for: rows x ceil(table_width / chunk_pages) chunks
// (fewer when the plan lengthens chunks) times the heads, one wave per item.
int launch_persistent(DecodeKernel kernel, const DecodeParams& P, int num_cus, hipStream_t stream) {
  const int64_t chunks = std::min<int64_t>((int64_t)P.num_rows * ((P.table_width + P.chunk_pages - 1) / P.chunk_pages),
                                           P.capacity);
  const int64_t wanted = (chunks * P.num_heads + 3) / 4;
  const int grid = (int)std::max<int64_t>(1, std::min<int64_t>(wanted, (int64_t)num_cus * resident_blocks_per_cu(kernel)));
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(256), 0, stream, P);
  return hipGetLastError() == hipSuccess ? CDB_OK : CDB_ERR_HIP;
}

// The fast form needs 16-token pages and chunks of kChunkPagesFast pages. The plan
// keeps chunks at chunk_pages unless the workspace cannot hold them; with at most
// ceil(table_width / chunk_pages) chunks per row it always can.
bool fast_form(const DecodeParams& P) {
  const int64_t per_row = (P.table_width + P.chunk_pages - 1) / P.chunk_pages;
  return P.block_size_log2 == 4 && P.chunk_pages == kChunkPagesFast && P.capacity >= (int64_t)P.num_rows * per_row;
}

template <typename T, int D, int R>
int launch_decode(const DecodeParams& P, int stages, int num_cus, hipStream_t stream) {
  if (stages & CDB_DECODE_STAGE_PLAN) {
    hipLaunchKernelGGL(decode_plan_kernel, dim3(1), dim3(kPlanThreads), 0, stream, P);
    if (hipGetLastError() != hipSuccess) return CDB_ERR_HIP;
  }
  if (!(stages & CDB_DECODE_STAGE_ATTEND)) return CDB_OK;
  const bool deep = fast_form(P) && P.num_rows <= kDeepRowsOf<D>;
  const int rc = !fast_form(P) ? launch_persistent(paged_decode_kernel<T, D, R>, P, num_cus, stream)
                 : deep        ? launch_persistent(paged_decode_deep_kernel<T, D, R>, P, num_cus, stream)
                               : launch_persistent(paged_decode_fast_kernel<T, D, R>, P, num_cus, stream);
  if (rc != CDB_OK) return rc;
  // A deep launch has merged and filled every row itself (against the merge launch, same box, per
  // layer, with the partials' 8-byte coherent stores: 0.1-0.5 us faster from 1 to 16 rows, 1-2 us
  // from 24 to 120 rows); the others end with the merge launch.
  if (deep) return CDB_OK;
  const int64_t waves = (int64_t)P.num_rows * P.num_heads;
  hipLaunchKernelGGL((decode_merge_kernel<T, D>), dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, stream, P);
  return hipGetLastError() == hipSuccess ? CDB_OK : CDB_ERR_HIP;
}

template <typename T, int R>
int dispatch_dim(const DecodeParams& P, int head_dim, int stages, int num_cus, hipStream_t stream) {
  switch (head_dim) {
    case 64: return launch_decode<T, 64, R>(P, stages, num_cus, stream);
    case 96: return launch_decode<T, 96, R>(P, stages, num_cus, stream);
    case 128: return launch_decode<T, 128, R>(P, stages, num_cus, stream);
    default: return CDB_ERR_UNSUPPORTED;
  }
}

template <typename T>
int dispatch_rope(const DecodeParams& P, int head_dim, int stages, int num_cus, hipStream_t stream) {
  if (P.rope_cos == nullptr) return dispatch_dim<T, 0>(P, head_dim, stages, num_cus, stream);
  if (P.rope_style == 1) return dispatch_dim<T, 1>(P, head_dim, stages, num_cus, stream);
  return dispatch_dim<T, 2>(P, head_dim, stages, num_cus, stream);
}

constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices] = {};
std::mutex g_scratch_mutex;

int scratch_address(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return CDB_ERR_HIP;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) return CDB_ERR_HIP;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return CDB_OK;
}

int decode_attention(const void* q, const void* k_new, const void* v_new, void* k_pool, void* v_pool,
                     int64_t layer_stride, int32_t num_cache_layers, int64_t pool_blocks, const int32_t* cache_layer,
                     int32_t cache_layer0, const int32_t* block_table, const int32_t* table_row,
                     int32_t table_width, const int32_t* seqlens, const float* rope_cos, const float* rope_sin,
                     int32_t rope_style, int32_t max_positions, const void* q_bias, const void* k_bias, void* out,
                     void* workspace, int64_t workspace_bytes, int32_t num_rows, int32_t num_heads,
                     int32_t num_kv_heads, int32_t head_dim, int32_t block_size, int32_t split_pages,
                     int32_t min_split_pages, float scale, int64_t q_stride, int64_t kv_stride, int32_t dtype,
                     int32_t stages, hipStream_t stream);

}  // namespace

extern "C" {

int64_t cdb_paged_decode_workspace_bytes(int32_t num_rows, int32_t num_heads, int32_t head_dim,
                                         int32_t max_seqlen, int32_t block_size, int32_t split_pages) {
  if (num_rows < 0 || num_heads <= 0 || head_dim <= 0 || max_seqlen <= 0 || block_size <= 0 || split_pages <= 0)
    return -1;
  const int64_t split_tokens = (int64_t)split_pages * block_size;
  const int64_t max_splits = (max_seqlen + split_tokens - 1) / split_tokens + 1;
  return header_bytes(num_rows, num_heads) + (int64_t)num_rows * max_splits * bytes_per_chunk(num_heads, head_dim);
}

int cdb_paged_decode_attention(const void* q, const void* k_new, const void* v_new, void* k_pool, void* v_pool,
                               int64_t layer_stride, int32_t num_cache_layers, int64_t pool_blocks,
                               const int32_t* cache_layer, int32_t cache_layer0,
                               const int32_t* block_table, const int32_t* table_row, int32_t table_width,
                               const int32_t* seqlens, const float* rope_cos, const float* rope_sin,
                               int32_t rope_style, int32_t max_positions, const void* q_bias, const void* k_bias,
                               void* out, void* workspace, int64_t workspace_bytes, int32_t num_rows,
                               int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                               int32_t split_pages, int32_t min_split_pages, float scale,
                               int64_t q_stride, int64_t kv_stride, int32_t dtype, hipStream_t stream) {
  return decode_attention(q, k_new, v_new, k_pool, v_pool, layer_stride, num_cache_layers, pool_blocks, cache_layer,
                          cache_layer0, block_table, table_row, table_width, seqlens, rope_cos, rope_sin, rope_style,
                          max_positions, q_bias, k_bias, out, workspace, workspace_bytes, num_rows, num_heads,
                          num_kv_heads, head_dim, block_size, split_pages, min_split_pages, scale, q_stride,
                          kv_stride, dtype, CDB_DECODE_STAGE_PLAN | CDB_DECODE_STAGE_ATTEND, stream);
}

int cdb_paged_decode_attention_staged(const void* q, const void* k_new, const void* v_new, void* k_pool,
                                      void* v_pool, int64_t layer_stride, int32_t num_cache_layers,
                                      int64_t pool_blocks, const int32_t* cache_layer, int32_t cache_layer0,
                                      const int32_t* block_table, const int32_t* table_row, int32_t table_width,
                                      const int32_t* seqlens, const float* rope_cos, const float* rope_sin,
                                      int32_t rope_style, int32_t max_positions, const void* q_bias,
                                      const void* k_bias, void* out, void* workspace, int64_t workspace_bytes,
                                      int32_t num_rows, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                      int32_t block_size, int32_t split_pages, int32_t min_split_pages, float scale,
                                      int64_t q_stride, int64_t kv_stride, int32_t dtype, int32_t stages,
                                      hipStream_t stream) {
  if (stages <= 0 || (stages & ~(CDB_DECODE_STAGE_PLAN | CDB_DECODE_STAGE_ATTEND))) return CDB_ERR_SHAPE;
  return decode_attention(q, k_new, v_new, k_pool, v_pool, layer_stride, num_cache_layers, pool_blocks, cache_layer,
                          cache_layer0, block_table, table_row, table_width, seqlens, rope_cos, rope_sin, rope_style,
                          max_positions, q_bias, k_bias, out, workspace, workspace_bytes, num_rows, num_heads,
                          num_kv_heads, head_dim, block_size, split_pages, min_split_pages, scale, q_stride,
                          kv_stride, dtype, stages, stream);
}

int cdb_paged_decode_attention_noalloc(const void* q, const void* k_new, const void* v_new, void* k_pool,
                                       void* v_pool, int64_t layer_stride, int32_t num_cache_layers,
                                       int64_t pool_blocks, const int32_t* cache_layer, int32_t cache_layer0,
                                       const int32_t* block_table, const int32_t* table_row, int32_t table_width,
                                       const int32_t* seqlens, const float* rope_cos, const float* rope_sin,
                                       int32_t rope_style, int32_t max_positions, const void* q_bias,
                                       const void* k_bias, void* out, int32_t num_rows, int32_t num_heads,
                                       int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                       int32_t split_pages, int32_t min_split_pages,
                                       float scale, int64_t q_stride, int64_t kv_stride, int32_t dtype,
                                       hipStream_t stream) {
  if (num_rows == 0) return CDB_OK;
  if (num_rows < 0 || num_heads <= 0 || head_dim <= 0) return CDB_ERR_SHAPE;
  // The plan lengthens chunks until they fit, down to one chunk per row: the scratch must hold
  // the header and one descriptor and partial per row.
  const int64_t need = header_bytes(num_rows, num_heads) + (int64_t)num_rows * bytes_per_chunk(num_heads, head_dim);
  if (need > CDB_DECODE_SCRATCH_BYTES) return CDB_ERR_CAPACITY;
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != CDB_OK) return rc;
  return decode_attention(q, k_new, v_new, k_pool, v_pool, layer_stride, num_cache_layers, pool_blocks, cache_layer,
                          cache_layer0, block_table, table_row, table_width, seqlens, rope_cos, rope_sin, rope_style,
                          max_positions, q_bias, k_bias, out, ws, CDB_DECODE_SCRATCH_BYTES, num_rows, num_heads,
                          num_kv_heads, head_dim, block_size, split_pages, min_split_pages, scale, q_stride,
                          kv_stride, dtype, CDB_DECODE_STAGE_PLAN | CDB_DECODE_STAGE_ATTEND, stream);
}

}  // extern "C"

namespace {

int decode_attention(const void* q, const void* k_new, const void* v_new, void* k_pool, void* v_pool,
                     int64_t layer_stride, int32_t num_cache_layers, int64_t pool_blocks, const int32_t* cache_layer,
                     int32_t cache_layer0, const int32_t* block_table, const int32_t* table_row,
                     int32_t table_width, const int32_t* seqlens, const float* rope_cos, const float* rope_sin,
                     int32_t rope_style, int32_t max_positions, const void* q_bias, const void* k_bias, void* out,
                     void* workspace, int64_t workspace_bytes, int32_t num_rows, int32_t num_heads,
                     int32_t num_kv_heads, int32_t head_dim, int32_t block_size, int32_t split_pages,
                     int32_t min_split_pages, float scale, int64_t q_stride, int64_t kv_stride, int32_t dtype,
                     int32_t stages, hipStream_t stream) {
  if (num_rows == 0) return CDB_OK;
  if (!q || !k_new || !v_new || !k_pool || !v_pool || !block_table || !seqlens || !out || !workspace)
    return CDB_ERR_NULL;
  if (num_rows < 0 || num_rows > kMaxRowsLds || num_heads <= 0 || num_kv_heads <= 0 ||
      num_heads % num_kv_heads != 0 || table_width <= 0)
    return CDB_ERR_SHAPE;
  const int chunk_pages = split_pages > 0 ? split_pages : min_split_pages;
  if (chunk_pages <= 0) return CDB_ERR_SHAPE;
  const int bs_log2 = ilog2_exact(block_size);
  if (bs_log2 < 0) return CDB_ERR_SHAPE;
  if (((int64_t)chunk_pages << bs_log2) > (1 << 29)) return CDB_ERR_SHAPE;
  if (rope_style < 0 || rope_style > 2) return CDB_ERR_SHAPE;
  if (rope_style != 0 && (!rope_cos || !rope_sin || max_positions <= 0)) return CDB_ERR_NULL;
  if (rope_style == 1 && head_dim != 128 && head_dim != 64 && head_dim != 96) return CDB_ERR_UNSUPPORTED;
  if (dtype != CDB_DTYPE_F32 && dtype != CDB_DTYPE_BF16) return CDB_ERR_UNSUPPORTED;
  // Split-half rotation pairs chunk c with chunk c ^ 8, i.e. D/2 = 8 chunks.
  if (rope_style == 1 && (head_dim / 16) * 8 != head_dim / 2) return CDB_ERR_UNSUPPORTED;
  if (num_cache_layers <= 0 || pool_blocks <= 0 || layer_stride < 0) return CDB_ERR_SHAPE;
  const int64_t header = header_bytes(num_rows, num_heads);
  const int64_t capacity = workspace_bytes > header ? (workspace_bytes - header) / bytes_per_chunk(num_heads, head_dim) : 0;
  // One chunk per row must fit; the item index (chunk * heads) must fit an int.
  if (capacity < num_rows) return CDB_ERR_CAPACITY;

  DecodeParams P;
  P.q = q; P.k_new = k_new; P.v_new = v_new; P.k_pool = k_pool; P.v_pool = v_pool;
  P.block_table = block_table; P.table_row = table_row; P.seqlens = seqlens; P.cache_layer = cache_layer;
  P.rope_cos = rope_style ? rope_cos : nullptr; P.rope_sin = rope_style ? rope_sin : nullptr;
  P.q_bias = q_bias; P.k_bias = k_bias; P.out = out;
  P.header = static_cast<int32_t*>(workspace);
  P.counters = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + counters_offset(num_rows));
  P.arrivals = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + arrivals_offset(num_rows));
  P.capacity = capacity < ((int64_t)1 << 31) / num_heads ? capacity : ((int64_t)1 << 31) / num_heads - 1;
  P.desc = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + header);
  P.partial = reinterpret_cast<float*>(static_cast<char*>(workspace) + header + capacity * kDescBytes);
  P.layer_stride = layer_stride; P.cache_layer0 = cache_layer0;
  P.q_stride = q_stride > 0 ? q_stride : (int64_t)num_heads * head_dim;
  P.kv_stride = kv_stride > 0 ? kv_stride : (int64_t)num_kv_heads * head_dim;
  if (P.q_stride < (int64_t)num_heads * head_dim || P.kv_stride < (int64_t)num_kv_heads * head_dim) return CDB_ERR_SHAPE;
  P.num_rows = num_rows; P.num_heads = num_heads; P.num_kv_heads = num_kv_heads;
  P.table_width = table_width; P.block_size_log2 = bs_log2; P.chunk_pages = chunk_pages;
  P.rope_style = rope_style; P.max_positions = max_positions;
  P.num_cache_layers = num_cache_layers; P.pool_blocks = pool_blocks;
  P.scale_log2 = scale * 1.4426950408889634f;

  if (g_num_cus == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return CDB_ERR_HIP;
    if (hipDeviceGetAttribute(&g_num_cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return CDB_ERR_HIP;
  }
  if (dtype == CDB_DTYPE_F32) return dispatch_rope<float>(P, head_dim, stages, g_num_cus, stream);
  return dispatch_rope<bf16_t>(P, head_dim, stages, g_num_cus, stream);
}

}  // namespace
