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
// Work decomposition (split-KV / flash-decoding):
//   * a row's context is cut into splits of `split_pages` pages; with
//     split_pages <= 0 every workgroup derives the same split size from the
//     launch's total page count: the smallest power of two in [min_split_pages,
//     max_split_pages] for which the items are at most four times the
//     persistent workgroups (coarsened further if the workspace is too small).
//     Longer splits mean fewer partials to merge and fewer per-item latency
//     chains; shorter ones keep narrow batches from leaving workgroups idle and
//     even out the tail;
//   * a work item is (row, split, group of 4 query heads); one workgroup of
//     4 waves takes an item, wave w owning query head 4*g + w;
//   * workgroups are persistent: workgroup i processes items i, i+G, ...,
//     so the grid does not depend on the context lengths (graph-capturable);
//   * each workgroup builds per-row metadata and split prefix sums in LDS;
//     items list every full-length split first and the rows' last (shorter)
//     splits after them, and an item finds its row by binary search;
//     workgroup 0 also stores the split prefix in the workspace header for the
//     merge kernel.
// Inside a wave, lane = 16 * slot + chunk: the 16 lanes of a DPP row split the
// head dimension into 16 chunks and the 4 rows ("slots") take interleaved
// tokens. q.k is reduced across a row with four DPP rotate-adds; each slot keeps
// its own online-softmax state, merged across slots at the end. An item's first
// K/V step, its query and the new token's key/value are all issued before the
// first wait, and every later step's loads are issued one step ahead (two
// register buffers).
// A row with one split writes its normalized output directly; otherwise the
// split's (unnormalized acc, max, sum) goes to the workspace and a second
// kernel merges the splits. The merge is a separate launch on purpose: merging
// in the last-arriving workgroup needs a device-scope release/acquire per item,
// which on a multi-XCD part writes back and invalidates the XCD's L2 and costs
// far more than the launch.
//
// Workspace: int32 header [split_tokens (-1: partial space too small),
// split_prefix[0..B]] padded to 256 bytes, then fp32 partials
// [total_splits, H, D + 2].

#include <mutex>

#include "cdb_common.h"
#include "../../include/cdb_amd.h"

namespace cdb {

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
  int32_t* header;              // [B + 2]: split_tokens (or -1), then the split prefix over rows
  float* partial;               // [total_splits, H, D + 2] when a row has > 1 split
  int64_t layer_stride;         // elements between cache layers
  int64_t q_stride, kv_stride;  // elements between consecutive rows of q and of k_new/v_new
  int32_t cache_layer0;
  int32_t num_rows, num_heads, num_kv_heads;
  int32_t table_width, block_size_log2, split_pages;
  int32_t rope_style;           // 0 none, 1 split-half, 2 interleaved pairs
  int32_t max_positions;
  int32_t num_cache_layers;     // valid cache_layer values are [0, num_cache_layers)
  int64_t pool_blocks;          // valid block ids are [0, pool_blocks)
  int64_t partial_capacity;     // splits the workspace holds
  int32_t min_split_pages, max_split_pages;  // range of the adaptive split size (split_pages <= 0)
  float scale_log2;             // softmax scale * log2(e)
};

constexpr int kMaxRowsLds = 2048;

template <int D> struct Layout {
  static constexpr int kChunk = D / 16;  // elements per lane
  static_assert(D % 16 == 0, "head_dim must be a multiple of 16");
};

// A row is served when its new-token position fits the block table and the
// RoPE table and its cache layer exists. Rows failing this get no work and a
// NaN output; padding rows (p < 0) get zeros.
CDB_DEVICE bool row_valid(const DecodeParams& P, int b, int p) {
  if (p < 0) return false;
  if ((int64_t)p >= ((int64_t)P.table_width << P.block_size_log2)) return false;
  if (P.rope_cos != nullptr && p >= P.max_positions) return false;
  const int layer = P.cache_layer0 + (P.cache_layer ? P.cache_layer[b] : 0);
  return layer >= 0 && layer < P.num_cache_layers;
}

// Rotate this lane's chunk of a head vector. `own`/`partner` are the lane's
// chunk and (for split-half) the chunk D/2 away; values are returned rounded to
// the storage type the way the reference's torch ops round them.
template <typename T, int D>
CDB_DEVICE void rope_chunk(const DecodeParams& P, int pos, int chunk, const float* own, const float* partner,
                           float* out) {
  constexpr int C = Layout<D>::kChunk;
  if (P.rope_style == 0 || P.rope_cos == nullptr) {
#pragma unroll
    for (int i = 0; i < C; ++i) out[i] = own[i];
    return;
  }
  const int half = D / 2;
  const float* cos_row = P.rope_cos + (int64_t)pos * half;
  const float* sin_row = P.rope_sin + (int64_t)pos * half;
  if (P.rope_style == 1) {
    // q*cos + rotate_half(q)*sin with cos/sin = cat(f, f); each op rounded. A
    // chunk lies inside one half, so its angles are C consecutive table entries.
    const int f0 = (chunk * C) % half;
    Vec<float, C> cv, sv;
    cv.load(cos_row + f0);
    sv.load(sin_row + f0);
    const bool first_half = chunk * C < half;
#pragma unroll
    for (int i = 0; i < C; ++i) {
      const float rot = first_half ? -partner[i] : partner[i];
      const float a = Elem<T>::round(mul_rn(own[i], __uint_as_float(cv.w[i])));
      const float b = Elem<T>::round(mul_rn(rot, __uint_as_float(sv.w[i])));
      out[i] = Elem<T>::round(add_rn(a, b));
    }
  } else {
    // Interleaved (even, odd) pairs rotated in fp32, rounded once at the end.
    Vec<float, C / 2> cv, sv;
    cv.load(cos_row + chunk * C / 2);
    sv.load(sin_row + chunk * C / 2);
#pragma unroll
    for (int i = 0; i < C; i += 2) {
      const float c = __uint_as_float(cv.w[i / 2]), s = __uint_as_float(sv.w[i / 2]);
      const float x0 = own[i], x1 = own[i + 1];
      out[i] = Elem<T>::round(sub_rn(mul_rn(x0, c), mul_rn(x1, s)));
      out[i + 1] = Elem<T>::round(add_rn(mul_rn(x1, c), mul_rn(x0, s)));
    }
  }
}

// This lane's chunk of one head vector and, for split-half RoPE, its partner
// chunk D/2 away, as loaded (rotation happens later so the loads can be issued
// early).
template <typename T, int D>
struct RawChunk {
  Vec<T, D / 16> own, partner;
};

template <typename T, int D>
CDB_DEVICE void load_raw(const DecodeParams& P, const T* base, int chunk, RawChunk<T, D>& r) {
  constexpr int C = Layout<D>::kChunk;
  r.own.load(base + chunk * C);
  if (P.rope_style == 1 && P.rope_cos != nullptr) r.partner.load(base + (chunk ^ 8) * C);
}

// Add an optional per-head bias to a loaded chunk and rotate it.
template <typename T, int D>
CDB_DEVICE void rotate_raw(const DecodeParams& P, const RawChunk<T, D>& r, const T* bias, int pos, int chunk,
                           float* out) {
  constexpr int C = Layout<D>::kChunk;
  float own[C], partner[C];
#pragma unroll
  for (int i = 0; i < C; ++i) own[i] = r.own.get(i);
  const bool split_half = P.rope_style == 1 && P.rope_cos != nullptr;
  if (split_half) {
#pragma unroll
    for (int i = 0; i < C; ++i) partner[i] = r.partner.get(i);
  }
  if (bias != nullptr) {
    Vec<T, C> bv;
    bv.load(bias + chunk * C);
#pragma unroll
    for (int i = 0; i < C; ++i) own[i] = Elem<T>::round(add_rn(own[i], bv.get(i)));
    if (split_half) {
      bv.load(bias + (chunk ^ 8) * C);
#pragma unroll
      for (int i = 0; i < C; ++i) partner[i] = Elem<T>::round(add_rn(partner[i], bv.get(i)));
    }
  }
  rope_chunk<T, D>(P, pos, chunk, own, partner, out);
}

template <typename T, int D>
CDB_DEVICE void load_rotated(const DecodeParams& P, const T* base, const T* bias, int pos, int chunk, float* out) {
  RawChunk<T, D> r;
  load_raw<T, D>(P, base, chunk, r);
  rotate_raw<T, D>(P, r, bias, pos, chunk, out);
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
// past t_end, or with an out-of-range block id, are masked and their registers
// zeroed so a zero softmax weight never multiplies garbage.
template <typename T, int D>
CDB_DEVICE void load_step(const DecodeParams& P, int window, int win_base, const T* k_base, const T* v_base,
                          int t0, int t_end, int slot, int chunk, int kvh, int bs_log2, int64_t row_elems,
                          Vec<T, D / 16> (&kv)[4], Vec<T, D / 16> (&vv)[4], bool (&valid)[4]) {
  constexpr int C = D / 16;
  // With pages of >= 16 tokens the whole step sits in one page: one wave-uniform lookup.
  const int step_blk = bs_log2 >= 4 ? __builtin_amdgcn_readlane(window, (t0 >> bs_log2) - win_base) : -1;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int t = t0 + 4 * u + slot;
    const int blk_any = bs_log2 >= 4 ? step_blk : window_block(window, win_base, t >> bs_log2);
    const int blk = t < t_end ? blk_any : -1;
    valid[u] = blk >= 0 && blk < P.pool_blocks;
    if (valid[u]) {
      const int64_t row = ((int64_t)blk << bs_log2) + (t & ((1 << bs_log2) - 1));
      const int64_t off = row * row_elems + (int64_t)kvh * D + chunk * C;
      kv[u].load(k_base + off);
      vv[u].load(v_base + off);
    } else {
#pragma unroll
      for (int w = 0; w < Vec<T, C>::kWords; ++w) kv[u].w[w] = vv[u].w[w] = 0u;
    }
  }
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// a.x * b.x + a.y * b.y + c over packed bf16 pairs, fp32 accumulate (v_dot2c_f32_bf16).
CDB_DEVICE float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c,
                                         false);
}

// The query in the form the step loop consumes: fp32 pre-scaled by
// scale*log2(e) for fp32 pools; for bf16 pools the rotated query's bf16 pairs
// (exact: RoPE output is rounded to bf16) with the scale applied to each score.
template <typename T, int D>
struct QueryReg {
  float f[D / 16];
  uint32_t p[D / 32 > 0 ? D / 32 : 1];
};

// Online-softmax update of one slot's state with its 4 tokens of a wave step.
// bf16: q.k is four v_dot2 per token; P.V pairs two tokens' probabilities,
// rounded to bf16 as flash-attention feeds P to its PV product, against the two
// tokens' values interleaved with v_perm.
template <typename T, int D>
CDB_DEVICE void attend_step(const QueryReg<T, D>& q, float scale_log2, const Vec<T, D / 16> (&kv)[4],
                            const Vec<T, D / 16> (&vv)[4], const bool (&valid)[4], float& m, float& l, float* acc) {
  constexpr int C = D / 16;
  constexpr bool kBf16 = sizeof(T) == 2;
  float sc[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    float dot = 0.f;
    if constexpr (kBf16) {
#pragma unroll
      for (int w = 0; w < C / 2; ++w) dot = dot2_bf16(q.p[w], kv[u].w[w], dot);
      dot = row16_sum(dot) * scale_log2;
    } else {
#pragma unroll
      for (int i = 0; i < C; ++i) dot = fmaf(q.f[i], kv[u].get(i), dot);
      dot = row16_sum(dot);
    }
    sc[u] = valid[u] ? dot : -INFINITY;
  }
  const float m_new = fmaxf(m, fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])));
  if (m_new == -INFINITY) return;
  const float alpha = exp2f(m - m_new);
  l *= alpha;
#pragma unroll
  for (int i = 0; i < C; ++i) acc[i] *= alpha;
  if constexpr (kBf16) {
#pragma unroll
    for (int u = 0; u < 4; u += 2) {
      const float p0 = exp2f(sc[u] - m_new), p1 = exp2f(sc[u + 1] - m_new);
      l += p0 + p1;
      const bf16x2_t pp = {(__bf16)p0, (__bf16)p1};
      const uint32_t pk = __builtin_bit_cast(uint32_t, pp);
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
      for (int i = 0; i < C; ++i) acc[i] = fmaf(pu, vv[u].get(i), acc[i]);
    }
  }
  m = m_new;
}

// In-place exclusive prefix of two count arrays at once: on entry a[b + 1] and
// c[b + 1] hold row b's counts (a[0] = c[0] = 0); on exit they hold the sums
// over rows before b + 1. Each of the 256 threads owns a contiguous run of
// rows; one wave-level scan of the run totals and the wave totals in LDS give
// every run its offset.
CDB_DEVICE void block_prefix2(int* a, int* c, int B, int tid, int wave, int lane, int* wave_tot) {
  const int per = (B + 255) >> 8;
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
    wave_tot[4 + wave] = ic;
  }
  __syncthreads();
  int ra = ia - sa, rc = ic - sc;
  for (int w = 0; w < wave; ++w) {
    ra += wave_tot[w];
    rc += wave_tot[4 + w];
  }
  for (int b = lo; b < hi; ++b) {
    ra += a[b + 1];
    rc += c[b + 1];
    a[b + 1] = ra;
    c[b + 1] = rc;
  }
  __syncthreads();
}

template <typename T, int D>
__global__ void __launch_bounds__(256) paged_decode_kernel(DecodeParams P) {
  constexpr int C = Layout<D>::kChunk;
  // Per-row metadata, loaded once per workgroup: new-token position (-1 when the
  // row gets no work), cache layer, block-table row and the split prefix sum.
  __shared__ int row_pos[kMaxRowsLds];
  __shared__ int row_where[kMaxRowsLds];  // cache layer | block-table row << 16
  __shared__ int split_prefix[kMaxRowsLds + 1];  // splits of rows before b (partial layout)
  __shared__ int full_prefix[kMaxRowsLds + 1];   // full-length splits of rows before b
  __shared__ int wave_pages[4];
  __shared__ int wave_tot[8];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int slot = lane >> 4;
  const int chunk = lane & 15;
  const int B = P.num_rows;
  const int bs_log2 = P.block_size_log2;
  const int block_size = 1 << bs_log2;
  const int head_groups = (P.num_heads + 3) >> 2;

  // Pages each served row reads (including the new token's page).
  int pages = 0;
  for (int b = tid; b < B; b += blockDim.x) {
    const int p = P.seqlens[b];
    const int trow = P.table_row ? P.table_row[b] : b;
    const bool ok = row_valid(P, b, p) && trow >= 0 && trow <= 0xffff;
    row_pos[b] = ok ? p : -1;
    row_where[b] = (P.cache_layer0 + (P.cache_layer ? P.cache_layer[b] : 0)) | (trow << 16);
    pages += ok ? ((p + block_size) >> bs_log2) : 0;
  }
  for (int m = 32; m >= 1; m >>= 1) pages += __shfl_xor(pages, m, 64);
  if (lane == 0) wave_pages[wave] = pages;
  __syncthreads();
  const int total_pages = wave_pages[0] + wave_pages[1] + wave_pages[2] + wave_pages[3];

  int split_pages = P.split_pages;
  if (split_pages <= 0) {
    const int64_t target = 4ll * gridDim.x;
    const int64_t want = ((int64_t)total_pages * head_groups + target - 1) / target;
    split_pages = P.min_split_pages;
    while (split_pages < want && split_pages < P.max_split_pages) split_pages <<= 1;
    // The split count is at most total_pages / split_pages + B: coarsen until the partials fit.
    while ((int64_t)total_pages / split_pages + B > P.partial_capacity && split_pages < (1 << 20)) split_pages <<= 1;
  }
  const int split_tokens = split_pages << bs_log2;

  for (int b = tid; b < B; b += blockDim.x) {
    const int p = row_pos[b];
    const int n = p >= 0 ? (p + split_tokens) / split_tokens : 0;
    split_prefix[b + 1] = n;
    full_prefix[b + 1] = n > 0 ? n - 1 : 0;
  }
  if (tid == 0) split_prefix[0] = full_prefix[0] = 0;
  __syncthreads();
  block_prefix2(split_prefix, full_prefix, B, tid, wave, lane, wave_tot);
  const int total_splits = split_prefix[B];
  const int total_full = full_prefix[B];
  // Items: every full-length split first (row order), then each row's last,
  // shorter split, so that round-robin assignment hands out the long items
  // first and the tail of the grid is made of short ones.
  const int total_items = (total_full + B) * head_groups;
  const bool overflow = total_splits > P.partial_capacity;

  if (blockIdx.x == 0) {
    for (int b = tid; b <= B; b += blockDim.x) P.header[1 + b] = split_prefix[b];
    if (tid == 0) P.header[0] = overflow ? -1 : split_tokens;
  }

  // Rows without work: padding rows read as zeros, rows out of range as NaN.
  for (int b = blockIdx.x; b < B; b += gridDim.x) {
    if (split_prefix[b + 1] != split_prefix[b]) continue;
    const float fill = P.seqlens[b] < 0 ? 0.f : __builtin_nanf("");
    T* o = static_cast<T*>(P.out) + (int64_t)b * P.num_heads * D;
    for (int e = tid; e < P.num_heads * D; e += blockDim.x) Elem<T>::store(o + e, fill);
  }

  const T* q_all = static_cast<const T*>(P.q);
  const T* k_new_all = static_cast<const T*>(P.k_new);
  const T* v_new_all = static_cast<const T*>(P.v_new);
  const int kv_group = P.num_heads / P.num_kv_heads;
  const int64_t row_elems = (int64_t)P.num_kv_heads * D;  // one cached token, all kv heads

  for (int item = blockIdx.x; item < total_items; item += gridDim.x) {
    const int g = item / head_groups;
    const int hg = item - g * head_groups;
    const int h = hg * 4 + wave;
    if (h >= P.num_heads) continue;  // wave-uniform; no block-level sync inside the item loop
    int b, s;
    if (g < total_full) {
      int lo = 0, hi = B - 1;  // row owning full split g: largest b with full_prefix[b] <= g
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (full_prefix[mid] <= g) lo = mid; else hi = mid - 1;
      }
      b = lo;
      s = g - full_prefix[b];
    } else {
      b = g - total_full;
      if (row_pos[b] < 0) continue;  // padding or out-of-range row: no work
      s = split_prefix[b + 1] - split_prefix[b] - 1;
    }
    const int split_global = split_prefix[b] + s;
    const int nsplit = split_prefix[b + 1] - split_prefix[b];
    if (nsplit > 1 && overflow) continue;  // the merge kernel writes NaN for this row
    const int p = row_pos[b];
    const int kvh = h / kv_group;
    const int where = row_where[b];
    const int layer = where & 0xffff;
    T* k_base = static_cast<T*>(P.k_pool) + (int64_t)layer * P.layer_stride;
    T* v_base = static_cast<T*>(P.v_pool) + (int64_t)layer * P.layer_stride;
    const int32_t* table = P.block_table + (int64_t)((uint32_t)where >> 16) * P.table_width;

    const int t_begin = s * split_tokens;
    const bool last_split = s == nsplit - 1;
    const int t_end = last_split ? p : t_begin + split_tokens;  // cached tokens only; p is handled below

    int win_base = t_begin >> bs_log2;
    int window = load_page_window(table, win_base, P.table_width, lane);
    // Keeps the pages of the step starting at t0 inside the window (wave-uniform).
    auto cover = [&](int t0) {
      if (((t0 + 15) >> bs_log2) - win_base >= 64) {
        win_base = t0 >> bs_log2;
        window = load_page_window(table, win_base, P.table_width, lane);
      }
    };

    // Issue the first step's loads before the query rotation so they overlap it.
    Vec<T, C> ka[4], va[4], kb[4], vb[4];
    bool vla[4], vlb[4];
    if (t_begin < t_end) {
      cover(t_begin);
      load_step<T, D>(P, window, win_base, k_base, v_base, t_begin, t_end, slot, chunk, kvh, bs_log2, row_elems,
                      ka, va, vla);
    }

    // The new token's key and value are needed only after the loop; issue their
    // loads now so they are not one more round trip at the end of the item.
    RawChunk<T, D> k_raw;
    Vec<T, C> vn;
    if (last_split) {
      load_raw<T, D>(P, k_new_all + (int64_t)b * P.kv_stride + (int64_t)kvh * D, chunk, k_raw);
      vn.load(v_new_all + (int64_t)b * P.kv_stride + (int64_t)kvh * D + chunk * C);
    }

    QueryReg<T, D> q;
    load_rotated<T, D>(P, q_all + (int64_t)b * P.q_stride + (int64_t)h * D,
                       P.q_bias ? static_cast<const T*>(P.q_bias) + (int64_t)h * D : nullptr, p, chunk, q.f);
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int w = 0; w < C / 2; ++w)
        q.p[w] = (uint32_t)f32_to_bf16(q.f[2 * w]) | ((uint32_t)f32_to_bf16(q.f[2 * w + 1]) << 16);
    } else {
#pragma unroll
      for (int i = 0; i < C; ++i) q.f[i] *= P.scale_log2;
    }

    float m = -INFINITY, l = 0.f;
    float acc[C];
#pragma unroll
    for (int i = 0; i < C; ++i) acc[i] = 0.f;

    // Two-stage pipeline: the next step's K/V loads are in flight while this step is reduced.
    for (int t0 = t_begin; t0 < t_end; t0 += 32) {
      const bool second = t0 + 16 < t_end;
      if (second) {
        cover(t0 + 16);
        load_step<T, D>(P, window, win_base, k_base, v_base, t0 + 16, t_end, slot, chunk, kvh, bs_log2,
                        row_elems, kb, vb, vlb);
      }
      attend_step<T, D>(q, P.scale_log2, ka, va, vla, m, l, acc);
      if (!second) break;
      if (t0 + 32 < t_end) {
        cover(t0 + 32);
        load_step<T, D>(P, window, win_base, k_base, v_base, t0 + 32, t_end, slot, chunk, kvh, bs_log2,
                        row_elems, ka, va, vla);
      }
      attend_step<T, D>(q, P.scale_log2, kb, vb, vlb, m, l, acc);
    }

    if (last_split) {
      // The new token: rotate and append its key/value, then attend to it from registers.
      float kr[C];
      const T* kbias = P.k_bias ? static_cast<const T*>(P.k_bias) + (int64_t)kvh * D : nullptr;
      rotate_raw<T, D>(P, k_raw, kbias, p, chunk, kr);
      const int p_page = p >> bs_log2;
      const int new_blk = p_page - win_base < 64 ? __builtin_amdgcn_readlane(window, p_page - win_base)
                                                 : table[p_page];
      if (slot == 0 && h % kv_group == 0 && new_blk >= 0 && new_blk < P.pool_blocks) {
        const int64_t row = ((int64_t)new_blk << bs_log2) + (p & (block_size - 1));
        const int64_t off = row * row_elems + (int64_t)kvh * D + chunk * C;
        Vec<T, C> kw;
#pragma unroll
        for (int i = 0; i < C; ++i) kw.set(i, kr[i]);
        kw.store(k_base + off);
        vn.store(v_base + off);
      }
      float dot = 0.f;
#pragma unroll
      for (int i = 0; i < C; ++i) dot = fmaf(q.f[i], kr[i], dot);
      dot = row16_sum(dot);
      if constexpr (sizeof(T) == 2) dot *= P.scale_log2;
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

    if (slot != 0) continue;
    if (nsplit == 1) {
      T* out_row = static_cast<T*>(P.out) + ((int64_t)b * P.num_heads + h) * D;
      const float inv = 1.f / l;
      Vec<T, C> o;
#pragma unroll
      for (int i = 0; i < C; ++i) o.set(i, acc[i] * inv);
      o.store(out_row + chunk * C);
    } else {
      float* part = P.partial + ((int64_t)split_global * P.num_heads + h) * (D + 2);
#pragma unroll
      for (int i = 0; i < C; ++i) part[chunk * C + i] = acc[i];
      if (chunk == 0) {
        part[D] = m_all;
        part[D + 1] = l;
      }
    }
  }
}

// Merge the split partials of every (row, head) whose row has more than one
// split; one wave per (row, head). Reads the split prefix the decode kernel
// left in the workspace header. Lane s holds split s's (max, sum) so the
// global max and the denominator are wave reductions; the accumulators are
// read eight splits at a time so their loads are in flight together.
template <typename T, int D>
__global__ void __launch_bounds__(256) decode_merge_kernel(DecodeParams P) {
  const int lane = threadIdx.x & 63;
  const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (w >= P.num_rows * P.num_heads) return;
  const int b = w / P.num_heads;
  const int h = w - b * P.num_heads;
  const int first = P.header[1 + b];
  const int nsplit = P.header[2 + b] - first;
  if (nsplit <= 1) return;
  T* out_row = static_cast<T*>(P.out) + ((int64_t)b * P.num_heads + h) * D;
  if (P.header[0] < 0) {
    for (int d = lane; d < D; d += 64) Elem<T>::store(out_row + d, __builtin_nanf(""));
    return;
  }
  const int64_t stride = (int64_t)P.num_heads * (D + 2);
  const float* part = P.partial + (int64_t)first * stride + (int64_t)h * (D + 2);
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
        a0[j] = ok && d0 < D ? ps[d0] : 0.f;
        a1[j] = ok && d1 < D ? ps[d1] : 0.f;
      }
    };
    // The first eight splits' accumulators are read with the (max, sum) pairs, so
    // their loads overlap instead of waiting for the wave reductions.
    load_group(0);
    float ms = -INFINITY, ls = 0.f;
    if (lane < cnt) {
      ms = chunk_part[lane * stride + D];
      ls = chunk_part[lane * stride + D + 1];
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

}  // namespace cdb

using namespace cdb;

// The fixed scratch of cdb_paged_decode_attention_noalloc: a file-scope device array, one copy per
// GPU, alive until the process ends. Host code never passes the array's name to a kernel (on the
// host it is only a stand-in symbol); scratch_address() resolves each device's own address once,
// with that device current, and the launches use that address.
static __device__ __align__(256) unsigned char scratch[CDB_DECODE_SCRATCH_BYTES];

namespace {

int g_num_cus = 0;

// Resident workgroups per CU for a kernel, cached per instantiation. The
// persistent decode kernel assigns items by blockIdx stride, so its grid must
// not exceed what is resident at once.
template <typename Kernel>
int resident_blocks_per_cu(Kernel kernel) {
  static int cached = 0;
  if (cached == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, 256, 0) != hipSuccess || n <= 0) n = 1;
    cached = n;
  }
  return cached;
}

int ilog2_exact(int x) {
  if (x <= 0 || (x & (x - 1))) return -1;
  int r = 0;
  while ((1 << r) < x) ++r;
  return r;
}

int64_t header_bytes(int64_t num_rows) { return ((num_rows + 2) * 4 + 255) / 256 * 256; }

template <typename T, int D>
int launch_decode(const DecodeParams& P, int num_cus, hipStream_t stream) {
  const int grid = num_cus * resident_blocks_per_cu(paged_decode_kernel<T, D>);
  hipLaunchKernelGGL((paged_decode_kernel<T, D>), dim3(grid), dim3(256), 0, stream, P);
  if (hipGetLastError() != hipSuccess) return CDB_ERR_HIP;
  const int64_t waves = (int64_t)P.num_rows * P.num_heads;
  hipLaunchKernelGGL((decode_merge_kernel<T, D>), dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, stream, P);
  return hipGetLastError() == hipSuccess ? CDB_OK : CDB_ERR_HIP;
}

template <typename T>
int dispatch_dim(const DecodeParams& P, int head_dim, int num_cus, hipStream_t stream) {
  switch (head_dim) {
    case 64: return launch_decode<T, 64>(P, num_cus, stream);
    case 96: return launch_decode<T, 96>(P, num_cus, stream);
    case 128: return launch_decode<T, 128>(P, num_cus, stream);
    default: return CDB_ERR_UNSUPPORTED;
  }
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
                     int32_t min_split_pages, int32_t max_split_pages, float scale, int64_t q_stride,
                     int64_t kv_stride, int32_t dtype, hipStream_t stream);

}  // namespace

extern "C" {

int64_t cdb_paged_decode_workspace_bytes(int32_t num_rows, int32_t num_heads, int32_t head_dim,
                                         int32_t max_seqlen, int32_t block_size, int32_t split_pages) {
  if (num_rows < 0 || num_heads <= 0 || head_dim <= 0 || max_seqlen <= 0 || block_size <= 0 || split_pages <= 0)
    return -1;
  const int64_t split_tokens = (int64_t)split_pages * block_size;
  const int64_t max_splits = (max_seqlen + split_tokens - 1) / split_tokens + 1;
  return header_bytes(num_rows) +
         (int64_t)num_rows * max_splits * num_heads * (head_dim + 2) * (int64_t)sizeof(float);
}

int cdb_paged_decode_attention(const void* q, const void* k_new, const void* v_new, void* k_pool, void* v_pool,
                               int64_t layer_stride, int32_t num_cache_layers, int64_t pool_blocks,
                               const int32_t* cache_layer, int32_t cache_layer0,
                               const int32_t* block_table, const int32_t* table_row, int32_t table_width,
                               const int32_t* seqlens, const float* rope_cos, const float* rope_sin,
                               int32_t rope_style, int32_t max_positions, const void* q_bias, const void* k_bias,
                               void* out, void* workspace, int64_t workspace_bytes, int32_t num_rows,
                               int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                               int32_t split_pages, int32_t min_split_pages, int32_t max_split_pages, float scale,
                               int64_t q_stride, int64_t kv_stride, int32_t dtype, hipStream_t stream) {
  return decode_attention(q, k_new, v_new, k_pool, v_pool, layer_stride, num_cache_layers, pool_blocks, cache_layer,
                          cache_layer0, block_table, table_row, table_width, seqlens, rope_cos, rope_sin, rope_style,
                          max_positions, q_bias, k_bias, out, workspace, workspace_bytes, num_rows, num_heads,
                          num_kv_heads, head_dim, block_size, split_pages, min_split_pages, max_split_pages, scale,
                          q_stride, kv_stride, dtype, stream);
}

int cdb_paged_decode_attention_noalloc(const void* q, const void* k_new, const void* v_new, void* k_pool,
                                       void* v_pool, int64_t layer_stride, int32_t num_cache_layers,
                                       int64_t pool_blocks, const int32_t* cache_layer, int32_t cache_layer0,
                                       const int32_t* block_table, const int32_t* table_row, int32_t table_width,
                                       const int32_t* seqlens, const float* rope_cos, const float* rope_sin,
                                       int32_t rope_style, int32_t max_positions, const void* q_bias,
                                       const void* k_bias, void* out, int32_t num_rows, int32_t num_heads,
                                       int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                       int32_t split_pages, int32_t min_split_pages, int32_t max_split_pages,
                                       float scale, int64_t q_stride, int64_t kv_stride, int32_t dtype,
                                       hipStream_t stream) {
  if (num_rows == 0) return CDB_OK;
  if (num_rows < 0 || num_heads <= 0 || head_dim <= 0) return CDB_ERR_SHAPE;
  // The kernel lengthens splits until the partials fit, down to one split per row: the scratch
  // must hold the header and one partial per row.
  const int64_t need = header_bytes(num_rows) + (int64_t)num_rows * num_heads * (head_dim + 2) * (int64_t)sizeof(float);
  if (need > CDB_DECODE_SCRATCH_BYTES) return CDB_ERR_CAPACITY;
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != CDB_OK) return rc;
  return decode_attention(q, k_new, v_new, k_pool, v_pool, layer_stride, num_cache_layers, pool_blocks, cache_layer,
                          cache_layer0, block_table, table_row, table_width, seqlens, rope_cos, rope_sin, rope_style,
                          max_positions, q_bias, k_bias, out, ws, CDB_DECODE_SCRATCH_BYTES, num_rows, num_heads,
                          num_kv_heads, head_dim, block_size, split_pages, min_split_pages, max_split_pages, scale,
                          q_stride, kv_stride, dtype, stream);
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
                     int32_t min_split_pages, int32_t max_split_pages, float scale, int64_t q_stride,
                     int64_t kv_stride, int32_t dtype, hipStream_t stream) {
  if (num_rows == 0) return CDB_OK;
  if (!q || !k_new || !v_new || !k_pool || !v_pool || !block_table || !seqlens || !out || !workspace)
    return CDB_ERR_NULL;
  if (num_rows < 0 || num_rows > kMaxRowsLds || num_heads <= 0 || num_kv_heads <= 0 ||
      num_heads % num_kv_heads != 0 || table_width <= 0)
    return CDB_ERR_SHAPE;
  if (split_pages <= 0 && (min_split_pages <= 0 || max_split_pages < min_split_pages ||
                           (min_split_pages & (min_split_pages - 1))))
    return CDB_ERR_SHAPE;
  const int bs_log2 = ilog2_exact(block_size);
  if (bs_log2 < 0) return CDB_ERR_SHAPE;
  if (rope_style < 0 || rope_style > 2) return CDB_ERR_SHAPE;
  if (rope_style != 0 && (!rope_cos || !rope_sin || max_positions <= 0)) return CDB_ERR_NULL;
  if (rope_style == 1 && head_dim != 128 && head_dim != 64 && head_dim != 96) return CDB_ERR_UNSUPPORTED;
  if (dtype != CDB_DTYPE_F32 && dtype != CDB_DTYPE_BF16) return CDB_ERR_UNSUPPORTED;
  // Split-half rotation pairs chunk c with chunk c ^ 8, i.e. D/2 = 8 chunks.
  if (rope_style == 1 && (head_dim / 16) * 8 != head_dim / 2) return CDB_ERR_UNSUPPORTED;
  if (num_cache_layers <= 0 || num_cache_layers > 0xffff || pool_blocks <= 0 || layer_stride < 0)
    return CDB_ERR_SHAPE;
  const int64_t header = header_bytes(num_rows);
  if (workspace_bytes < header) return CDB_ERR_CAPACITY;

  DecodeParams P;
  P.q = q; P.k_new = k_new; P.v_new = v_new; P.k_pool = k_pool; P.v_pool = v_pool;
  P.block_table = block_table; P.table_row = table_row; P.seqlens = seqlens; P.cache_layer = cache_layer;
  P.rope_cos = rope_style ? rope_cos : nullptr; P.rope_sin = rope_style ? rope_sin : nullptr;
  P.q_bias = q_bias; P.k_bias = k_bias; P.out = out;
  P.header = static_cast<int32_t*>(workspace);
  P.partial = reinterpret_cast<float*>(static_cast<char*>(workspace) + header);
  P.layer_stride = layer_stride; P.cache_layer0 = cache_layer0;
  P.q_stride = q_stride > 0 ? q_stride : (int64_t)num_heads * head_dim;
  P.kv_stride = kv_stride > 0 ? kv_stride : (int64_t)num_kv_heads * head_dim;
  if (P.q_stride < (int64_t)num_heads * head_dim || P.kv_stride < (int64_t)num_kv_heads * head_dim) return CDB_ERR_SHAPE;
  P.num_rows = num_rows; P.num_heads = num_heads; P.num_kv_heads = num_kv_heads;
  P.table_width = table_width; P.block_size_log2 = bs_log2; P.split_pages = split_pages;
  P.rope_style = rope_style; P.max_positions = max_positions;
  P.num_cache_layers = num_cache_layers; P.pool_blocks = pool_blocks;
  P.min_split_pages = min_split_pages; P.max_split_pages = max_split_pages;
  P.partial_capacity = (workspace_bytes - header) / ((int64_t)num_heads * (head_dim + 2) * (int64_t)sizeof(float));
  P.scale_log2 = scale * 1.4426950408889634f;

  if (g_num_cus == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return CDB_ERR_HIP;
    if (hipDeviceGetAttribute(&g_num_cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return CDB_ERR_HIP;
  }
  if (dtype == CDB_DTYPE_F32) return dispatch_dim<float>(P, head_dim, g_num_cus, stream);
  return dispatch_dim<bf16_t>(P, head_dim, g_num_cus, stream);
}

}  // namespace
