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
//   * a row's context is cut into splits of `split_pages` pages;
//   * a work item is (row, split, group of 4 query heads); one workgroup of
//     4 waves takes an item, wave w owning query head 4*g + w;
//   * workgroups are persistent: workgroup i processes items i, i+G, ...,
//     so the grid does not depend on the context lengths (graph-capturable);
//   * each workgroup rebuilds the per-row split prefix sum in LDS and maps an
//     item to its row by binary search.
// Inside a wave, lane = 16 * slot + chunk: the 16 lanes of a DPP row split the
// head dimension into 16 chunks and the 4 rows ("slots") take interleaved
// tokens. q.k is reduced across a row with four DPP rotate-adds; each slot keeps
// its own online-softmax state, merged across slots at the end.
// A row with one split writes its normalized output directly; otherwise the
// split's (unnormalized acc, max, sum) goes to the workspace and
// cdb_decode_combine merges the splits.

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
  float scale_log2;             // softmax scale * log2(e)
};

constexpr int kMaxRowsLds = 2048;

template <int D> struct Layout {
  static constexpr int kChunk = D / 16;  // elements per lane
  static_assert(D % 16 == 0, "head_dim must be a multiple of 16");
};

// A row is served when its new-token position fits the block table and the
// RoPE table and its cache layer exists. Rows failing this get no work and a
// NaN output (the combine kernel writes it); padding rows (p < 0) get zeros.
CDB_DEVICE bool row_valid(const DecodeParams& P, int b, int p) {
  if (p < 0) return false;
  if ((int64_t)p >= ((int64_t)P.table_width << P.block_size_log2)) return false;
  if (P.rope_cos != nullptr && p >= P.max_positions) return false;
  const int layer = P.cache_layer0 + (P.cache_layer ? P.cache_layer[b] : 0);
  return layer >= 0 && layer < P.num_cache_layers;
}

// Number of splits of row b (0 for padding and invalid rows).
CDB_DEVICE int row_splits(const DecodeParams& P, int b, int split_tokens) {
  const int p = P.seqlens[b];
  return row_valid(P, b, p) ? (p + split_tokens) / split_tokens : 0;
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
    // q*cos + rotate_half(q)*sin with cos/sin = cat(f, f); each op rounded.
#pragma unroll
    for (int i = 0; i < C; ++i) {
      const int d = chunk * C + i;
      const int f = d < half ? d : d - half;
      const float rot = d < half ? -partner[i] : partner[i];
      const float a = Elem<T>::round(mul_rn(own[i], cos_row[f]));
      const float b = Elem<T>::round(mul_rn(rot, sin_row[f]));
      out[i] = Elem<T>::round(add_rn(a, b));
    }
  } else {
    // Interleaved (even, odd) pairs rotated in fp32, rounded once at the end.
#pragma unroll
    for (int i = 0; i < C; i += 2) {
      const int f = (chunk * C + i) >> 1;
      const float c = cos_row[f], s = sin_row[f];
      const float x0 = own[i], x1 = own[i + 1];
      out[i] = Elem<T>::round(sub_rn(mul_rn(x0, c), mul_rn(x1, s)));
      out[i + 1] = Elem<T>::round(add_rn(mul_rn(x1, c), mul_rn(x0, s)));
    }
  }
}

// Load this lane's chunk of a [rows, heads, D] vector (plus its split-half
// partner chunk), add an optional per-head bias, and rotate.
template <typename T, int D>
CDB_DEVICE void load_rotated(const DecodeParams& P, const T* base, const T* bias, int pos, int chunk, float* out) {
  constexpr int C = Layout<D>::kChunk;
  float own[C], partner[C];
  Vec<T, C> v;
  v.load(base + chunk * C);
#pragma unroll
  for (int i = 0; i < C; ++i) own[i] = v.get(i);
  const bool split_half = P.rope_style == 1 && P.rope_cos != nullptr;
  if (split_half) {
    v.load(base + (chunk ^ 8) * C);
#pragma unroll
    for (int i = 0; i < C; ++i) partner[i] = v.get(i);
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
__global__ void __launch_bounds__(256) paged_decode_kernel(DecodeParams P) {
  constexpr int C = Layout<D>::kChunk;
  __shared__ int split_prefix[kMaxRowsLds + 1];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int slot = lane >> 4;
  const int chunk = lane & 15;
  const int B = P.num_rows;
  const int bs_log2 = P.block_size_log2;
  const int block_size = 1 << bs_log2;
  const int split_tokens = P.split_pages << bs_log2;
  const int head_groups = (P.num_heads + 3) >> 2;

  // Per-row split counts -> exclusive prefix in LDS (row-major item order).
  for (int b = tid; b < B; b += blockDim.x) split_prefix[b + 1] = row_splits(P, b, split_tokens);
  if (tid == 0) split_prefix[0] = 0;
  __syncthreads();
  // Sequential scan by wave 0 in 64-wide pieces with a carry (B <= 4096).
  if (wave == 0) {
    int carry = 0;
    for (int base = 0; base < B; base += 64) {
      int idx = base + lane;
      int v = idx < B ? split_prefix[idx + 1] : 0;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        int n = __shfl_up(v, off, 64);
        if (lane >= off) v += n;
      }
      if (idx < B) split_prefix[idx + 1] = v + carry;
      carry += __shfl(v, 63, 64);
    }
  }
  __syncthreads();
  const int total_splits = split_prefix[B];
  const int total_items = total_splits * head_groups;
  // Rows with several splits need workspace; if it is too small, the combine
  // kernel flags those rows with NaN instead of this kernel writing past it.
  const bool partial_ok = total_splits <= P.partial_capacity;

  const T* q_all = static_cast<const T*>(P.q);
  const T* k_new_all = static_cast<const T*>(P.k_new);
  const T* v_new_all = static_cast<const T*>(P.v_new);
  const int kv_group = P.num_heads / P.num_kv_heads;
  const int64_t row_elems = (int64_t)P.num_kv_heads * D;  // one cached token, all kv heads

  for (int item = blockIdx.x; item < total_items; item += gridDim.x) {
    const int split_global = item / head_groups;
    const int hg = item - split_global * head_groups;
    const int h = hg * 4 + wave;
    if (h >= P.num_heads) continue;  // wave-uniform; no block-level sync inside the item loop
    // Row owning this split: largest b with split_prefix[b] <= split_global.
    int lo = 0, hi = B - 1;
    while (lo < hi) {
      int mid = (lo + hi + 1) >> 1;
      if (split_prefix[mid] <= split_global) lo = mid; else hi = mid - 1;
    }
    const int b = lo;
    const int s = split_global - split_prefix[b];
    const int nsplit = split_prefix[b + 1] - split_prefix[b];
    const int p = P.seqlens[b];
    const int kvh = h / kv_group;
    const int layer = P.cache_layer0 + (P.cache_layer ? P.cache_layer[b] : 0);
    T* k_base = static_cast<T*>(P.k_pool) + (int64_t)layer * P.layer_stride;
    T* v_base = static_cast<T*>(P.v_pool) + (int64_t)layer * P.layer_stride;
    const int32_t* table = P.block_table + (int64_t)(P.table_row ? P.table_row[b] : b) * P.table_width;

    // Rotated query chunk, pre-scaled into the log2 domain.
    float q[C];
    load_rotated<T, D>(P, q_all + (int64_t)b * P.q_stride + (int64_t)h * D,
                       P.q_bias ? static_cast<const T*>(P.q_bias) + (int64_t)h * D : nullptr, p, chunk, q);
#pragma unroll
    for (int i = 0; i < C; ++i) q[i] *= P.scale_log2;

    const int t_begin = s * split_tokens;
    const bool last_split = s == nsplit - 1;
    const int t_end = last_split ? p : t_begin + split_tokens;  // cached tokens only; p handled below

    float m = -INFINITY, l = 0.f;
    float acc[C];
#pragma unroll
    for (int i = 0; i < C; ++i) acc[i] = 0.f;

    // Stream the cached tokens four at a time per slot (16 per wave step).
    for (int t0 = t_begin; t0 < t_end; t0 += 16) {
      float sc[4];
      bool valid[4];
      Vec<T, C> kv[4], vv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int t = t0 + 4 * u + slot;
        const int blk = t < t_end ? table[t >> bs_log2] : -1;
        valid[u] = blk >= 0 && blk < P.pool_blocks;
        if (valid[u]) {
          const int64_t row = (int64_t)blk * block_size + (t & (block_size - 1));
          const int64_t off = row * row_elems + (int64_t)kvh * D + chunk * C;
          kv[u].load(k_base + off);
          vv[u].load(v_base + off);
        } else {
          // Masked tokens get zero weight; zero their registers so 0 * garbage cannot make a NaN.
#pragma unroll
          for (int w = 0; w < Vec<T, C>::kWords; ++w) kv[u].w[w] = vv[u].w[w] = 0u;
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        float dot = 0.f;
#pragma unroll
        for (int i = 0; i < C; ++i) dot = fmaf(q[i], kv[u].get(i), dot);
        dot = row16_sum(dot);
        sc[u] = valid[u] ? dot : -INFINITY;
      }
      const float mloc = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
      const float m_new = fmaxf(m, mloc);
      if (m_new != -INFINITY) {
        const float alpha = exp2f(m - m_new);
        l *= alpha;
#pragma unroll
        for (int i = 0; i < C; ++i) acc[i] *= alpha;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float pu = exp2f(sc[u] - m_new);
          l += pu;
#pragma unroll
          for (int i = 0; i < C; ++i) acc[i] = fmaf(pu, vv[u].get(i), acc[i]);
        }
        m = m_new;
      }
    }

    if (last_split) {
      // The new token: rotate and append its key/value, then attend to it from registers.
      float kr[C];
      const T* kbias = P.k_bias ? static_cast<const T*>(P.k_bias) + (int64_t)kvh * D : nullptr;
      load_rotated<T, D>(P, k_new_all + (int64_t)b * P.kv_stride + (int64_t)kvh * D, kbias, p, chunk, kr);
      Vec<T, C> vn;
      vn.load(v_new_all + (int64_t)b * P.kv_stride + (int64_t)kvh * D + chunk * C);
      const int new_blk = table[p >> bs_log2];
      if (slot == 0 && h % kv_group == 0 && new_blk >= 0 && new_blk < P.pool_blocks) {
        const int blk = new_blk;
        const int64_t row = (int64_t)blk * block_size + (p & (block_size - 1));
        const int64_t off = row * row_elems + (int64_t)kvh * D + chunk * C;
        Vec<T, C> kw;
#pragma unroll
        for (int i = 0; i < C; ++i) kw.set(i, kr[i]);
        kw.store(k_base + off);
        vn.store(v_base + off);
      }
      float dot = 0.f;
#pragma unroll
      for (int i = 0; i < C; ++i) dot = fmaf(q[i], kr[i], dot);
      dot = row16_sum(dot);
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
      if (nsplit == 1) {
        const float inv = 1.f / l;
        Vec<T, C> o;
#pragma unroll
        for (int i = 0; i < C; ++i) o.set(i, acc[i] * inv);
        o.store(static_cast<T*>(P.out) + ((int64_t)b * P.num_heads + h) * D + chunk * C);
      } else if (partial_ok) {
        float* part = P.partial + ((int64_t)(split_prefix[b] + s) * P.num_heads + h) * (D + 2);
#pragma unroll
        for (int i = 0; i < C; ++i) part[chunk * C + i] = acc[i];
        if (chunk == 0) {
          part[D] = m_all;
          part[D + 1] = l;
        }
      }
    }
  }
}

// Merge per-split partials of rows with more than one split; zero padding rows.
// One wave per (row, head).
template <typename T, int D>
__global__ void __launch_bounds__(256) decode_combine_kernel(DecodeParams P) {
  const int lane = threadIdx.x & 63;
  const int wave_global = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int B = P.num_rows;
  if (wave_global >= B * P.num_heads) return;
  const int b = wave_global / P.num_heads;
  const int h = wave_global - b * P.num_heads;
  const int split_tokens = P.split_pages << P.block_size_log2;
  const int p = P.seqlens[b];
  const int nsplit = row_splits(P, b, split_tokens);
  T* out = static_cast<T*>(P.out) + ((int64_t)b * P.num_heads + h) * D;
  if (nsplit == 1) return;
  if (nsplit == 0) {
    const float fill = p < 0 ? 0.f : __builtin_nanf("");
    for (int d = lane; d < D; d += 64) Elem<T>::store(out + d, fill);
    return;
  }
  // Exclusive prefix of split counts over rows before b, and the total.
  int first = 0, total = 0;
  for (int r = lane; r < B; r += 64) {
    const int n = row_splits(P, r, split_tokens);
    if (r < b) first += n;
    total += n;
  }
  for (int m = 32; m >= 1; m >>= 1) {
    first += __shfl_xor(first, m, 64);
    total += __shfl_xor(total, m, 64);
  }
  if (total > P.partial_capacity) {
    for (int d = lane; d < D; d += 64) Elem<T>::store(out + d, __builtin_nanf(""));
    return;
  }
  const float* part = P.partial + ((int64_t)first * P.num_heads + h) * (D + 2);
  const int64_t stride = (int64_t)P.num_heads * (D + 2);
  float m_all = -INFINITY;
  for (int s = 0; s < nsplit; ++s) m_all = fmaxf(m_all, part[s * stride + D]);
  float num0 = 0.f, num1 = 0.f, den = 0.f;
  const int d0 = lane, d1 = lane + 64;
  for (int s = 0; s < nsplit; ++s) {
    const float* ps = part + s * stride;
    const float w = exp2f(ps[D] - m_all);
    den = fmaf(w, ps[D + 1], den);
    if (d0 < D) num0 = fmaf(w, ps[d0], num0);
    if (d1 < D) num1 = fmaf(w, ps[d1], num1);
  }
  const float inv = 1.f / den;
  if (d0 < D) Elem<T>::store(out + d0, num0 * inv);
  if (d1 < D) Elem<T>::store(out + d1, num1 * inv);
}

}  // namespace cdb

using namespace cdb;

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

template <typename T, int D>
int launch_decode(const DecodeParams& P, int num_cus, hipStream_t stream) {
  const int grid = num_cus * resident_blocks_per_cu(paged_decode_kernel<T, D>);
  hipLaunchKernelGGL((paged_decode_kernel<T, D>), dim3(grid), dim3(256), 0, stream, P);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return CDB_ERR_HIP;
  const int waves = P.num_rows * P.num_heads;
  const int blocks = (waves + 3) / 4;
  if (blocks > 0) {
    hipLaunchKernelGGL((decode_combine_kernel<T, D>), dim3(blocks), dim3(256), 0, stream, P);
    e = hipGetLastError();
    if (e != hipSuccess) return CDB_ERR_HIP;
  }
  return CDB_OK;
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

}  // namespace

extern "C" {

int64_t cdb_paged_decode_workspace_bytes(int32_t num_rows, int32_t num_heads, int32_t head_dim,
                                         int32_t max_seqlen, int32_t block_size, int32_t split_pages) {
  if (num_rows < 0 || num_heads <= 0 || head_dim <= 0 || max_seqlen <= 0 || block_size <= 0 || split_pages <= 0)
    return -1;
  const int64_t split_tokens = (int64_t)split_pages * block_size;
  const int64_t max_splits = (max_seqlen + split_tokens - 1) / split_tokens;
  return (int64_t)num_rows * max_splits * num_heads * (head_dim + 2) * (int64_t)sizeof(float);
}

int cdb_paged_decode_attention(const void* q, const void* k_new, const void* v_new, void* k_pool, void* v_pool,
                               int64_t layer_stride, int32_t num_cache_layers, int64_t pool_blocks,
                               const int32_t* cache_layer, int32_t cache_layer0,
                               const int32_t* block_table, const int32_t* table_row, int32_t table_width,
                               const int32_t* seqlens, const float* rope_cos, const float* rope_sin,
                               int32_t rope_style, int32_t max_positions, const void* q_bias, const void* k_bias,
                               void* out, void* workspace, int64_t workspace_bytes, int32_t num_rows,
                               int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                               int32_t split_pages, float scale, int64_t q_stride, int64_t kv_stride,
                               int32_t dtype, hipStream_t stream) {
  if (num_rows == 0) return CDB_OK;
  if (!q || !k_new || !v_new || !k_pool || !v_pool || !block_table || !seqlens || !out) return CDB_ERR_NULL;
  if (num_rows < 0 || num_rows > kMaxRowsLds || num_heads <= 0 || num_kv_heads <= 0 ||
      num_heads % num_kv_heads != 0 || table_width <= 0 || split_pages <= 0)
    return CDB_ERR_SHAPE;
  const int bs_log2 = ilog2_exact(block_size);
  if (bs_log2 < 0) return CDB_ERR_SHAPE;
  if (rope_style < 0 || rope_style > 2) return CDB_ERR_SHAPE;
  if (rope_style != 0 && (!rope_cos || !rope_sin || max_positions <= 0)) return CDB_ERR_NULL;
  if (rope_style == 1 && head_dim != 128 && head_dim != 64 && head_dim != 96) return CDB_ERR_UNSUPPORTED;
  if (dtype != CDB_DTYPE_F32 && dtype != CDB_DTYPE_BF16) return CDB_ERR_UNSUPPORTED;
  // Split-half rotation pairs chunk c with chunk c ^ 8, i.e. D/2 = 8 chunks.
  if (rope_style == 1 && (head_dim / 16) * 8 != head_dim / 2) return CDB_ERR_UNSUPPORTED;
  if (workspace == nullptr && workspace_bytes != 0) return CDB_ERR_NULL;
  if (num_cache_layers <= 0 || pool_blocks <= 0 || layer_stride < 0) return CDB_ERR_SHAPE;

  DecodeParams P;
  P.q = q; P.k_new = k_new; P.v_new = v_new; P.k_pool = k_pool; P.v_pool = v_pool;
  P.block_table = block_table; P.table_row = table_row; P.seqlens = seqlens; P.cache_layer = cache_layer;
  P.rope_cos = rope_style ? rope_cos : nullptr; P.rope_sin = rope_style ? rope_sin : nullptr;
  P.q_bias = q_bias; P.k_bias = k_bias; P.out = out; P.partial = static_cast<float*>(workspace);
  P.layer_stride = layer_stride; P.cache_layer0 = cache_layer0;
  P.q_stride = q_stride > 0 ? q_stride : (int64_t)num_heads * head_dim;
  P.kv_stride = kv_stride > 0 ? kv_stride : (int64_t)num_kv_heads * head_dim;
  if (P.q_stride < (int64_t)num_heads * head_dim || P.kv_stride < (int64_t)num_kv_heads * head_dim) return CDB_ERR_SHAPE;
  P.num_rows = num_rows; P.num_heads = num_heads; P.num_kv_heads = num_kv_heads;
  P.table_width = table_width; P.block_size_log2 = bs_log2; P.split_pages = split_pages;
  P.rope_style = rope_style; P.max_positions = max_positions;
  P.num_cache_layers = num_cache_layers; P.pool_blocks = pool_blocks;
  P.partial_capacity = workspace_bytes / ((int64_t)num_heads * (head_dim + 2) * (int64_t)sizeof(float));
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

}  // extern "C"
