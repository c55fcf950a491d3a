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
// Tiling: a workgroup (4 waves) owns 64 query tokens of one sequence and one
// query head; wave w owns 16 of them. Keys are streamed in blocks of 32:
// the block's K (row-major) and V (transposed, [D][key]) are staged in LDS
// once per workgroup and shared by the 4 waves.
//   S^T = K Q^T   -> MFMA with A = K rows from LDS, B = the wave's Q^T
//   O^T += V^T P^T -> MFMA with A = V^T from LDS, B = P^T straight from the
//                     S^T accumulators (same lane layout: lane l owns query l%16)
// Computing the transposed products keeps every lane's softmax statistics
// (query l%16) aligned with the accumulators it rescales, so no cross-lane
// moves are needed beyond the 4-lane max/sum over key groups.
// Along the contraction dimension the MFMA k-index is bound to head-dim or key
// indices by a permutation shared by both operands, which lets each lane read
// 16 contiguous bytes.
//   bf16: __builtin_amdgcn_mfma_f32_16x16x32_bf16 (8 elements per lane per op)
//   fp32: __builtin_amdgcn_mfma_f32_16x16x4f32    (1 element per lane per op)

#include "cdb_common.h"
#include "../../include/cdb_amd.h"

namespace cdb {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

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
  void* out;                   // [T, H, D]
  int64_t pool_blocks;
  int32_t num_tiles, num_seqs;
  int32_t num_heads, num_kv_heads, table_width, block_size_log2;
  float scale_log2;
};

constexpr int kKeys = 32;      // keys per block
constexpr int kQTile = 64;     // queries per workgroup
constexpr int kLdsPages = 1024;  // block ids kept in LDS per workgroup (longer prefixes read the table)

template <typename T> struct Mfma;

template <> struct Mfma<bf16_t> {
  static constexpr int kVec = 8;  // elements per 16-byte lane vector == elements per MFMA k-slice
  // acc += A(lane vector) x B(lane vector)
  static CDB_DEVICE f32x4_t mma(const Vec<bf16_t, 8>& a, const Vec<bf16_t, 8>& b, f32x4_t acc) {
    bf16x8_t av, bv;
    __builtin_memcpy(&av, a.w, 16);
    __builtin_memcpy(&bv, b.w, 16);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc, 0, 0, 0);
  }
};

template <> struct Mfma<float> {
  static constexpr int kVec = 4;
  // A 16-byte lane vector holds 4 k-slices; one fp32 MFMA per element.
  static CDB_DEVICE f32x4_t mma(const Vec<float, 4>& a, const Vec<float, 4>& b, f32x4_t acc) {
#pragma unroll
    for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.get(i), b.get(i), acc, 0, 0, 0);
    return acc;
  }
};

template <typename T, int D>
__global__ void __launch_bounds__(256) prefill_attention_kernel(PrefillParams P) {
  constexpr int V = Mfma<T>::kVec;          // elements per lane vector
  constexpr int kChunks = D / (4 * V);      // 16-byte vectors per lane across D
  constexpr int kDTiles = D / 16;           // output tiles of 16 head-dim rows
  constexpr int kKPad = V;                  // LDS row padding (elements) against bank conflicts
  // V^T rows of 36 elements: the transposed stores below (one dword per key pair,
  // 16 pairs x 4 d-chunks per wave) then land in 64 distinct banks.
  constexpr int kVtPad = 4;
  static_assert(D % (4 * V) == 0, "head_dim must split into 4 lane groups of 16-byte vectors");

  // Two key blocks in flight: the next block's K/V is loaded into registers
  // while the current one is multiplied, then stored to the other buffer.
  __shared__ __attribute__((aligned(16))) T k_lds[2][kKeys][D + kKPad];
  __shared__ __attribute__((aligned(16))) T vt_lds[2][D][kKeys + kVtPad];
  __shared__ int page_lds[kLdsPages];

  // One workgroup per (tile, head), heads fastest: the host lists the tiles
  // longest prefix first, so the heaviest workgroups of every head start first.
  const int tile = blockIdx.x / P.num_heads;
  const int h = blockIdx.x - tile * P.num_heads;
  if (tile >= P.num_tiles) return;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int col = lane & 15;   // query (S^T/O^T column) or key/d row for A operands
  const int grp = lane >> 4;   // k-group

  const int s = P.tile_seq[tile];
  const int q_begin = P.cu_q[s];
  const int q_len = P.cu_q[s + 1] - q_begin;
  const int past = P.past[s];
  const int tile_q0 = P.tile_q0[tile];
  const int kvh = h / (P.num_heads / P.num_kv_heads);
  const int32_t* table = P.block_table + (int64_t)P.table_row[s] * P.table_width;
  const int bs_log2 = P.block_size_log2;
  const int bs_mask = (1 << bs_log2) - 1;
  const int64_t row_elems = (int64_t)P.num_kv_heads * D;
  const T* k_base = static_cast<const T*>(P.k_pool) + (int64_t)P.layer * P.layer_stride;
  const T* v_base = static_cast<const T*>(P.v_pool) + (int64_t)P.layer * P.layer_stride;

  // This lane's query (column of S^T / O^T).
  const int q_local = tile_q0 + wave * 16 + col;
  const bool q_valid = q_local < q_len;
  const int q_pos = past + q_local;

  // Q^T operand: lane holds query `col`, vector chunk c covers d in [c*4V + grp*V, +V).
  Vec<T, V> qv[kChunks];
  {
    const T* qrow = static_cast<const T*>(P.q) + ((int64_t)(q_begin + (q_valid ? q_local : 0)) * P.num_heads + h) * D;
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      if (q_valid) {
        qv[c].load(qrow + c * 4 * V + grp * V);
      } else {
#pragma unroll
        for (int w = 0; w < Vec<T, V>::kWords; ++w) qv[c].w[w] = 0u;
      }
    }
  }

  f32x4_t o[kDTiles];
#pragma unroll
  for (int j = 0; j < kDTiles; ++j) o[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;

  // Keys needed by the workgroup: up to the last valid query's position.
  const int last_local = min(tile_q0 + kQTile, q_len) - 1;
  const int key_end = past + last_local + 1;
  const int wave_last = min(tile_q0 + wave * 16 + 15, q_len - 1);  // last query of this wave
  const int wave_key_end = past + wave_last + 1;

  // Block ids of the prefix, once per workgroup.
  const int key_pages = (key_end + bs_mask) >> bs_log2;
  const bool pages_in_lds = key_pages <= kLdsPages;
  if (pages_in_lds) {
    for (int i = tid; i < key_pages; i += 256) page_lds[i] = i < P.table_width ? table[i] : -1;
  }
  __syncthreads();

  // Staging work: (16-byte d-chunk, key pair) combinations. A thread loads both
  // keys of its pair so it can store V^T one key pair per dword (bf16) or per
  // 8 bytes (fp32) instead of one element at a time.
  constexpr int kChunksPerKey = D / V;
  constexpr int kPairs = kKeys / 2;
  constexpr int kCombos = kChunksPerKey * kPairs;
  constexpr int kCombosPerThread = (kCombos + 255) / 256;
  Vec<T, V> kreg[2 * kCombosPerThread], vreg[2 * kCombosPerThread];
  // Global -> registers for keys kb .. kb+31 (zeros past key_end or for unmapped pages).
  auto load_block = [&](int kb) {
#pragma unroll
    for (int r = 0; r < kCombosPerThread; ++r) {
      const int combo = tid + r * 256;
      const int c = combo / kPairs;
      const int pair = combo - c * kPairs;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int kp = kb + 2 * pair + e;
        int blk = -1;
        if (combo < kCombos && kp < key_end) {
          const int page = kp >> bs_log2;
          blk = pages_in_lds ? page_lds[page] : (page < P.table_width ? table[page] : -1);
        }
        Vec<T, V>& kr = kreg[2 * r + e];
        Vec<T, V>& vr = vreg[2 * r + e];
        if (blk >= 0 && blk < P.pool_blocks) {
          const int64_t off =
              ((int64_t)blk * (bs_mask + 1) + (kp & bs_mask)) * row_elems + (int64_t)kvh * D + c * V;
          kr.load(k_base + off);
          vr.load(v_base + off);
        } else {
#pragma unroll
          for (int w = 0; w < Vec<T, V>::kWords; ++w) kr.w[w] = vr.w[w] = 0u;
        }
      }
    }
  };
  // Registers -> LDS buffer `buf`: K row-major, V transposed.
  auto store_block = [&](int buf) {
#pragma unroll
    for (int r = 0; r < kCombosPerThread; ++r) {
      const int combo = tid + r * 256;
      if (combo >= kCombos) continue;
      const int c = combo / kPairs;
      const int pair = combo - c * kPairs;
      kreg[2 * r].store(&k_lds[buf][2 * pair][c * V]);
      kreg[2 * r + 1].store(&k_lds[buf][2 * pair + 1][c * V]);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        if constexpr (sizeof(T) == 2) {
          const uint32_t a = vreg[2 * r].w[i >> 1], b = vreg[2 * r + 1].w[i >> 1];
          // (key 2*pair, key 2*pair+1) of element i: low or high halves of a and b.
          const uint32_t packed = (i & 1) ? __builtin_amdgcn_perm(b, a, 0x07060302u)
                                          : __builtin_amdgcn_perm(b, a, 0x05040100u);
          *reinterpret_cast<uint32_t*>(&vt_lds[buf][c * V + i][2 * pair]) = packed;
        } else {
          *reinterpret_cast<uint2*>(&vt_lds[buf][c * V + i][2 * pair]) =
              make_uint2(vreg[2 * r].w[i], vreg[2 * r + 1].w[i]);
        }
      }
    }
  };

  if (key_end > 0) {
    load_block(0);
    store_block(0);
  }
  __syncthreads();

  int buf = 0;
  for (int kb = 0; kb < key_end; kb += kKeys, buf ^= 1) {
    const bool has_next = kb + kKeys < key_end;
    if (has_next) load_block(kb + kKeys);  // in flight during this block's products

    if (kb < wave_key_end) {
      // S^T for key tiles 0 (keys kb..kb+15) and 1 (kb+16..kb+31): lane holds keys 4*grp+i.
      f32x4_t st[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        st[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < kChunks; ++c) {
          Vec<T, V> kv;
          kv.load(&k_lds[buf][t * 16 + col][c * 4 * V + grp * V]);
          st[t] = Mfma<T>::mma(kv, qv[c], st[t]);
        }
      }
      // Scale, causal mask, online softmax over this lane's 8 keys and its 3 peers.
      // Only blocks that reach past the wave's first query or the last key need
      // the mask (wave-uniform test).
      const bool masked = kb + kKeys - 1 > past + tile_q0 + wave * 16 || kb + kKeys > key_end;
      float sv[2][4];
      float mloc = -INFINITY;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int kp = kb + t * 16 + grp * 4 + i;
          const float x = st[t][i] * P.scale_log2;
          sv[t][i] = !masked || (kp <= q_pos && kp < key_end) ? x : -INFINITY;
          mloc = fmaxf(mloc, sv[t][i]);
        }
      mloc = fmaxf(mloc, shfl_xor_f32(mloc, 16));
      mloc = fmaxf(mloc, shfl_xor_f32(mloc, 32));
      // Key 0 is visible to every query (its position is >= 0 and key_end > 0), so
      // from the first block on m_new is finite: exp2(-inf) = 0 covers the first
      // rescale and every masked key without special cases. v_exp_f32 (exp2 with
      // results below 2^-126 flushed to 0) is enough for softmax weights.
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

      if constexpr (sizeof(T) == 2) {
        // One bf16 MFMA covers 32 keys: k-slice grp*8 + i <-> key (i < 4 ? 4*grp + i : 16 + 4*grp + i - 4).
        Vec<T, 8> pb;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pb.set(i, p[0][i]);
          pb.set(4 + i, p[1][i]);
        }
#pragma unroll
        for (int j = 0; j < kDTiles; ++j) {
          Vec<T, 8> va;
          const T* vrow = &vt_lds[buf][j * 16 + col][0];
          const uint2 lo = *reinterpret_cast<const uint2*>(vrow + 4 * grp);
          const uint2 hi = *reinterpret_cast<const uint2*>(vrow + 16 + 4 * grp);
          va.w[0] = lo.x; va.w[1] = lo.y; va.w[2] = hi.x; va.w[3] = hi.y;
          o[j] = Mfma<T>::mma(va, pb, o[j]);
        }
      } else {
        // fp32: per tile t, MFMA i uses k-slice grp <-> key 16*t + 4*grp + i.
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          Vec<T, 4> pb;
#pragma unroll
          for (int i = 0; i < 4; ++i) pb.set(i, p[t][i]);
#pragma unroll
          for (int j = 0; j < kDTiles; ++j) {
            Vec<T, 4> va;
            va.load(&vt_lds[buf][j * 16 + col][16 * t + 4 * grp]);
            o[j] = Mfma<T>::mma(va, pb, o[j]);
          }
        }
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
  T* orow = static_cast<T*>(P.out) + ((int64_t)(q_begin + q_local) * P.num_heads + h) * D;
#pragma unroll
  for (int j = 0; j < kDTiles; ++j) {
    Vec<T, 4> ov;
#pragma unroll
    for (int i = 0; i < 4; ++i) ov.set(i, o[j][i] * inv);
    ov.store(orow + j * 16 + 4 * grp);
  }
}

}  // namespace cdb

using namespace cdb;

extern "C" {

int cdb_prefill_attention(const void* q, const void* k_pool, const void* v_pool, int64_t layer_stride, int32_t layer,
                          int32_t num_cache_layers, int64_t pool_blocks, const int32_t* block_table, const int32_t* table_row,
                          int32_t table_width, const int32_t* cu_q, const int32_t* past, int32_t num_seqs,
                          const int32_t* tile_seq, const int32_t* tile_q0, int32_t num_tiles, void* out,
                          int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale,
                          int32_t dtype, hipStream_t stream) {
  if (num_tiles == 0) return CDB_OK;
  if (!q || !k_pool || !v_pool || !block_table || !table_row || !cu_q || !past || !tile_seq || !tile_q0 || !out)
    return CDB_ERR_NULL;
  if (num_tiles < 0 || num_seqs <= 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads ||
      table_width <= 0 || layer < 0 || layer >= num_cache_layers || pool_blocks <= 0)
    return CDB_ERR_SHAPE;
  int bs_log2 = 0;
  while ((1 << bs_log2) < block_size) ++bs_log2;
  if (block_size <= 0 || (1 << bs_log2) != block_size) return CDB_ERR_SHAPE;
  PrefillParams P{q, k_pool, v_pool, layer_stride, layer, block_table, table_row, cu_q, past, tile_seq, tile_q0, out,
                  pool_blocks, num_tiles, num_seqs, num_heads, num_kv_heads, table_width, bs_log2,
                  scale * 1.4426950408889634f};
  if ((int64_t)num_tiles * num_heads > 0x7fffffff) return CDB_ERR_SHAPE;
  const dim3 grid((unsigned)(num_tiles * num_heads));
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, dim3(256), 0, stream, P);
    return hipGetLastError() == hipSuccess ? CDB_OK : CDB_ERR_HIP;
  };
  if (dtype == CDB_DTYPE_BF16) {
    switch (head_dim) {
      case 64: return go(prefill_attention_kernel<bf16_t, 64>);
      case 96: return go(prefill_attention_kernel<bf16_t, 96>);
      case 128: return go(prefill_attention_kernel<bf16_t, 128>);
      default: return CDB_ERR_UNSUPPORTED;
    }
  }
  if (dtype == CDB_DTYPE_F32) {
    switch (head_dim) {
      case 64: return go(prefill_attention_kernel<float, 64>);
      case 96: return go(prefill_attention_kernel<float, 96>);
      case 128: return go(prefill_attention_kernel<float, 128>);
      default: return CDB_ERR_UNSUPPORTED;
    }
  }
  return CDB_ERR_UNSUPPORTED;
}

}  // extern "C"
