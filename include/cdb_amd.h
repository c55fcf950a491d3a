/* C ABI of the MI355X continuous-depth-batching decode-step kernels.
 *
 * Every entry point takes plain device pointers, element counts and an
 * explicit hipStream_t, allocates nothing, and returns CDB_OK (0) or a
 * negative CDB_ERR_* code; no C++ exception crosses this boundary. All
 * buffers are owned by the caller, so every call is capturable into a HIP
 * graph. Tensors are dense and row-major; "dtype" selects fp32 or bf16
 * storage for activations, weights and KV pages (accumulation is fp32).
 *
 * Paged KV layout: cache layer l's keys are the rows of
 *   k_pool + l * layer_stride  viewed as [pool_blocks * block_size, Hkv, D]
 * (values likewise from v_pool), which is the reference's per-layer cache
 * tensor shape (continuous_batching/cache.py:131-144). Token position t of a
 * sequence lives at row block_table[t / block_size] * block_size + t % block_size
 * (continuous_batching/cache_manager.py:190-213).
 */
#ifndef CDB_AMD_H_
#define CDB_AMD_H_

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  CDB_OK = 0,
  CDB_ERR_NULL = -1,        /* a required pointer is null */
  CDB_ERR_SHAPE = -2,       /* an extent or stride is out of range */
  CDB_ERR_UNSUPPORTED = -3, /* dtype / head_dim combination not compiled */
  CDB_ERR_HIP = -4,         /* a HIP launch failed */
  CDB_ERR_CAPACITY = -5     /* a caller buffer is too small */
};

enum { CDB_DTYPE_F32 = 0, CDB_DTYPE_BF16 = 1 };

/* Bytes of fp32 workspace cdb_paged_decode_attention needs for num_rows rows
 * whose new-token positions are all < max_seqlen. Returns -1 on bad input. */
int64_t cdb_paged_decode_workspace_bytes(int32_t num_rows, int32_t num_heads, int32_t head_dim, int32_t max_seqlen,
                                         int32_t block_size, int32_t split_pages);

/* Mixed-depth paged decode attention with fused RoPE and KV append.
 *
 * Replaces flash_attn_with_kvcache as called by the reference's paged decode
 * branch (transformers integrations/flash_paged.py:100-147, reached from
 * ouro/modeling_ouro.py:407-428 and huginn/modeling_huginn.py:275-300), plus
 * the RoPE applied just before it (ouro/modeling_ouro.py:179-204 split-half,
 * rope_style 1; huginn/modeling_huginn.py:178-196 interleaved, rope_style 2).
 *
 * q [B,H,D], k_new/v_new [B,Hkv,D] are the un-rotated projections of the
 * batch's new tokens. Row b appends its rotated key and its value at position
 * p = seqlens[b] (FA's cache_seqlens) in cache layer cache_layer[b] (or
 * cache_layer0 for every row when cache_layer is null) and attends over
 * positions 0..p with softmax scale `scale`. seqlens[b] < 0 marks a padding
 * row (no KV write, zero output). Block table row for batch row b is
 * table_row[b] (or b when null). rope_cos/rope_sin are [max_positions, D/2]
 * fp32 tables holding the values the reference's rotary module produces
 * (rounded to the model dtype for Ouro); rope_style 0 applies no rotation.
 * q_bias [H,D] / k_bias [Hkv,D] are optional pre-rotation biases (Huginn's
 * qk_bias). Rows whose position or cache layer is out of range get a NaN
 * output and no KV write. workspace: cdb_paged_decode_workspace_bytes(...). */
int cdb_paged_decode_attention(const void* q, const void* k_new, const void* v_new, void* k_pool, void* v_pool,
                               int64_t layer_stride, int32_t num_cache_layers, int64_t pool_blocks,
                               const int32_t* cache_layer, int32_t cache_layer0, const int32_t* block_table,
                               const int32_t* table_row, int32_t table_width, const int32_t* seqlens,
                               const float* rope_cos, const float* rope_sin, int32_t rope_style,
                               int32_t max_positions, const void* q_bias, const void* k_bias, void* out,
                               void* workspace, int64_t workspace_bytes, int32_t num_rows, int32_t num_heads,
                               int32_t num_kv_heads, int32_t head_dim, int32_t block_size, int32_t split_pages,
                               float scale, int32_t dtype, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* CDB_AMD_H_ */
