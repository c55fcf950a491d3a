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

/* Bytes of decode workspace for num_rows rows whose new-token positions are
 * all < max_seqlen with chunks of split_pages pages: an int32 header of
 * num_rows + 2 entries padded to 256 bytes, 1 KiB of work-queue counters and
 * one int32 arrival counter per (row, head) padded to 256 bytes (all zeroed by
 * the plan), then per chunk a 64-byte descriptor and an
 * fp32 partial of num_heads * (head_dim + 2) floats. A smaller workspace is
 * legal as long as it holds the header and one chunk per row: the plan then
 * lengthens the chunks until they fit. Returns -1 on bad input. */
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
 * p = seqlens[b] (FA's cache_seqlens) in cache layer cache_layer0 + cache_layer[b]
 * (cache_layer0 alone when cache_layer is null: a row's KV slot offset
 * slot*num_layers goes in cache_layer, the physical layer in cache_layer0) and attends over
 * positions 0..p with softmax scale `scale`. seqlens[b] < 0 marks a padding
 * row (no KV write, zero output). Block table row for batch row b is
 * table_row[b] (or b when null). rope_cos/rope_sin are [max_positions, D/2]
 * fp32 tables holding the values the reference's rotary module produces
 * (rounded to the model dtype for Ouro); rope_style 0 applies no rotation.
 * q_bias [H,D] / k_bias [Hkv,D] are optional pre-rotation biases (Huginn's
 * qk_bias). Rows whose position or cache layer is out of range get a NaN
 * output and no KV write. workspace: cdb_paged_decode_workspace_bytes(...).
 * q_stride / kv_stride: elements between consecutive rows of q and of
 * k_new/v_new (0 = dense), so q, k and v may be column slices of one fused
 * QKV projection output.
 * Each row's context is cut into chunks of split_pages pages (min_split_pages
 * when split_pages <= 0), processed in parallel and merged in chunk order, so a row's output does not
 * depend on which other rows share the launch. Only a workspace too small for
 * the launch's chunks lengthens them.
 * Returns CDB_ERR_CAPACITY when workspace_bytes cannot hold the header and one
 * chunk per row. */
int cdb_paged_decode_attention(const void* q, const void* k_new, const void* v_new, void* k_pool, void* v_pool,
                               int64_t layer_stride, int32_t num_cache_layers, int64_t pool_blocks,
                               const int32_t* cache_layer, int32_t cache_layer0, const int32_t* block_table,
                               const int32_t* table_row, int32_t table_width, const int32_t* seqlens,
                               const float* rope_cos, const float* rope_sin, int32_t rope_style,
                               int32_t max_positions, const void* q_bias, const void* k_bias, void* out,
                               void* workspace, int64_t workspace_bytes, int32_t num_rows, int32_t num_heads,
                               int32_t num_kv_heads, int32_t head_dim, int32_t block_size, int32_t split_pages,
                               int32_t min_split_pages, float scale,
                               int64_t q_stride, int64_t kv_stride, int32_t dtype, hipStream_t stream);

/* Stages of cdb_paged_decode_attention_staged. */
enum { CDB_DECODE_STAGE_PLAN = 1, CDB_DECODE_STAGE_ATTEND = 2 };

/* cdb_paged_decode_attention in two stages, for a batch whose rows run through
 * several layers with the same positions (seqlens), table rows (table_row) and
 * cache-layer offsets (cache_layer), as the reference's recurrent stage runs its
 * rows through every layer of the loop block (continuous_api.py:1171-1183,
 * ouro/modeling_ouro.py:407-428). CDB_DECODE_STAGE_PLAN writes the chunk plan
 * of those rows into the workspace; CDB_DECODE_STAGE_ATTEND runs attention and
 * the merge from the plan last written to this workspace, which must describe
 * the same rows (only cache_layer0, q/k/v, the pools and out may differ).
 * stages = PLAN | ATTEND is cdb_paged_decode_attention. Arguments and errors as
 * cdb_paged_decode_attention; CDB_ERR_SHAPE for any other stages value. */
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
                                      hipStream_t stream);

/* No counterpart in the reference. cdb_paged_decode_attention for callers that cannot allocate
 * device memory: code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc. Same arguments and results without the workspace: the split header and partials
 * live in a fixed device array of CDB_DECODE_SCRATCH_BYTES per GPU (resolved once per device,
 * held until the process ends). The call allocates nothing and frees nothing. Nothing in the
 * scratch must start at zero: each call's plan writes its header and zeroes its counters before
 * the decode kernel reads them.
 * Every call on one GPU shares that GPU's array, so calls that overlap on one GPU (two streams,
 * or two threads) race; serialize them. Returns CDB_ERR_CAPACITY when the header plus one
 * chunk per row (a 64-byte descriptor and num_heads * (head_dim + 2) floats) exceeds the
 * scratch after the header, queue counters and arrival counters (at 16 heads x 128: more than
 * 1984 rows); a smaller surplus only lengthens the chunks. */
#define CDB_DECODE_SCRATCH_BYTES ((int64_t)16 << 20)
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
                                       hipStream_t stream);

/* Fused RMSNorm sandwich over rows of `width` elements.
 *   norm_w(x) = R(w * R(x * rsqrt(mean(x^2) + eps)))  (R rounds to the storage dtype)
 *   mode 0: out_h = norm_a(x)
 *   mode 1: out_h = R(residual + norm_a(x)); out_y = norm_b(out_h)   (Ouro layer,
 *           ouro/modeling_ouro.py:445-450 and :481-502)
 *   mode 2: out_h = norm_a(R(residual + x)); out_y = norm_b(out_h)   (Huginn block,
 *           huginn/modeling_huginn.py:141-146 and :335-338)
 * out_y is written only when w_b is non-null. out_h may alias x or residual. */
int cdb_rmsnorm_fused(const void* x, const void* residual, const void* w_a, const void* w_b, void* out_h,
                      void* out_y, int64_t rows, int32_t width, int32_t mode, float eps_a, float eps_b,
                      int32_t dtype, hipStream_t stream);

/* cdb_rmsnorm_fused with x given as the fp32 split-K partials of the projection
 * that produces it (cdb_linear_parts): x[r, c] = R(sum over s < splits, in
 * order, of x_parts[s, r, c]), the projection's own rounded output, then the
 * same modes as cdb_rmsnorm_fused. bf16 only; x_parts [splits, rows, width]
 * contiguous and 16-byte aligned; 1 <= splits <= 64. Fuses the O and down
 * projections' outputs into the residual norms that follow them
 * (ouro/modeling_ouro.py:168,431 into :445-450 and :481-502). */
int cdb_rmsnorm_fused_parts(const float* x_parts, int32_t splits, const void* residual, const void* w_a,
                            const void* w_b, void* out_h, void* out_y, int64_t rows, int32_t width, int32_t mode,
                            float eps_a, float eps_b, int32_t dtype, hipStream_t stream);

/* out[r, :] = R(R(silu(g)) * u) for gate_up[r] = [g | u] of 2*width elements
 * (ouro/modeling_ouro.py:167-169, huginn/modeling_huginn.py:314-316). */
int cdb_silu_mul(const void* gate_up, void* out, int64_t rows, int32_t width, int32_t dtype, hipStream_t stream);

/* Row gather/scatter: dst[dst_index[i]] = src[src_index[i]] for i < rows, rows of
 * row_bytes bytes (a multiple of 4). A null index means the identity; a negative
 * (or out-of-range) src index writes zeros; a negative dst index skips the row.
 * Replaces the hidden-bank index_select/index_copy_ of cdb/model_runner.py:685-693,
 * :559 and :1101, the embedding lookup of cdb/adapters/ouro.py:199-212 and the
 * device token gather of cdb/model_runner.py:439-457. */
int cdb_copy_rows(const void* src, const int64_t* src_index, int64_t src_rows, void* dst, const int64_t* dst_index,
                  int64_t dst_rows, int64_t rows, int64_t row_bytes, hipStream_t stream);

/* Block-table cell updates with the count in device memory: table[idx[i]] = val[i]
 * for i < min(*count, capacity); cells outside [0, cells) are skipped. It lets a
 * launch's metadata upload carry the table cells its rows' new blocks changed and
 * a captured graph apply them, in place of a separate flush
 * (the block-table refresh of cdb/cache.py:115-144, cache_manager.py:72-90). */
int cdb_table_updates(int32_t* table, int64_t cells, const int64_t* idx, const int32_t* val, const int32_t* count,
                      int32_t capacity, hipStream_t stream);

/* Exit routing of one recurrent launch on the device, in launch order: writes
 * lists = [n_exit, n_stay, the n_exit exiting rows, the n_stay staying rows], the
 * rows being indices into the launch (exit_flags[r] != 0: row r leaves for the coda)
 * and rows with a negative bank slot (padding) in neither list. Replaces the
 * per-row routing pass over the launch's decisions on the synchronous horizon
 * (cdb/continuous_api.py:1171-1183 after cdb/model_runner.py:694-699,796-821):
 * exiting rows go to the coda queue in this order, staying rows back to the head of
 * the depth queue in this order. lists holds 2 + rows ints. */
int cdb_route_compact(const uint8_t* exit_flags, const int64_t* bank_slots, int32_t rows, int32_t* lists,
                      hipStream_t stream);

/* Greedy sampling: out[r] = first index of the maximum of logits[r, :vocab]
 * (torch.argmax semantics incl. NaN; cdb/model_runner.py:1062,1105). */
int cdb_argmax(const void* logits, int64_t* out, int64_t rows, int32_t vocab, int32_t dtype, hipStream_t stream);

/* Early-exit gate and decision for one recurrent launch.
 * kind 0: signal[b] = R(hidden[b] . weight + bias) -- Ouro's Linear(E,1) gate
 *         (cdb/adapters/ouro.py:286-291);
 * kind 1: signal[b] = R(||hidden[b] - prev[b]|| / max(||hidden[b]||, 1e-9)) --
 *         Huginn's latent difference (huginn/exit_gates.py:33-40).
 * The token policy state (fp64 cdf/survival, pending signal) is kept in arrays
 * of state_capacity entries indexed by state_index[b] (< 0: padding row). The
 * decision follows cdb/exit_policy.py:150-169 and cdb/continuous_api.py:1671-1724:
 * forced exit at step max_steps-1; a replayed synthetic_depth[b] >= 0 exits at
 * step >= depth; otherwise, with has_threshold, rule 0 accumulates the sigmoid
 * hazard (rounded to the storage dtype when round_hazard) into the cdf and exits
 * when cdf >= threshold, rule 1 exits when signal < threshold, both only once
 * step+1 >= min_steps. delayed=1 decides on the previous launch's signal
 * (DecisionHorizon.OFFSET_ONE). exit_flags[b] is 1 for an exit. */
int cdb_exit_gate(const void* hidden, const void* prev, const void* weight, const void* bias, void* signal,
                  double* cdf, double* survival, float* pending, int64_t state_capacity, const int64_t* state_index,
                  const int32_t* steps, const int32_t* synthetic_depth, uint8_t* exit_flags, int64_t rows,
                  int32_t width, int32_t kind, int32_t rule, int32_t delayed, int32_t round_hazard,
                  int32_t min_steps, int32_t max_steps, double threshold, int32_t has_threshold, int32_t dtype,
                  hipStream_t stream);

/* Reset the gate state of n fresh tokens: cdf 0, survival 1, no pending signal
 * (TokenExitPolicyState(), cdb/exit_policy.py:43-48). */
int cdb_exit_gate_reset(double* cdf, double* survival, float* pending, int64_t state_capacity,
                        const int64_t* index, int64_t n, hipStream_t stream);

/* Copy-on-exit KV propagation (kv_policy "last_exited"): for token i at pool row
 * rows[i] that exited at KV slot exit_slot[i], copy its K and V rows from cache
 * layer layer_base + exit_slot*core_layers + l to layer_base + s*core_layers + l
 * for every core layer l and every deeper slot s < num_slots
 * (cdb/continuous_api.py:1225-1245, kv_cache_policy.py:235-258, cdb/cache.py:105-113). */
int cdb_exit_kv_copy(void* k_pool, void* v_pool, int64_t layer_stride, int64_t pool_rows, int32_t num_kv_heads,
                     int32_t head_dim, const int64_t* rows, const int32_t* exit_slot, int64_t n, int32_t layer_base,
                     int32_t core_layers, int32_t num_slots, int32_t dtype, hipStream_t stream);

/* Prefill-side RoPE + paged KV write for T tokens: q_out = rotate(q [+ q_bias]);
 * rotate(k [+ k_bias]) and v are written to cache layer `layer` at pool rows
 * rows[t] (negative rows write nothing). Replaces the write half of
 * PagedAttentionCache.update (continuous_batching/cache.py:284-318) and the
 * RoPE before it. q, k and v may be column slices of one fused QKV output:
 * q_stride / kv_stride are the elements between consecutive tokens (0: dense
 * [T, H, D] / [T, Hkv, D]); q_out is dense. */
int cdb_rope_kv_write(const void* q, const void* k, const void* v, void* q_out, void* k_pool, void* v_pool,
                      int64_t layer_stride, int32_t layer, const int64_t* rows, int64_t pool_rows,
                      const int32_t* positions, const float* rope_cos, const float* rope_sin, int32_t rope_style,
                      int32_t max_positions, const void* q_bias, const void* k_bias, int64_t tokens,
                      int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int64_t q_stride, int64_t kv_stride,
                      int32_t dtype, hipStream_t stream);

/* Varlen causal prefill attention over the paged pool on MFMA tiles.
 * Replaces flash_attn_varlen_func as the reference's prefill calls it after
 * the chunk's KV write (continuous_batching/prefill_graph.py:265-309,
 * transformers integrations/flash_paged.py:62-86). Sequence s has query tokens
 * cu_q[s] .. cu_q[s+1]-1 of q [T,H,D] (already rotated) at positions
 * past[s] + i; each attends to positions 0..(its own) of cache layer `layer`
 * through block-table row table_row[s]. The chunk's own K/V must already be in
 * the pool. Work is split into tiles of 128 query tokens: tile n covers
 * sequence tile_seq[n], queries tile_q0[n] .. +127. out is [T,H,D]. scale must
 * be positive and finite (CDB_ERR_SHAPE otherwise). */
int cdb_prefill_attention(const void* q, const void* k_pool, const void* v_pool, int64_t layer_stride, int32_t layer,
                          int32_t num_cache_layers, int64_t pool_blocks, const int32_t* block_table,
                          const int32_t* table_row, int32_t table_width, const int32_t* cu_q, const int32_t* past,
                          int32_t num_seqs, const int32_t* tile_seq, const int32_t* tile_q0, int32_t num_tiles,
                          void* out, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                          float scale, int32_t dtype, hipStream_t stream);

/* Bytes of the partial-result buffer cdb_prefill_attention_split needs for
 * num_slots partial slots (-1 for invalid arguments). No reference counterpart:
 * a sizing helper for the split work list below. */
int64_t cdb_prefill_partial_bytes(int32_t num_slots, int32_t num_heads, int32_t head_dim);

/* cdb_prefill_attention with the key range of long tiles split over several
 * workgroups (bf16 only), so that one long sequence does not set the length of
 * the whole launch; same operation, same outputs up to fp32 rounding of the
 * merge. Replaces the same flash_attn_varlen_func call as cdb_prefill_attention
 * (continuous_batching/prefill_graph.py:265-309).
 *   items  [num_items][4] int32: (sequence, first query of the 128-query tile,
 *          first key block | end key block << 16 (blocks of 32 keys),
 *          partial slot, or -1 for a whole tile written straight to out).
 *          A part must not start past the tile's first query position.
 *   merges [num_merges][4] int32: (sequence, first query, first slot, parts):
 *          the parts of one split tile occupy consecutive slots.
 *   partials: cdb_prefill_partial_bytes(num_slots, ...) bytes of scratch.
 * Two launches on `stream`: the tiles and parts, then the merge. */
int cdb_prefill_attention_split(const void* q, const void* k_pool, const void* v_pool, int64_t layer_stride,
                                int32_t layer, int32_t num_cache_layers, int64_t pool_blocks,
                                const int32_t* block_table, const int32_t* table_row, int32_t table_width,
                                const int32_t* cu_q, const int32_t* past, int32_t num_seqs, const int32_t* items,
                                int32_t num_items, const int32_t* merges, int32_t num_merges, int32_t num_slots,
                                void* partials, int64_t partials_bytes, void* out, int32_t num_heads,
                                int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale,
                                int32_t dtype, hipStream_t stream);

/* Repack a bf16 weight w [rows, in_features] (row stride ldw) into the operand
 * order cdb_linear reads: for each tile of 16 rows and each 32-element step of
 * in_features, a contiguous 1 KiB block whose 16-byte unit l holds
 * w[16 t + l % 16][32 s + 8 (l / 16) .. +8]; tiles follow each other, steps
 * within a tile likewise. w_packed holds rows * in_features elements. rows must
 * be a multiple of 16 and in_features of 32. Run once per weight at load time. */
int cdb_linear_pack_weight(const void* w, int64_t ldw, void* w_packed, int64_t rows, int32_t in_features,
                           int32_t dtype, hipStream_t stream);

/* Dense projection of a decode batch: y[r, n] = R(sum_k x[r, k] * w[n, k]) for
 * r < rows, n < out_features, bf16 only (fp32 accumulation, one rounding),
 * with w given packed by cdb_linear_pack_weight. rows <= 64, or up to 256 when
 * in_features is 2048 and out_features a multiple of 128 of at least 4096, or
 * up to 128 when in_features is 5280 and out_features at least 4096 (a
 * wide-tile kernel); other shapes above 64 rows return CDB_ERR_SHAPE.
 * Replaces the nn.Linear calls of a recurrent step (ouro/modeling_ouro.py:162-168,
 * :371-374,390-392,431; huginn/modeling_huginn.py:239-242,310-316,372).
 * gated != 0: w holds 2*out_features rows, gate rows then up rows (the MLP's
 * concatenated gate/up projection), and y[r, n] = R(R(silu(g)) * u) with
 * g = R(x.w[n]) and u = R(x.w[out_features + n]) (ouro/modeling_ouro.py:168,
 * huginn/modeling_huginn.py:315-316). Row strides ldx, ldy are in elements
 * (multiples of 8 and 4); out_features must be a multiple of 16 and
 * in_features a multiple of 32. */
int cdb_linear(const void* x, int64_t ldx, const void* w_packed, void* y, int64_t ldy, int32_t rows,
               int32_t out_features, int32_t in_features, int32_t gated, int32_t dtype, hipStream_t stream);

/* Number of K ranges cdb_linear_parts splits a projection of this shape into,
 * or 0 when it has no split form for it (then use cdb_linear or a library GEMM).
 * Split forms exist for bf16 with in_features 2048 (up to 128 rows) or 5632 (up
 * to 256 rows) and out_features a multiple of 64 -- the Ouro O and down
 * projections (ouro/modeling_ouro.py:168,431) -- and with in_features 5280 or
 * 17920 (up to 256 rows) and out_features a multiple of 16 -- the Huginn O and
 * down projections (huginn/modeling_huginn.py:242,302,311,316). */
int32_t cdb_linear_parts_splits(int64_t rows, int32_t out_features, int32_t in_features, int32_t dtype);

/* Split-K projection: parts[s, r, n] = fp32 sum over k in the s-th of
 * splits = cdb_linear_parts_splits(...) equal K ranges of x[r, k] * w[n, k],
 * unrounded, for the consumer to add in order and round once
 * (cdb_rmsnorm_fused_parts). w packed by cdb_linear_pack_weight; parts holds
 * parts_elems >= splits * rows * out_features floats, 16-byte aligned; x row
 * stride ldx a multiple of 8 elements. Shapes without a split form return
 * CDB_ERR_SHAPE. Same projections as cdb_linear (ouro/modeling_ouro.py:168,431). */
int cdb_linear_parts(const void* x, int64_t ldx, const void* w_packed, float* parts, int64_t parts_elems,
                     int32_t rows, int32_t out_features, int32_t in_features, int32_t dtype, hipStream_t stream);

/* Workspace bytes cdb_linear_argmax needs: rows * (out_features / 16) * 8
 * (-1 for invalid sizes). */
int64_t cdb_linear_argmax_workspace_bytes(int32_t rows, int32_t out_features);

/* Greedy coda in one call: out[r] = the first n maximizing R(sum_k x[r, k] *
 * w[n, k]) over n < out_features, NaN counting as the maximum (torch.argmax over
 * the bf16 logits). It replaces lm_head followed by argmax
 * (cdb/model_runner.py:1062,1105; ouro/modeling_ouro.py:755-775). The logits
 * are never stored. The projection kernel keeps, per row and 16-column tile,
 * the best rounded value and its column in `workspace`; a second kernel
 * combines them. bf16, w packed by cdb_linear_pack_weight, 1 <= rows <= 64,
 * out_features a multiple of 16, in_features a multiple of 32, ldx a multiple
 * of 8; workspace 16-byte aligned, at least cdb_linear_argmax_workspace_bytes
 * bytes (CDB_ERR_CAPACITY otherwise).
 * With embed non-null ([out_features, width] bf16, the token embedding) the
 * same call also runs the next token's prelude for rows with a successor:
 * bank[bank_slots[r]] = embed[out[r]] when 0 <= bank_slots[r] < bank_rows --
 * the eager re-entry's embedding lookup (cdb/model_runner.py:439-457,
 * cdb/adapters/ouro.py:199-212) fused into the coda. embed and bank 16-byte
 * aligned, width a multiple of 8. */
int cdb_linear_argmax(const void* x, int64_t ldx, const void* w_packed, int64_t* out, void* workspace,
                      int64_t workspace_bytes, int32_t rows, int32_t out_features, int32_t in_features,
                      const void* embed, void* bank, int64_t bank_rows, const int64_t* bank_slots, int32_t width,
                      int32_t dtype, hipStream_t stream);

/* One greedy coda tick in a single call on `stream`, replacing the coda stage's
 * slot upload, hidden-row gather, LM head + argmax, token download and the
 * successors' gate-state reset (cdb/model_runner.py:1036-1125, 439-457,
 * 1359-1363; cdb/exit_policy.py:43-48):
 *   1. dev_upload[:count] = host_upload[:count] (pinned host memory), where the
 *      upload is [coda rows' bank slots (rows) | each row's successor bank slot
 *      or -1 (rows) | the successors' slots (num_successors)] when embed is given
 *      and only the first part otherwise (count = 2*rows + num_successors or rows);
 *   2. hidden[r] = bank[dev_upload[r]]  (hidden: [rows, width] device scratch);
 *   3. cdb_linear_argmax over hidden (ldx = in_features = width) into tokens,
 *      with the successors' embedding rows written when embed is given;
 *   4. host_tokens[:rows] = tokens  (pinned host memory, asynchronous);
 *   5. the gate state of the num_successors successor slots is reset.
 * The same preconditions as cdb_linear_argmax apply (bf16, 1 <= rows <= 64). The
 * host buffers must stay untouched until the stream has passed this call. */
int cdb_coda_greedy(const int64_t* host_upload, int64_t* dev_upload, int32_t rows, int32_t num_successors,
                    void* bank, int64_t bank_rows, int32_t width, void* hidden, const void* w_packed, int32_t vocab,
                    int64_t* tokens, void* workspace, int64_t workspace_bytes, const void* embed,
                    int64_t* host_tokens, double* cdf, double* survival, float* pending, int64_t state_capacity,
                    int32_t dtype, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* CDB_AMD_H_ */
