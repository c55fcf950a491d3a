// Row-wise stage kernels of the CDB decode step (CDNA4): RMSNorm sandwiches,
// SiLU gating, hidden-bank row compaction, greedy argmax, the early-exit gate
// with its cumulative-hazard policy, exit-KV propagation, and the prefill
// RoPE + paged KV write.
//
// All kernels are HBM- or latency-bound row operations: rows are streamed
// with 16-byte vector loads, reductions use wave shuffles plus one LDS pass,
// and nothing is reshaped into a GEMM.

#include "cdb_common.h"
#include "../../include/cdb_amd.h"

namespace cdb {

constexpr int kThreads = 256;

// ---------------------------------------------------------------------------
// Block reductions (256 threads = 4 waves).
// ---------------------------------------------------------------------------
CDB_DEVICE float block_sum(float v, float* lds) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) lds[wave] = v;
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) total += lds[w];
  return total;
}

// ---------------------------------------------------------------------------
// RMSNorm sandwiches (ouro/modeling_ouro.py:445-450, 481-502;
// huginn/modeling_huginn.py:141-146, 335-338).
//   norm_w(x) = R(w * R(x * rsqrt(mean(x^2) + eps)))   (R = round to storage)
// mode 0: h = norm_a(x)
// mode 1: h = R(r + norm_a(x));  y = norm_b(h)      (Ouro residual sandwich)
// mode 2: h = norm_a(R(r + x));  y = norm_b(h)      (Huginn residual sandwich)
// y is produced only when w_b is given. h may alias r or x (each thread only
// rewrites elements it has already read).
// ---------------------------------------------------------------------------
struct NormParams {
  const void* x;
  const float* x_parts;  // when non-null, x is R(sum over x_splits of x_parts[s]) ([x_splits, rows, width] fp32)
  int32_t x_splits;
  const void* residual;
  const void* w_a;
  const void* w_b;
  void* out_h;
  void* out_y;
  int64_t rows;
  int32_t width;
  int32_t mode;
  float eps_a, eps_b;
};

template <typename T, int NV>
__global__ void __launch_bounds__(kThreads) rmsnorm_kernel(NormParams P) {
  constexpr int V = 16 / sizeof(T);  // elements per 16-byte vector
  // Split partials loaded together before any is added: the reads of one row's
  // partials then overlap instead of paying one cache round trip per split.
  constexpr int kPartChunk = NV == 1 ? 8 : (NV <= 4 ? 4 : 2);
  __shared__ float lds[kThreads / 64];
  const int64_t row = blockIdx.x;
  if (row >= P.rows) return;
  const int W = P.width;
  const T* x = static_cast<const T*>(P.x) + row * W;
  const T* r = P.residual ? static_cast<const T*>(P.residual) + row * W : nullptr;
  const T* wa = static_cast<const T*>(P.w_a);
  const T* wb = static_cast<const T*>(P.w_b);
  T* out_h = static_cast<T*>(P.out_h) + row * W;
  T* out_y = P.out_y ? static_cast<T*>(P.out_y) + row * W : nullptr;
  const bool second = wb != nullptr && out_y != nullptr;

  float v[NV][V];
  float rv[NV][V];
  bool live[NV];
  // The weight vectors do not depend on the row's reductions: their loads are issued
  // with the row's, so no reduction waits on them.
  Vec<T, V> wav[NV], wbv[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int col = (k * kThreads + threadIdx.x) * V;
    live[k] = col < W;
    if (live[k]) {
      wav[k].load(wa + col);
      if (second) wbv[k].load(wb + col);
      if (r) {
        Vec<T, V> b;
        b.load(r + col);
#pragma unroll
        for (int i = 0; i < V; ++i) rv[k][i] = b.get(i);
      }
    }
  }
  if (P.x_parts) {
    // Split-K partials of the producing projection, summed in split order and rounded
    // once, as the projection's own output would be. A chunk's loads use a clamped
    // split index, so they are unconditional; only the adds are predicated.
#pragma unroll
    for (int k = 0; k < NV; ++k)
#pragma unroll
      for (int i = 0; i < V; ++i) v[k][i] = 0.f;
    const int splits = P.x_splits;
    for (int s0 = 0; s0 < splits; s0 += kPartChunk) {
      float4 q[kPartChunk][NV][V / 4];
#pragma unroll
      for (int c = 0; c < kPartChunk; ++c) {
        const int sp = min(s0 + c, splits - 1);
#pragma unroll
        for (int k = 0; k < NV; ++k) {
          const int col = (k * kThreads + threadIdx.x) * V;
          if (!live[k]) continue;
          const float* part = P.x_parts + ((int64_t)sp * P.rows + row) * W + col;
#pragma unroll
          for (int j = 0; j < V / 4; ++j) q[c][k][j] = *reinterpret_cast<const float4*>(part + 4 * j);
        }
      }
#pragma unroll
      for (int c = 0; c < kPartChunk; ++c) {
        if (s0 + c >= splits) break;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
          if (!live[k]) continue;
#pragma unroll
          for (int j = 0; j < V / 4; ++j) {
            v[k][4 * j] += q[c][k][j].x;
            v[k][4 * j + 1] += q[c][k][j].y;
            v[k][4 * j + 2] += q[c][k][j].z;
            v[k][4 * j + 3] += q[c][k][j].w;
          }
        }
      }
    }
#pragma unroll
    for (int k = 0; k < NV; ++k)
#pragma unroll
      for (int i = 0; i < V; ++i) v[k][i] = Elem<T>::round(v[k][i]);
  } else {
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      if (!live[k]) continue;
      const int col = (k * kThreads + threadIdx.x) * V;
      Vec<T, V> a;
      a.load(x + col);
#pragma unroll
      for (int i = 0; i < V; ++i) v[k][i] = a.get(i);
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    if (!live[k]) continue;
    if (P.mode == 2) {
#pragma unroll
      for (int i = 0; i < V; ++i) v[k][i] = Elem<T>::round(add_rn(rv[k][i], v[k][i]));
    }
#pragma unroll
    for (int i = 0; i < V; ++i) ss = fmaf(v[k][i], v[k][i], ss);
  }
  const float inv_a = rsqrtf(block_sum(ss, lds) / (float)W + P.eps_a);
  float ss2 = 0.f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    if (!live[k]) continue;
    const int col = (k * kThreads + threadIdx.x) * V;
    Vec<T, V> o;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      float n = Elem<T>::round(mul_rn(v[k][i], inv_a));
      n = Elem<T>::round(mul_rn(wav[k].get(i), n));
      if (P.mode == 1) n = Elem<T>::round(add_rn(rv[k][i], n));
      v[k][i] = n;
      o.set(i, n);
      ss2 = fmaf(n, n, ss2);
    }
    o.store(out_h + col);
  }
  if (!second) return;
  const float inv_b = rsqrtf(block_sum(ss2, lds) / (float)W + P.eps_b);
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    if (!live[k]) continue;
    const int col = (k * kThreads + threadIdx.x) * V;
    const Vec<T, V>& w = wbv[k];
    Vec<T, V> o;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float n = Elem<T>::round(mul_rn(v[k][i], inv_b));
      o.set(i, Elem<T>::round(mul_rn(w.get(i), n)));
    }
    o.store(out_y + col);
  }
}

// ---------------------------------------------------------------------------
// SiLU gating: out = R(R(silu(g)) * u) for gu = [g | u] (ouro/modeling_ouro.py:167-169,
// huginn/modeling_huginn.py:314-316).
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(kThreads) silu_mul_kernel(const T* gu, T* out, int64_t rows, int32_t width) {
  constexpr int V = 16 / sizeof(T);
  const int64_t per_row = width / V;
  const int64_t total = rows * per_row;
  for (int64_t idx = blockIdx.x * (int64_t)kThreads + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * kThreads) {
    const int64_t row = idx / per_row;
    const int64_t col = (idx - row * per_row) * V;
    Vec<T, V> g, u, o;
    g.load(gu + row * 2 * width + col);
    u.load(gu + row * 2 * width + width + col);
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float x = g.get(i);
      float s;
      if constexpr (sizeof(T) == 2) s = silu_bf16(x);  // x is a bf16 value
      else s = x / (1.0f + expf(-x));
      o.set(i, Elem<T>::round(mul_rn(s, u.get(i))));
    }
    o.store(out + row * width + col);
  }
}

// ---------------------------------------------------------------------------
// Block-table cell updates whose count lives in device memory: table[idx[i]] =
// val[i] for i < min(*count, capacity), cells outside [0, cells) skipped. The
// count is read on the device, so a captured graph applies whatever the launch's
// metadata upload carried (cdb/cache.py:115-144 refreshes the same table rows).
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(kThreads) table_update_kernel(int32_t* table, int64_t cells, const int64_t* idx,
                                                               const int32_t* val, const int32_t* count,
                                                               int32_t capacity) {
  const int n = min(*count, capacity);
  for (int i = blockIdx.x * kThreads + threadIdx.x; i < n; i += gridDim.x * kThreads) {
    const int64_t c = idx[i];
    if (c >= 0 && c < cells) table[c] = val[i];
  }
}

// ---------------------------------------------------------------------------
// Row copy with optional gather/scatter indices: dst[di[i]] = src[si[i]].
// si[i] < 0 writes zeros; di[i] < 0 skips the row. Covers the hidden-bank
// index_select/index_copy_ (cdb/model_runner.py:685-693, :559, :1101), the
// embedding lookup into bank slots, and token gathers from staged outputs.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(kThreads) copy_rows_kernel(const uint8_t* src, const int64_t* si, uint8_t* dst,
                                                            const int64_t* di, int64_t rows, int64_t row_bytes,
                                                            int64_t src_rows, int64_t dst_rows) {
  const bool vec16 = (row_bytes & 15) == 0 && ((uintptr_t)src & 15) == 0 && ((uintptr_t)dst & 15) == 0;
  const int64_t unit = vec16 ? 16 : 4;
  const int64_t units = row_bytes / unit;
  const int64_t total = rows * units;
  for (int64_t idx = blockIdx.x * (int64_t)kThreads + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * kThreads) {
    const int64_t i = idx / units;
    const int64_t u = idx - i * units;
    const int64_t d = di ? di[i] : i;
    if (d < 0 || d >= dst_rows) continue;
    const int64_t s = si ? si[i] : i;
    uint8_t* dp = dst + d * row_bytes + u * unit;
    if (vec16) {
      uint4 val = make_uint4(0, 0, 0, 0);
      if (s >= 0 && s < src_rows) val = *reinterpret_cast<const uint4*>(src + s * row_bytes + u * unit);
      *reinterpret_cast<uint4*>(dp) = val;
    } else {
      uint32_t val = 0;
      if (s >= 0 && s < src_rows) val = *reinterpret_cast<const uint32_t*>(src + s * row_bytes + u * unit);
      *reinterpret_cast<uint32_t*>(dp) = val;
    }
  }
}

// ---------------------------------------------------------------------------
// Greedy argmax over the vocabulary (cdb/model_runner.py:1062,1105): first
// index of the maximum; a NaN counts as the maximum, as torch.argmax does.
// ---------------------------------------------------------------------------

template <typename T>
__global__ void __launch_bounds__(kThreads) argmax_kernel(const T* logits, int64_t* out, int64_t rows, int32_t vocab) {
  constexpr int V = 16 / sizeof(T);  // elements per 16-byte vector
  constexpr int kUnroll = 8;         // vectors in flight per thread
  __shared__ float lv[kThreads / 64];
  __shared__ int li[kThreads / 64];
  const int64_t row = blockIdx.x;
  if (row >= rows) return;
  const T* x = logits + row * vocab;
  float best = -INFINITY;
  int bi = 0x7fffffff;
  // Whole 16-byte vectors when the row is aligned, issued kUnroll at a time; the
  // order in which a thread meets its elements does not matter since ties are
  // broken by index.
  const bool aligned = (vocab % V) == 0 && ((uintptr_t)x & 15) == 0;
  const int nvec = aligned ? vocab / V : 0;
  for (int base = threadIdx.x; base < nvec; base += kThreads * kUnroll) {
    Vec<T, V> buf[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int vi = base + u * kThreads;
      if (vi < nvec) buf[u].load(x + (int64_t)vi * V);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int vi = base + u * kThreads;
      if (vi >= nvec) continue;
#pragma unroll
      for (int e = 0; e < V; ++e) {
        const float v = buf[u].get(e);
        const int j = vi * V + e;
        if (argmax_better(v, j, best, bi)) { best = v; bi = j; }
      }
    }
  }
  for (int j = nvec * V + threadIdx.x; j < vocab; j += kThreads) {
    const float v = Elem<T>::load(x + j);
    if (argmax_better(v, j, best, bi)) { best = v; bi = j; }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float ov = shfl_xor_f32(best, m);
    const int oi = __shfl_xor(bi, m, 64);
    if (argmax_better(ov, oi, best, bi)) { best = ov; bi = oi; }
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { lv[wave] = best; li[wave] = bi; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kThreads / 64; ++w)
      if (argmax_better(lv[w], li[w], best, bi)) { best = lv[w]; bi = li[w]; }
    out[row] = bi == 0x7fffffff ? 0 : bi;
  }
}

// ---------------------------------------------------------------------------
// Early-exit gate and decision (cdb/adapters/ouro.py:286-291 gate Linear(E,1);
// cdb/exit_policy.py:150-169 decision; cdb/continuous_api.py:1671-1724 routing
// rules; huginn/exit_gates.py:33-40 latent difference).
//
// kind 0 (hazard gate): logit = R(h . w + bias), written to signal[b].
// kind 1 (latent difference): signal = R(||h - prev|| / max(||h||, R(1e-9))),
//   computed from rounded elementwise differences.
// The per-token policy state (cdf, survival in fp64; pending signal) lives in
// arrays indexed by state_index[b] (the token's hidden slot). Then:
//   consumed = SAME_STEP ? this signal : the pending one (none at step 0)
//   hazard   = sigmoid(consumed) (rounded to storage when round_hazard)
//   cdf += hazard * survival; survival *= 1 - hazard      (fp64)
//   exit = step == max_steps-1
//       || synthetic_depth >= 0 ? step >= synthetic_depth
//       || step+1 >= min_steps && (cdf >= thr | signal < thr)
// A negative synthetic depth means "no replayed depth"; a negative threshold
// disables the live policy. Rows with state_index < 0 are padding.
// ---------------------------------------------------------------------------
struct GateParams {
  const void* hidden;      // [B, W]
  const void* prev;        // [B, W] (kind 1) or null
  const void* weight;      // [W] (kind 0)
  const void* bias;        // [1] or null
  void* signal;            // [B] storage dtype
  double* cdf;             // [N]
  double* survival;        // [N]
  float* pending;          // [N] pending signal for the delayed horizon (NaN = none)
  const int64_t* state_index;   // [B]
  const int32_t* steps;         // [B]
  const int32_t* synthetic;     // [B] or null
  uint8_t* exit_flags;          // [B]
  int64_t rows;
  int64_t state_capacity;
  int32_t width;
  int32_t kind;            // 0 hazard, 1 latent difference
  int32_t rule;            // 0 cumulative hazard, 1 direct threshold
  int32_t delayed;         // 1: decide on the previous step's signal
  int32_t round_hazard;
  int32_t min_steps, max_steps;
  double threshold;
  int32_t has_threshold;
};

template <typename T>
__global__ void __launch_bounds__(kThreads) exit_gate_kernel(GateParams P) {
  constexpr int V = 16 / sizeof(T);
  __shared__ float lds[kThreads / 64];
  const int64_t row = blockIdx.x;
  if (row >= P.rows) return;
  const int W = P.width;
  const T* h = static_cast<const T*>(P.hidden) + row * W;
  float acc = 0.f, acc2 = 0.f;
  for (int col = threadIdx.x * V; col < W; col += kThreads * V) {
    Vec<T, V> a;
    a.load(h + col);
    if (P.kind == 0) {
      Vec<T, V> w;
      w.load(static_cast<const T*>(P.weight) + col);
#pragma unroll
      for (int i = 0; i < V; ++i) acc = fmaf(a.get(i), w.get(i), acc);
    } else {
      Vec<T, V> p;
      p.load(static_cast<const T*>(P.prev) + row * W + col);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float d = Elem<T>::round(sub_rn(a.get(i), p.get(i)));
        acc = fmaf(d, d, acc);
        acc2 = fmaf(a.get(i), a.get(i), acc2);
      }
    }
  }
  acc = block_sum(acc, lds);
  if (P.kind == 1) acc2 = block_sum(acc2, lds);
  if (threadIdx.x != 0) return;
  float signal;
  if (P.kind == 0) {
    const float b = P.bias ? Elem<T>::load(static_cast<const T*>(P.bias)) : 0.f;
    signal = Elem<T>::round(acc + b);
  } else {
    const float num = Elem<T>::round(sqrtf(acc));
    // clamp_min(1e-9) on a model-dtype norm: the bound is itself in the model dtype.
    const float den = fmaxf(Elem<T>::round(sqrtf(acc2)), Elem<T>::round(1e-9f));
    signal = Elem<T>::round(num / den);
  }
  Elem<T>::store(static_cast<T*>(P.signal) + row, signal);
  const int64_t si = P.state_index[row];
  if (si < 0 || si >= P.state_capacity) {
    P.exit_flags[row] = 0;
    return;
  }
  const int step = P.steps[row];
  bool exit_now = step >= P.max_steps - 1;
  const int synth = P.synthetic ? P.synthetic[row] : -1;
  float consumed = signal;
  bool have_signal = true;
  if (P.delayed) {
    consumed = P.pending[si];
    have_signal = consumed == consumed;  // NaN marks "no pending signal"
    P.pending[si] = signal;
  }
  if (!exit_now) {
    if (synth >= 0) {
      // Replayed depth: the delayed horizon applies it to the previous step.
      const int source = P.delayed ? step - 1 : step;
      exit_now = (!P.delayed || step > 0) && source >= synth;
    } else if (P.has_threshold && have_signal) {
      const int source = P.delayed ? step - 1 : step;
      const bool can_exit = source + 1 >= P.min_steps;
      if (P.rule == 0) {
        float hz = 1.0f / (1.0f + expf(-consumed));
        if (P.round_hazard) hz = Elem<T>::round(hz);
        const double hazard = (double)hz;
        double cdf = P.cdf[si];
        double surv = P.survival[si];
        cdf += hazard * surv;
        surv *= 1.0 - hazard;
        P.cdf[si] = cdf;
        P.survival[si] = surv;
        exit_now = can_exit && cdf >= P.threshold;
      } else {
        exit_now = can_exit && (double)consumed < P.threshold;
      }
    }
  }
  P.exit_flags[row] = exit_now ? 1 : 0;
}

// Reset the policy state of fresh tokens (cdb/exit_policy.py:43-48).
__global__ void gate_state_reset_kernel(double* cdf, double* survival, float* pending, const int64_t* index,
                                        int64_t n, int64_t capacity) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t s = index[i];
  if (s < 0 || s >= capacity) return;
  cdf[s] = 0.0;
  survival[s] = 1.0;
  pending[s] = __builtin_nanf("");
}

// ---------------------------------------------------------------------------
// Exit-KV propagation for the copy-on-exit layout (cdb/continuous_api.py:1225-1245,
// kv_cache_policy.py:235-258, cdb/cache.py:105-113): for token i at pool row
// rows[i] that exited at slot exit_slot[i], copy its K and V in cache layer
// base + exit_slot*C + l into base + s*C + l for every core layer l and every
// deeper slot s. One work unit per (token, layer, target slot).
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(kThreads) exit_kv_copy_kernel(uint8_t* k_pool, uint8_t* v_pool,
                                                               int64_t layer_stride_bytes, int64_t row_bytes,
                                                               const int64_t* rows, const int32_t* exit_slot,
                                                               int64_t n, int32_t layer_base, int32_t core_layers,
                                                               int32_t num_slots, int64_t pool_rows) {
  const int64_t units_per_row = row_bytes / 16;
  const int64_t per_token = (int64_t)core_layers * (num_slots - 1) * units_per_row;
  const int64_t total = n * per_token;
  for (int64_t idx = blockIdx.x * (int64_t)kThreads + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * kThreads) {
    const int64_t i = idx / per_token;
    int64_t rem = idx - i * per_token;
    const int64_t u = rem % units_per_row;
    rem /= units_per_row;
    const int l = (int)(rem % core_layers);
    const int t = (int)(rem / core_layers);  // 0 .. num_slots-2
    const int src_slot = exit_slot[i];
    const int dst_slot = src_slot + 1 + t;
    const int64_t row = rows[i];
    if (src_slot < 0 || dst_slot >= num_slots || row < 0 || row >= pool_rows) continue;
    const int64_t src_off = (int64_t)(layer_base + src_slot * core_layers + l) * layer_stride_bytes + row * row_bytes + u * 16;
    const int64_t dst_off = (int64_t)(layer_base + dst_slot * core_layers + l) * layer_stride_bytes + row * row_bytes + u * 16;
    *reinterpret_cast<uint4*>(k_pool + dst_off) = *reinterpret_cast<const uint4*>(k_pool + src_off);
    *reinterpret_cast<uint4*>(v_pool + dst_off) = *reinterpret_cast<const uint4*>(v_pool + src_off);
  }
}

// ---------------------------------------------------------------------------
// Prefill: rotate q and k of T tokens and write k, v into cache layer `layer`
// at pool rows rows[t] (cb/cache.py:284-318 index_copy_ with write indices;
// RoPE as in the decode kernel). rows[t] < 0 writes nothing (padding / trash).
// One wave per (token, head); lanes split D into 16 chunks (4 lanes idle per
// chunk group are not needed: lanes >= 16 only help with other heads).
// ---------------------------------------------------------------------------
struct RopeWriteParams {
  const void* q;        // [T, H, D]
  const void* k;        // [T, Hkv, D]
  const void* v;        // [T, Hkv, D]
  void* q_out;          // [T, H, D]
  void* k_pool;
  void* v_pool;
  int64_t layer_stride;
  const int64_t* rows;  // [T]
  const int32_t* positions;  // [T]
  const float* rope_cos;
  const float* rope_sin;
  const void* q_bias;
  const void* k_bias;
  int64_t tokens;
  int64_t pool_rows;
  int64_t q_stride, kv_stride;  // elements between consecutive tokens of q and of k / v
  int32_t layer;
  int32_t num_heads, num_kv_heads, rope_style, max_positions;
};

// N consecutive floats at p, with the widest loads p's guaranteed byte alignment allows.
template <int N, int kAlign>
CDB_DEVICE void load_floats(const float* p, float (&out)[N]) {
  if constexpr (kAlign % 16 == 0 && N % 4 == 0) {
#pragma unroll
    for (int j = 0; j < N / 4; ++j) {
      const float4 v = reinterpret_cast<const float4*>(p)[j];
      out[4 * j] = v.x; out[4 * j + 1] = v.y; out[4 * j + 2] = v.z; out[4 * j + 3] = v.w;
    }
  } else if constexpr (kAlign % 8 == 0 && N % 2 == 0) {
#pragma unroll
    for (int j = 0; j < N / 2; ++j) {
      const float2 v = reinterpret_cast<const float2*>(p)[j];
      out[2 * j] = v.x; out[2 * j + 1] = v.y;
    }
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) out[j] = p[j];
  }
}

constexpr int pow2_alignment(int bytes) { return bytes % 16 == 0 ? 16 : bytes % 8 == 0 ? 8 : 4; }

template <typename T, int D>
CDB_DEVICE void rotate_chunk(const RopeWriteParams& P, const T* base, const T* bias, int pos, int chunk, float* out) {
  constexpr int C = D / 16;
  float own[C], partner[C];
  Vec<T, C> v;
  v.load(base + chunk * C);
#pragma unroll
  for (int i = 0; i < C; ++i) own[i] = v.get(i);
  const bool split_half = P.rope_style == 1;
  if (split_half) {
    v.load(base + (chunk ^ 8) * C);
#pragma unroll
    for (int i = 0; i < C; ++i) partner[i] = v.get(i);
  }
  if (bias) {
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
  if (P.rope_style == 0) {
#pragma unroll
    for (int i = 0; i < C; ++i) out[i] = own[i];
    return;
  }
  // A table row is D/2 floats (a multiple of 16 bytes for the supported head sizes);
  // a chunk's angles are one run of consecutive entries, read as vectors.
  const int half = D / 2;
  const float* cr = P.rope_cos + (int64_t)pos * half;
  const float* sr = P.rope_sin + (int64_t)pos * half;
  if (split_half) {
    // Elements d and d + D/2 share angle d mod D/2: the chunk's angles start at (chunk mod 8) * C.
    float cs[C], sn[C];
    const int f0 = (chunk & 7) * C;
    load_floats<C, pow2_alignment(C * 4)>(cr + f0, cs);
    load_floats<C, pow2_alignment(C * 4)>(sr + f0, sn);
    const bool low = chunk < 8;
#pragma unroll
    for (int i = 0; i < C; ++i) {
      const float rot = low ? -partner[i] : partner[i];
      out[i] = Elem<T>::round(add_rn(Elem<T>::round(mul_rn(own[i], cs[i])), Elem<T>::round(mul_rn(rot, sn[i]))));
    }
  } else {
    // Interleaved pairs (2f, 2f + 1) share angle f: the chunk's angles start at chunk * C / 2.
    float cs[C / 2], sn[C / 2];
    const int f0 = chunk * (C / 2);
    load_floats<C / 2, pow2_alignment(C * 2)>(cr + f0, cs);
    load_floats<C / 2, pow2_alignment(C * 2)>(sr + f0, sn);
#pragma unroll
    for (int i = 0; i < C; i += 2) {
      const float c = cs[i >> 1], sv = sn[i >> 1];
      out[i] = Elem<T>::round(sub_rn(mul_rn(own[i], c), mul_rn(own[i + 1], sv)));
      out[i + 1] = Elem<T>::round(add_rn(mul_rn(own[i + 1], c), mul_rn(own[i], sv)));
    }
  }
}

template <typename T, int D>
__global__ void __launch_bounds__(kThreads) rope_kv_write_kernel(RopeWriteParams P) {
  constexpr int C = D / 16;
  const int lane = threadIdx.x & 63;
  const int64_t group = blockIdx.x * (int64_t)(kThreads / 16) + (threadIdx.x >> 4);  // 16-lane group id
  const int chunk = lane & 15;
  const int64_t per_token = P.num_heads + P.num_kv_heads;
  if (group >= P.tokens * per_token) return;
  const int64_t t = group / per_token;
  const int hh = (int)(group - t * per_token);
  const int pos = P.positions[t];
  const bool rope_ok = P.rope_style == 0 || (pos >= 0 && pos < P.max_positions);
  if (hh < P.num_heads) {
    const int h = hh;
    float o[C];
    const T* src = static_cast<const T*>(P.q) + t * P.q_stride + (int64_t)h * D;
    T* dst = static_cast<T*>(P.q_out) + (t * P.num_heads + h) * D + chunk * C;
    Vec<T, C> ov;
    if (rope_ok) {
      rotate_chunk<T, D>(P, src, P.q_bias ? static_cast<const T*>(P.q_bias) + (int64_t)h * D : nullptr, pos, chunk, o);
#pragma unroll
      for (int i = 0; i < C; ++i) ov.set(i, o[i]);
    } else {
#pragma unroll
      for (int i = 0; i < C; ++i) ov.set(i, __builtin_nanf(""));
    }
    ov.store(dst);
    return;
  }
  const int kvh = hh - P.num_heads;
  // The value row is read first: it depends on neither the pool row nor the key's
  // rotation, and issued after the key store it would wait for that store.
  Vec<T, C> vv;
  vv.load(static_cast<const T*>(P.v) + t * P.kv_stride + (int64_t)kvh * D + chunk * C);
  const int64_t row = P.rows[t];
  if (row < 0 || row >= P.pool_rows || !rope_ok) return;
  float o[C];
  rotate_chunk<T, D>(P, static_cast<const T*>(P.k) + t * P.kv_stride + (int64_t)kvh * D,
                     P.k_bias ? static_cast<const T*>(P.k_bias) + (int64_t)kvh * D : nullptr, pos, chunk, o);
  const int64_t off = (int64_t)P.layer * P.layer_stride + (row * P.num_kv_heads + kvh) * D + chunk * C;
  Vec<T, C> kw;
#pragma unroll
  for (int i = 0; i < C; ++i) kw.set(i, o[i]);
  kw.store(static_cast<T*>(P.k_pool) + off);
  vv.store(static_cast<T*>(P.v_pool) + off);
}

}  // namespace cdb

using namespace cdb;

namespace {

inline int grid_for(int64_t work, int per_block = kThreads) {
  int64_t g = (work + per_block - 1) / per_block;
  if (g < 1) g = 1;
  if (g > 65536) g = 65536;
  return (int)g;
}

template <typename T>
int launch_norm(const NormParams& P, hipStream_t s) {
  constexpr int V = 16 / sizeof(T);
  const int nv = (P.width + kThreads * V - 1) / (kThreads * V);
  const dim3 grid((unsigned)P.rows);
  if (nv <= 1) hipLaunchKernelGGL((rmsnorm_kernel<T, 1>), grid, dim3(kThreads), 0, s, P);
  else if (nv <= 2) hipLaunchKernelGGL((rmsnorm_kernel<T, 2>), grid, dim3(kThreads), 0, s, P);
  else if (nv <= 4) hipLaunchKernelGGL((rmsnorm_kernel<T, 4>), grid, dim3(kThreads), 0, s, P);
  else if (nv <= 8) hipLaunchKernelGGL((rmsnorm_kernel<T, 8>), grid, dim3(kThreads), 0, s, P);
  else return CDB_ERR_UNSUPPORTED;
  return hipGetLastError() == hipSuccess ? CDB_OK : CDB_ERR_HIP;
}

template <typename T, int D>
int launch_rope_write(const RopeWriteParams& P, hipStream_t s) {
  const int64_t groups = P.tokens * (P.num_heads + P.num_kv_heads);
  hipLaunchKernelGGL((rope_kv_write_kernel<T, D>), dim3(grid_for(groups, kThreads / 16)), dim3(kThreads), 0, s, P);
  return hipGetLastError() == hipSuccess ? CDB_OK : CDB_ERR_HIP;
}

}  // namespace

// ---------------------------------------------------------------------------
// Exit routing of one recurrent launch, in launch order
// ---------------------------------------------------------------------------

// lists = [exits, stays, exit rows..., staying rows...] over the launch's rows; a row
// whose bank slot is negative is padding and is in neither list. One workgroup: each
// thread counts a contiguous run of rows, a scan over the runs places them.
constexpr int kRouteThreads = 256;

__global__ void __launch_bounds__(kRouteThreads) route_compact_kernel(const uint8_t* exit_flags,
                                                                      const int64_t* bank_slots, int32_t rows,
                                                                      int32_t* lists) {
  __shared__ int wave_total[2][kRouteThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = (rows + kRouteThreads - 1) / kRouteThreads;
  const int lo = min(tid * per, rows), hi = min(lo + per, rows);
  int exits = 0, stays = 0;
  for (int r = lo; r < hi; ++r) {
    if (bank_slots[r] < 0) continue;
    if (exit_flags[r]) ++exits; else ++stays;
  }
  int run_exits = exits, run_stays = stays;  // inclusive scan over the wave's runs
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int e = __shfl_up(run_exits, off, 64), s = __shfl_up(run_stays, off, 64);
    if (lane >= off) {
      run_exits += e;
      run_stays += s;
    }
  }
  if (lane == 63) {
    wave_total[0][wave] = run_exits;
    wave_total[1][wave] = run_stays;
  }
  __syncthreads();
  int exit_at = run_exits - exits, stay_at = run_stays - stays, all_exits = 0, all_stays = 0;
#pragma unroll
  for (int w = 0; w < kRouteThreads / 64; ++w) {
    if (w < wave) {
      exit_at += wave_total[0][w];
      stay_at += wave_total[1][w];
    }
    all_exits += wave_total[0][w];
    all_stays += wave_total[1][w];
  }
  for (int r = lo; r < hi; ++r) {
    if (bank_slots[r] < 0) continue;
    if (exit_flags[r]) lists[2 + exit_at++] = r;
    else lists[2 + all_exits + stay_at++] = r;
  }
  if (tid == 0) {
    lists[0] = all_exits;
    lists[1] = all_stays;
  }
}

extern "C" {

int cdb_rmsnorm_fused(const void* x, const void* residual, const void* w_a, const void* w_b, void* out_h,
                      void* out_y, int64_t rows, int32_t width, int32_t mode, float eps_a, float eps_b,
                      int32_t dtype, hipStream_t stream) {
  if (rows == 0) return CDB_OK;
  if (!x || !w_a || !out_h) return CDB_ERR_NULL;
  if (mode < 0 || mode > 2 || rows < 0 || width <= 0 || rows > 0x7fffffff) return CDB_ERR_SHAPE;
  if (mode != 0 && !residual) return CDB_ERR_NULL;
  if (w_b && !out_y) return CDB_ERR_NULL;
  NormParams P{x, nullptr, 0, residual, w_a, w_b, out_h, out_y, rows, width, mode, eps_a, eps_b};
  if (dtype == CDB_DTYPE_F32) {
    if (width % 4) return CDB_ERR_SHAPE;
    return launch_norm<float>(P, stream);
  }
  if (dtype == CDB_DTYPE_BF16) {
    if (width % 8) return CDB_ERR_SHAPE;
    return launch_norm<bf16_t>(P, stream);
  }
  return CDB_ERR_UNSUPPORTED;
}

int cdb_rmsnorm_fused_parts(const float* x_parts, int32_t splits, const void* residual, const void* w_a,
                            const void* w_b, void* out_h, void* out_y, int64_t rows, int32_t width, int32_t mode,
                            float eps_a, float eps_b, int32_t dtype, hipStream_t stream) {
  if (rows == 0) return CDB_OK;
  if (!x_parts || !w_a || !out_h) return CDB_ERR_NULL;
  if (mode < 0 || mode > 2 || rows < 0 || width <= 0 || rows > 0x7fffffff || splits < 1 || splits > 64)
    return CDB_ERR_SHAPE;
  if (mode != 0 && !residual) return CDB_ERR_NULL;
  if (w_b && !out_y) return CDB_ERR_NULL;
  if (((uintptr_t)x_parts & 15)) return CDB_ERR_SHAPE;
  NormParams P{nullptr, x_parts, splits, residual, w_a, w_b, out_h, out_y, rows, width, mode, eps_a, eps_b};
  if (dtype == CDB_DTYPE_BF16) {
    if (width % 8) return CDB_ERR_SHAPE;
    return launch_norm<bf16_t>(P, stream);
  }
  return CDB_ERR_UNSUPPORTED;
}

int cdb_silu_mul(const void* gate_up, void* out, int64_t rows, int32_t width, int32_t dtype, hipStream_t stream) {
  if (rows == 0) return CDB_OK;
  if (!gate_up || !out) return CDB_ERR_NULL;
  if (rows < 0 || width <= 0) return CDB_ERR_SHAPE;
  if (dtype == CDB_DTYPE_F32) {
    if (width % 4) return CDB_ERR_SHAPE;
    hipLaunchKernelGGL((silu_mul_kernel<float>), dim3(grid_for(rows * width / 4)), dim3(kThreads), 0, stream,
                       static_cast<const float*>(gate_up), static_cast<float*>(out), rows, width);
  } else if (dtype == CDB_DTYPE_BF16) {
    if (width % 8) return CDB_ERR_SHAPE;
    hipLaunchKernelGGL((silu_mul_kernel<bf16_t>), dim3(grid_for(rows * width / 8)), dim3(kThreads), 0, stream,
                       static_cast<const bf16_t*>(gate_up), static_cast<bf16_t*>(out), rows, width);
  } else {
    return CDB_ERR_UNSUPPORTED;
  }
  return hipGetLastError() == hipSuccess ? CDB_OK : CDB_ERR_HIP;
}

int cdb_copy_rows(const void* src, const int64_t* src_index, int64_t src_rows, void* dst, const int64_t* dst_index,
                  int64_t dst_rows, int64_t rows, int64_t row_bytes, hipStream_t stream) {
  if (rows == 0) return CDB_OK;
  if (!src || !dst) return CDB_ERR_NULL;
  if (rows < 0 || row_bytes <= 0 || (row_bytes & 3) || src_rows < 0 || dst_rows < 0) return CDB_ERR_SHAPE;
  const int64_t unit = ((row_bytes & 15) == 0) ? 16 : 4;
  hipLaunchKernelGGL(copy_rows_kernel, dim3(grid_for(rows * (row_bytes / unit))), dim3(kThreads), 0, stream,
                     static_cast<const uint8_t*>(src), src_index, static_cast<uint8_t*>(dst), dst_index, rows,
                     row_bytes, src_rows, dst_rows);
  return hipGetLastError() == hipSuccess ? CDB_OK : CDB_ERR_HIP;
}

int cdb_table_updates(int32_t* table, int64_t cells, const int64_t* idx, const int32_t* val, const int32_t* count,
                      int32_t capacity, hipStream_t stream) {
  if (capacity == 0) return CDB_OK;
  if (!table || !idx || !val || !count) return CDB_ERR_NULL;
  if (capacity < 0 || cells <= 0) return CDB_ERR_SHAPE;
  hipLaunchKernelGGL(table_update_kernel, dim3(grid_for(capacity)), dim3(kThreads), 0, stream, table, cells, idx, val,
                     count, capacity);
  return hipGetLastError() == hipSuccess ? CDB_OK : CDB_ERR_HIP;
}

int cdb_route_compact(const uint8_t* exit_flags, const int64_t* bank_slots, int32_t rows, int32_t* lists,
                      hipStream_t stream) {
  if (rows == 0) return CDB_OK;
  if (!exit_flags || !bank_slots || !lists) return CDB_ERR_NULL;
  if (rows < 0) return CDB_ERR_SHAPE;
  hipLaunchKernelGGL(route_compact_kernel, dim3(1), dim3(kRouteThreads), 0, stream, exit_flags, bank_slots, rows,
                     lists);
  return hipGetLastError() == hipSuccess ? CDB_OK : CDB_ERR_HIP;
}

int cdb_argmax(const void* logits, int64_t* out, int64_t rows, int32_t vocab, int32_t dtype, hipStream_t stream) {
  if (rows == 0) return CDB_OK;
  if (!logits || !out) return CDB_ERR_NULL;
  if (rows < 0 || vocab <= 0 || rows > 0x7fffffff) return CDB_ERR_SHAPE;
  if (dtype == CDB_DTYPE_F32)
    hipLaunchKernelGGL((argmax_kernel<float>), dim3((unsigned)rows), dim3(kThreads), 0, stream,
                       static_cast<const float*>(logits), out, rows, vocab);
  else if (dtype == CDB_DTYPE_BF16)
    hipLaunchKernelGGL((argmax_kernel<bf16_t>), dim3((unsigned)rows), dim3(kThreads), 0, stream,
                       static_cast<const bf16_t*>(logits), out, rows, vocab);
  else
    return CDB_ERR_UNSUPPORTED;
  return hipGetLastError() == hipSuccess ? CDB_OK : CDB_ERR_HIP;
}

int cdb_exit_gate(const void* hidden, const void* prev, const void* weight, const void* bias, void* signal,
                  double* cdf, double* survival, float* pending, int64_t state_capacity, const int64_t* state_index,
                  const int32_t* steps, const int32_t* synthetic_depth, uint8_t* exit_flags, int64_t rows,
                  int32_t width, int32_t kind, int32_t rule, int32_t delayed, int32_t round_hazard,
                  int32_t min_steps, int32_t max_steps, double threshold, int32_t has_threshold, int32_t dtype,
                  hipStream_t stream) {
  if (rows == 0) return CDB_OK;
  if (!hidden || !signal || !cdf || !survival || !pending || !state_index || !steps || !exit_flags)
    return CDB_ERR_NULL;
  if (kind == 0 && !weight) return CDB_ERR_NULL;
  if (kind == 1 && !prev) return CDB_ERR_NULL;
  if (rows < 0 || rows > 0x7fffffff || width <= 0 || kind < 0 || kind > 1 || rule < 0 || rule > 1 ||
      max_steps <= 0 || state_capacity <= 0)
    return CDB_ERR_SHAPE;
  GateParams P{hidden, prev, weight, bias, signal, cdf, survival, pending, state_index, steps, synthetic_depth,
               exit_flags, rows, state_capacity, width, kind, rule, delayed, round_hazard, min_steps, max_steps, threshold,
               has_threshold};
  if (dtype == CDB_DTYPE_F32) {
    if (width % 4) return CDB_ERR_SHAPE;
    hipLaunchKernelGGL((exit_gate_kernel<float>), dim3((unsigned)rows), dim3(kThreads), 0, stream, P);
  } else if (dtype == CDB_DTYPE_BF16) {
    if (width % 8) return CDB_ERR_SHAPE;
    hipLaunchKernelGGL((exit_gate_kernel<bf16_t>), dim3((unsigned)rows), dim3(kThreads), 0, stream, P);
  } else {
    return CDB_ERR_UNSUPPORTED;
  }
  return hipGetLastError() == hipSuccess ? CDB_OK : CDB_ERR_HIP;
}

int cdb_exit_gate_reset(double* cdf, double* survival, float* pending, int64_t state_capacity,
                        const int64_t* index, int64_t n, hipStream_t stream) {
  if (n == 0) return CDB_OK;
  if (!cdf || !survival || !pending || !index) return CDB_ERR_NULL;
  if (n < 0) return CDB_ERR_SHAPE;
  hipLaunchKernelGGL(gate_state_reset_kernel, dim3(grid_for(n)), dim3(kThreads), 0, stream, cdf, survival, pending,
                     index, n, state_capacity);
  return hipGetLastError() == hipSuccess ? CDB_OK : CDB_ERR_HIP;
}

int cdb_exit_kv_copy(void* k_pool, void* v_pool, int64_t layer_stride, int64_t pool_rows, int32_t num_kv_heads,
                     int32_t head_dim, const int64_t* rows, const int32_t* exit_slot, int64_t n, int32_t layer_base,
                     int32_t core_layers, int32_t num_slots, int32_t dtype, hipStream_t stream) {
  if (n == 0 || num_slots <= 1) return CDB_OK;
  if (!k_pool || !v_pool || !rows || !exit_slot) return CDB_ERR_NULL;
  if (n < 0 || core_layers <= 0 || layer_base < 0 || pool_rows <= 0 || num_kv_heads <= 0 || head_dim <= 0)
    return CDB_ERR_SHAPE;
  const int64_t elem = dtype == CDB_DTYPE_F32 ? 4 : dtype == CDB_DTYPE_BF16 ? 2 : 0;
  if (!elem) return CDB_ERR_UNSUPPORTED;
  const int64_t row_bytes = (int64_t)num_kv_heads * head_dim * elem;
  if (row_bytes % 16) return CDB_ERR_SHAPE;
  const int64_t work = n * core_layers * (num_slots - 1) * (row_bytes / 16);
  hipLaunchKernelGGL(exit_kv_copy_kernel, dim3(grid_for(work)), dim3(kThreads), 0, stream,
                     static_cast<uint8_t*>(k_pool), static_cast<uint8_t*>(v_pool), layer_stride * elem, row_bytes,
                     rows, exit_slot, n, layer_base, core_layers, num_slots, pool_rows);
  return hipGetLastError() == hipSuccess ? CDB_OK : CDB_ERR_HIP;
}

int cdb_rope_kv_write(const void* q, const void* k, const void* v, void* q_out, void* k_pool, void* v_pool,
                      int64_t layer_stride, int32_t layer, const int64_t* rows, int64_t pool_rows,
                      const int32_t* positions, const float* rope_cos, const float* rope_sin, int32_t rope_style,
                      int32_t max_positions, const void* q_bias, const void* k_bias, int64_t tokens,
                      int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int64_t q_stride, int64_t kv_stride,
                      int32_t dtype, hipStream_t stream) {
  if (tokens == 0) return CDB_OK;
  if (!q || !k || !v || !q_out || !k_pool || !v_pool || !rows || !positions) return CDB_ERR_NULL;
  if (rope_style < 0 || rope_style > 2) return CDB_ERR_SHAPE;
  if (rope_style && (!rope_cos || !rope_sin)) return CDB_ERR_NULL;
  if (tokens < 0 || num_heads <= 0 || num_kv_heads <= 0 || layer < 0 || pool_rows <= 0) return CDB_ERR_SHAPE;
  if (q_stride <= 0) q_stride = (int64_t)num_heads * head_dim;
  if (kv_stride <= 0) kv_stride = (int64_t)num_kv_heads * head_dim;
  if (q_stride < (int64_t)num_heads * head_dim || kv_stride < (int64_t)num_kv_heads * head_dim) return CDB_ERR_SHAPE;
  RopeWriteParams P{q, k, v, q_out, k_pool, v_pool, layer_stride, rows, positions, rope_cos, rope_sin, q_bias,
                    k_bias, tokens, pool_rows, q_stride, kv_stride, layer, num_heads, num_kv_heads, rope_style,
                    max_positions};
  auto by_dim = [&](auto tag) -> int {
    using T = decltype(tag);
    switch (head_dim) {
      case 64: return launch_rope_write<T, 64>(P, stream);
      case 96: return launch_rope_write<T, 96>(P, stream);
      case 128: return launch_rope_write<T, 128>(P, stream);
      default: return CDB_ERR_UNSUPPORTED;
    }
  };
  if (dtype == CDB_DTYPE_F32) return by_dim(float{});
  if (dtype == CDB_DTYPE_BF16) return by_dim(bf16_t{});
  return CDB_ERR_UNSUPPORTED;
}

int cdb_coda_greedy(const int64_t* host_upload, int64_t* dev_upload, int32_t rows, int32_t num_successors,
                    void* bank, int64_t bank_rows, int32_t width, void* hidden, const void* w_packed, int32_t vocab,
                    int64_t* tokens, void* workspace, int64_t workspace_bytes, const void* embed,
                    int64_t* host_tokens, double* cdf, double* survival, float* pending, int64_t state_capacity,
                    int32_t dtype, hipStream_t stream) {
  if (rows == 0) return CDB_OK;
  if (!host_upload || !dev_upload || !bank || !hidden || !w_packed || !tokens || !workspace || !host_tokens)
    return CDB_ERR_NULL;
  if (rows < 0 || num_successors < 0 || num_successors > rows || width <= 0 || bank_rows <= 0 || vocab <= 0)
    return CDB_ERR_SHAPE;
  if (num_successors > 0 && (!embed || !cdf || !survival || !pending)) return CDB_ERR_NULL;
  if (dtype != CDB_DTYPE_BF16) return CDB_ERR_UNSUPPORTED;
  // Upload layout: [coda rows' bank slots | per-row successor slot or -1 | successors' slots],
  // the last two parts only when the successors' prelude is fused (embed given).
  const int64_t count = embed ? 2 * (int64_t)rows + num_successors : rows;
  if (hipMemcpyAsync(dev_upload, host_upload, count * sizeof(int64_t), hipMemcpyHostToDevice, stream) != hipSuccess)
    return CDB_ERR_HIP;
  const int64_t row_bytes = (int64_t)width * 2;
  int code = cdb_copy_rows(bank, dev_upload, bank_rows, hidden, nullptr, rows, rows, row_bytes, stream);
  if (code) return code;
  code = cdb_linear_argmax(hidden, width, w_packed, tokens, workspace, workspace_bytes, rows, vocab, width, embed,
                           embed ? bank : nullptr, embed ? bank_rows : 0, embed ? dev_upload + rows : nullptr,
                           embed ? width : 0, dtype, stream);
  if (code) return code;
  if (hipMemcpyAsync(host_tokens, tokens, rows * sizeof(int64_t), hipMemcpyDeviceToHost, stream) != hipSuccess)
    return CDB_ERR_HIP;
  if (num_successors > 0)
    return cdb_exit_gate_reset(cdf, survival, pending, state_capacity, dev_upload + 2 * (int64_t)rows,
                               num_successors, stream);
  return CDB_OK;
}

}  // extern "C"
