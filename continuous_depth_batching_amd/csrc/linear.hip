// Decode-batch dense projection y = x W^T on MFMA tiles (CDNA4), for the few
// rows a recurrent launch carries.
//
// Replaces the nn.Linear projections of a recurrent step as the reference runs
// them through torch (q/k/v/o_proj ouro/modeling_ouro.py:371-374,390-392,431;
// gate/up/down_proj :162-168; Huginn Wqkv/proj/fc/adapter
// huginn/modeling_huginn.py:239-242,310-316,372). With at most 64 rows the
// product is bound by streaming W from HBM (2 flops per weight element per
// row, far under the MFMA ridge), so the kernel is built to keep that stream
// deep rather than to reuse tiles:
//   * W is stored pre-packed in MFMA operand order (cdb_linear_pack_weight):
//     for each tile of 16 rows and each 32-element contraction step, the 1 KiB
//     block that one wave loads as its A operand -- lane (r, g) holding
//     W[16 t + r][32 s + 8 g .. +8] -- is contiguous, and a tile's blocks follow
//     each other along K. Every weight load is one fully contiguous 1 KiB wave
//     access, and a wave's batch of S steps is S KiB in a row;
//   * a workgroup owns NB tiles of 16 output columns and splits the contraction
//     dimension K between its waves; every weight element is read exactly once,
//     with non-temporal loads so x stays resident in L2;
//   * MFMA 16x16x32 bf16 with A = 16 rows of W and B = x^T (up to 4 tiles of
//     16 rows of x): lane (m, g) loads x[m][32 s + 8 g .. +8], the same
//     contraction indices as its A vector, and the accumulator C[n][m] lands
//     in lane (m % 16, n / 4);
//   * the waves' partial tiles are summed in LDS in a fixed order (slot w holds
//     wave w + wave w+8), so results do not depend on scheduling;
//   * gated mode (the MLP's gate_up): the workgroup also owns the matching 16
//     up-projection rows W[N + n] and writes R(R(silu(R(g))) * R(u)) directly,
//     the rounding chain of torch's bf16 silu and multiply, so the [rows, 2N]
//     gate_up activation never reaches memory.
// Output rows are rounded to bf16 once, after the fp32 sum over all of K.

#include "cdb_common.h"
#include "../../include/cdb_amd.h"

namespace cdb {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

// Kept at 64 bytes, which the launch preloads into scalar registers: the
// output forms share the two output pointers.
struct LinearParams {
  const bf16_t* x;  // [M, K], row stride ldx elements
  const bf16_t* w;  // packed [N, K] (gated: [2N, K], gate rows then up rows)
  union {
    bf16_t* y;        // [M, N], row stride ldy
    float* best_val;  // argmax form: per row and 16-column tile, the largest rounded value ...
  };
  union {
    float* parts;       // split-K form: fp32 partial sums [splits, M, N] instead of y
    int32_t* best_idx;  // argmax form: ... and its first column ([M, N / 16] each)
  };
  int64_t ldx, ldy;
  int32_t M, N, K;
  int32_t steps_per_wave;  // 32-element contraction steps per wave
};

constexpr int kLinearMaxRows = 64;
constexpr int kLinearWideMaxRows = 256;
constexpr int kLinearMaxWaves = 16;

CDB_DEVICE bf16x8_t load_w(const bf16_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const bf16x8_t*>(p));
}
CDB_DEVICE bf16x8_t load_x(const bf16_t* p) { return *reinterpret_cast<const bf16x8_t*>(p); }

// Sum of partial tile `tile` over the first `slots` LDS slots, added in slot order.
// Every slot is read up front so the reads overlap instead of each waiting for the
// previous add. Past `slots` the last written slot is read again and not used (a
// select, not an add of zero, so a -0 sum keeps its sign).
template <int SLOTS, int NT, int MT>
CDB_DEVICE f32x4_t sum_slots(const f32x4_t (&red)[SLOTS][NT][MT][kWave], int tile, int mt, int l, int slots) {
  f32x4_t part[SLOTS];
#pragma unroll
  for (int sl = 0; sl < SLOTS; ++sl) part[sl] = red[min(sl, slots - 1)][tile][mt][l];
  f32x4_t v = part[0];
#pragma unroll
  for (int sl = 1; sl < SLOTS; ++sl) {
    const f32x4_t w = v + part[sl];
    v = sl < slots ? w : v;
  }
  return v;
}

// MT: 16-row tiles of x (1, 2 or 4). NB: 16-column tiles of y per workgroup; every
// wave computes all of them, so each x vector it loads feeds NB (gated: 2*NB)
// MFMAs. S: contraction steps loaded per batch. SLOTS: LDS partial tiles (waves
// w, w + SLOTS, w + 2*SLOTS, ... add into slot w in that order). ARGMAX: instead
// of y, store each row's greedy-argmax candidate of every 16-column tile (the
// largest bf16-rounded output and its first column, torch.argmax order), for
// linear_argmax_merge_kernel.
template <int MT, int NB, int S, int SLOTS, bool GATED, int MAXT, bool ARGMAX = false>
__global__ void __launch_bounds__(MAXT) linear_kernel(LinearParams p) {
  constexpr int NT = GATED ? 2 * NB : NB;  // W row tiles: gate tiles, then up tiles
  __shared__ f32x4_t red[SLOTS][NT][MT][kWave];

  const int lane = threadIdx.x & (kWave - 1);
  // Wave-uniform in a scalar register, so the step loop and its bounds stay scalar.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int nwaves = blockDim.x / kWave;
  const int r = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16 * NB;

  // Packed W: the block of tile t, step s starts at element (t * steps + s) * 512.
  const int total = p.K / 32;
  const bf16_t* wrow[NT];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    wrow[j] = p.w + ((int64_t)(n0 / 16 + j) * total) * 512 + 8 * lane;
    if constexpr (GATED) wrow[NB + j] = p.w + ((int64_t)((p.N + n0) / 16 + j) * total) * 512 + 8 * lane;
  }
  const bf16_t* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xrow[mt] = p.x + (int64_t)min(mt * 16 + r, p.M - 1) * p.ldx + 8 * g;

  f32x4_t acc[NT][MT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int s_begin = wave * p.steps_per_wave;
  const int s_end = min(s_begin + p.steps_per_wave, total);
  for (int s = s_begin; s < s_end; s += S) {
    // Straight-line batch of S steps: steps past the wave's range (only in the last
    // wave's last batch) reload its last step in bounds and contribute a zero W tile.
    // x first: loads complete in issue order, so the first MFMA then waits only for
    // the batch's x (an L2 hit) and its own weight block, not for every weight block.
    bf16x8_t wv[NT][S], xv[MT][S];
#pragma unroll
    for (int t = 0; t < S; ++t) {
      const int64_t k = (int64_t)min(s + t, s_end - 1) * 32;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) xv[mt][t] = load_x(xrow[mt] + k);
    }
#pragma unroll
    for (int t = 0; t < S; ++t) {
      const int64_t blk = (int64_t)min(s + t, s_end - 1) * 512;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) wv[nt][t] = load_w(wrow[nt] + blk);
    }
    // Keep the whole batch of loads in flight before the first MFMA waits on one.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < S; ++t) {
      const bool valid = s + t < s_end;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const bf16x8_t a = valid ? wv[nt][t] : bf16x8_t{};
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, xv[mt][t], acc[nt][mt], 0, 0, 0);
      }
    }
  }

  // Fixed-order reduction of the waves' partial tiles.
  if (wave < SLOTS) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) red[wave][nt][mt][lane] = acc[nt][mt];
  }
  for (int grp = 1; grp * SLOTS < nwaves; ++grp) {
    __syncthreads();
    if (wave / SLOTS == grp) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) red[wave - grp * SLOTS][nt][mt][lane] += acc[nt][mt];
    }
  }
  __syncthreads();

  const int slots = min(nwaves, SLOTS);
  if constexpr (ARGMAX) {
    // One wave per (column tile, row tile): lane l holds row l % 16, columns
    // 4 (l / 16) .. +3; the four lane groups of a row are then combined.
    for (int idx = threadIdx.x; idx < NB * MT * kWave; idx += blockDim.x) {
      const int j = idx / (MT * kWave);
      const int mt = (idx / kWave) % MT;
      const int l = idx & (kWave - 1);
      const int m = mt * 16 + (l & 15);
      const f32x4_t v = sum_slots(red, j, mt, l, slots);
      const int c0 = n0 + 16 * j + 4 * (l >> 4);
      float best = -INFINITY;
      int bi = 0x7fffffff;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float r = round_bf16(v[i]);
        if (argmax_better(r, c0 + i, best, bi)) { best = r; bi = c0 + i; }
      }
#pragma unroll
      for (int mask = 16; mask <= 32; mask <<= 1) {
        const float ov = shfl_xor_f32(best, mask);
        const int oi = __shfl_xor(bi, mask, 64);
        if (argmax_better(ov, oi, best, bi)) { best = ov; bi = oi; }
      }
      if (l < 16 && m < p.M) {
        const int64_t e = (int64_t)m * (p.N / 16) + n0 / 16 + j;
        p.best_val[e] = best;
        p.best_idx[e] = bi;
      }
    }
    return;
  }

  // Epilogue: one thread per (column tile, row tile, lane) of the output.
  for (int idx = threadIdx.x; idx < NB * MT * kWave; idx += blockDim.x) {
    const int j = idx / (MT * kWave);
    const int mt = (idx / kWave) % MT;
    const int l = idx & (kWave - 1);
    const int m = mt * 16 + (l & 15);
    if (m < p.M) {
      const f32x4_t v = sum_slots(red, j, mt, l, slots);
      f32x4_t u = {};
      if constexpr (GATED) u = sum_slots(red, NB + j, mt, l, slots);
      Vec<bf16_t, 4> o;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (GATED) {
          const float gate = round_bf16(v[i]);
          const float act = silu_bf16(gate);
          o.set(i, act * round_bf16(u[i]));
        } else {
          o.set(i, v[i]);
        }
      }
      o.store(p.y + (int64_t)m * p.ldy + n0 + 16 * j + 4 * (l >> 4));
    }
  }
}

// ---------------------------------------------------------------------------
// Wide-tile variant for batches of 33 to 256 rows. A workgroup owns 16*MT rows
// x 4*16*NTW columns with the full K; wave w owns column tiles w*NTW .. and
// every row tile, so each weight byte is loaded by exactly one wave:
//   * weight blocks stream from the packed layout into a ring of STAGES chunks
//     of registers (SC steps each), STAGES chunks ahead of the MFMAs that use
//     them, so the HBM latency is covered without waiting per chunk;
//   * x chunks go through LDS, double-buffered, in operand order (16-byte
//     unit (r, g) of block (row tile, step) holds x[16 t + r][32 s + 8 g ..]);
//   * workgroups of one column range (different row ranges) sit on one XCD,
//     so the weights cross HBM once;
//   * PIPE: x chunks are triple-buffered and stored two chunks ahead, and each
//     step's x operands are read from LDS while the previous step's MFMAs run
//     (without it a step's reads wait for the previous step's last MFMA, and
//     its MFMAs for the reads). Every output still adds its K steps in order
//     in one accumulator, so the results are bit-identical either way.
// ---------------------------------------------------------------------------
// Slot of x unit (row r of a 16-row tile, step t of the chunk, k group g) within
// its 64-unit block: the MFMA lane that reads it is r + 16 g, with r swizzled by
// an XOR of (t, g) so that the eight (SC = 2) or sixteen (SC = 4) units one row
// contributes to a chunk -- stored by consecutive threads -- land on distinct
// LDS banks. For each (t, g) the XOR permutes r, so a step's 64 units stay one
// contiguous block and the reads stay conflict-free.
template <int SC>
CDB_DEVICE int x_slot(int r, int t, int g) {
  static_assert(SC == 2 || SC == 4, "x chunks of 2 or 4 steps");
  const int sw = SC == 2 ? 2 * (4 * (t & 1) + g) : 4 * (t & 3) + g;
  return (r ^ sw) + 16 * g;
}

// KSPLIT > 1: K is cut into KSPLIT ranges of KSTEPS steps; each workgroup covers
// one range and stores fp32 partial sums to p.parts[split], for a consumer that
// adds them in split order and rounds once (the residual RMSNorm).
// NTAIL: N is a multiple of 16 but not of 64 * NTW, so the last column range is
// narrower; without it N must be a multiple of 64 * NTW.
template <int MT, int NTW, int SC, int STAGES, bool GATED, int KSTEPS, int KSPLIT = 1, bool NTAIL = false,
          bool PIPE = false>
__global__ void __launch_bounds__(256) linear_wide_kernel(LinearParams p) {
  constexpr int NT = GATED ? 2 * NTW : NTW;
  constexpr int ROWS = 16 * MT;
  constexpr int KC = 32 * SC;
  constexpr int UNITS = ROWS * KC / 8;
  static_assert(UNITS % 256 == 0, "x chunk must split evenly over the workgroup");
  static_assert(!PIPE || STAGES >= 3, "the pipelined form stores x two chunks ahead of its use");
  constexpr int UPT = UNITS / 256;
  __shared__ bf16x8_t xs[PIPE ? 3 : 2][MT][SC][kWave];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);

  // Workgroups that share a (column range, K split) -- all its row ranges -- sit on one XCD.
  // With NTAIL the last column range may cover fewer than 4 * NTW 16-column tiles, and
  // the waves past N load the last tile (in bounds) and store nothing.
  const int n_tiles = NTAIL ? (p.N / 16 + 4 * NTW - 1) / (4 * NTW) : p.N / (64 * NTW);
  const int m_tiles = (p.M + ROWS - 1) / ROWS;
  const int xcd = blockIdx.x & 7, q = blockIdx.x >> 3;
  const int mi = q % m_tiles;
  const int pair = (q / m_tiles) * 8 + xcd;  // column range + K split
  if (pair >= n_tiles * KSPLIT) return;     // padding workgroup of the XCD-major order: exits before any barrier
  const int ni = pair % n_tiles, ks = pair / n_tiles;
  const int m0 = mi * ROWS;
  const int n0 = ni * 64 * NTW;

  // The K range is a compile-time constant so the chunk loop unrolls completely:
  // the compiler's wait-count pass then sees every load of the register rings in
  // order and waits exactly for the chunk it is about to use.
  constexpr int total = KSTEPS;
  constexpr int nchunks = (total + SC - 1) / SC;
  const int tile_steps = p.K / 32;  // steps of one packed weight tile
  const int k_first = ks * KSTEPS;
  const bf16_t* wp[NT];
#pragma unroll
  for (int j = 0; j < NTW; ++j) {
    const int tile = NTAIL ? min(n0 / 16 + wave * NTW + j, p.N / 16 - 1) : n0 / 16 + wave * NTW + j;
    wp[j] = p.w + ((int64_t)tile * tile_steps + k_first) * 512 + 8 * lane;
    if constexpr (GATED)
      wp[NTW + j] = p.w + ((int64_t)(NTAIL ? p.N / 16 + tile : (p.N + n0) / 16 + wave * NTW + j) * tile_steps +
                           k_first) * 512 + 8 * lane;
  }
  // x staging: thread unit u reads 16 bytes of one row (units of a row are
  // consecutive, so the global reads coalesce) and stores them to that row's
  // operand slot in LDS.
  const bf16_t* xsrc[UPT];
  int xk[UPT], xdst[UPT];
#pragma unroll
  for (int i = 0; i < UPT; ++i) {
    const int u = tid + 256 * i;
    const int row = u / (KC / 8), k8 = u % (KC / 8);
    xsrc[i] = p.x + (int64_t)min(m0 + row, p.M - 1) * p.ldx + (int64_t)k_first * 32;
    xk[i] = 8 * k8;
    xdst[i] = (((row >> 4) * SC + (k8 >> 2)) * kWave) + x_slot<SC>(row & 15, k8 >> 2, k8 & 3);
  }
  // This lane's operand unit (row lane % 16, k group lane / 16) of each step.
  int xrd[SC];
#pragma unroll
  for (int t = 0; t < SC; ++t) xrd[t] = x_slot<SC>(lane & 15, t, lane >> 4);
  auto load_x = [&](int c, bf16x8_t (&xr)[UPT]) {
#pragma unroll
    for (int i = 0; i < UPT; ++i) xr[i] = cdb::load_x(xsrc[i] + min(c * KC + xk[i], total * 32 - 8));
  };
  auto store_x = [&](int buf, const bf16x8_t (&xr)[UPT]) {
    bf16x8_t* base = &xs[buf][0][0][0];
#pragma unroll
    for (int i = 0; i < UPT; ++i) base[xdst[i]] = xr[i];
  };
  auto load_w = [&](int c, bf16x8_t (&wr)[NT][SC]) {
#pragma unroll
    for (int t = 0; t < SC; ++t) {
      const int64_t blk = (int64_t)min(c * SC + t, total - 1) * 512;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) wr[nt][t] = cdb::load_w(wp[nt] + blk);
    }
  };

  f32x4_t acc[NT][MT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // Chunk j's weights live in ring[j % STAGES] and its x in xring[j % STAGES] from STAGES
  // chunks before it is used; x moves to LDS one chunk ahead of its MFMAs (two with PIPE).
  bf16x8_t ring[STAGES][NT][SC];
  bf16x8_t xring[STAGES][UPT];
#pragma unroll
  for (int st = 0; st < STAGES; ++st) {  // chunks past the end reload in-bounds data
    load_w(st, ring[st]);
    load_x(st, xring[st]);
  }
  store_x(0, xring[0]);
  if constexpr (PIPE) {
    if (nchunks > 1) store_x(1, xring[1]);
  }
  __syncthreads();

  if constexpr (PIPE) {
    // Chunk c's x sits in xs[c % 3]. Step (c, t)'s operands are read during step
    // (c, t - 1) -- or, for t = 0, during chunk c - 1's last step, after the barrier
    // that ended chunk c - 2 published xs[c % 3]. Chunk c stores chunk c + 2's x into
    // xs[(c + 2) % 3], whose last reads (chunk c - 1's) all completed before the
    // barrier that ended chunk c - 1 (the barrier waits for this wave's LDS reads).
    auto read_b = [&](int c, int t, bf16x8_t (&b)[MT]) {
      const bool valid = c * SC + t < total;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) b[mt] = valid ? xs[c % 3][mt][t][xrd[t]] : bf16x8_t{};
    };
    bf16x8_t b[MT];
    read_b(0, 0, b);
#pragma unroll
    for (int c0 = 0; c0 < nchunks; c0 += STAGES) {
#pragma unroll
      for (int st = 0; st < STAGES; ++st) {
        const int c = c0 + st;
        if (c < nchunks) {
#pragma unroll
          for (int t = 0; t < SC; ++t) {
            const bool valid = c * SC + t < total;
            const bool next = t + 1 < SC || c + 1 < nchunks;
            bf16x8_t bn[MT];
            if (t + 1 < SC) read_b(c, t + 1, bn);
            else if (c + 1 < nchunks) read_b(c + 1, 0, bn);
            // Keeps the reads above this step's MFMAs: left to itself the scheduler
            // sinks each read below the last MFMA that uses the register it refills.
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
              const bf16x8_t a = valid ? ring[st][nt][t] : bf16x8_t{};
#pragma unroll
              for (int mt = 0; mt < MT; ++mt)
                acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[mt], acc[nt][mt], 0, 0, 0);
            }
            if (next) {
#pragma unroll
              for (int mt = 0; mt < MT; ++mt) b[mt] = bn[mt];
            }
          }
          if (c + STAGES < nchunks) load_w(c + STAGES, ring[st]);
          if (c + 2 < nchunks) store_x((c + 2) % 3, xring[(st + 2) % STAGES]);
          if (c + STAGES < nchunks) load_x(c + STAGES, xring[st]);
          lds_barrier();
        }
      }
    }
  } else {
#pragma unroll
    for (int c0 = 0; c0 < nchunks; c0 += STAGES) {
#pragma unroll
      for (int st = 0; st < STAGES; ++st) {
        const int c = c0 + st;
        if (c < nchunks) {
          const int cur = c & 1;
          const bool more = c + 1 < nchunks;
#pragma unroll
          for (int t = 0; t < SC; ++t) {
            const bool valid = c * SC + t < total;
            bf16x8_t b[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) b[mt] = valid ? xs[cur][mt][t][xrd[t]] : bf16x8_t{};
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
              const bf16x8_t a = valid ? ring[st][nt][t] : bf16x8_t{};
#pragma unroll
              for (int mt = 0; mt < MT; ++mt)
                acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[mt], acc[nt][mt], 0, 0, 0);
            }
          }
          if (c + STAGES < nchunks) load_w(c + STAGES, ring[st]);
          if (more) store_x(cur ^ 1, xring[(st + 1) % STAGES]);
          if (c + STAGES < nchunks) load_x(c + STAGES, xring[st]);
          lds_barrier();
        }
      }
    }
  }

#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = m0 + 16 * mt + (lane & 15);
    if (m >= p.M) continue;
    if constexpr (KSPLIT > 1) {
#pragma unroll
      for (int j = 0; j < NTW; ++j) {
        if (NTAIL && n0 + 16 * (wave * NTW + j) >= p.N) continue;  // wave-uniform: a tile past N
        float* dst = p.parts + ((int64_t)ks * p.M + m) * p.N + n0 + 16 * (wave * NTW + j) + 4 * (lane >> 4);
        *reinterpret_cast<f32x4_t*>(dst) = acc[j][mt];
      }
      continue;
    }
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
      if (NTAIL && n0 + 16 * (wave * NTW + j) >= p.N) continue;  // wave-uniform: a tile past N
      Vec<bf16_t, 4> o;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (GATED) {
          const float gate = round_bf16(acc[j][mt][i]);
          const float act = silu_bf16(gate);
          o.set(i, act * round_bf16(acc[NTW + j][mt][i]));
        } else {
          o.set(i, acc[j][mt][i]);
        }
      }
      o.store(p.y + (int64_t)m * p.ldy + n0 + 16 * (wave * NTW + j) + 4 * (lane >> 4));
    }
  }
}

template <int MT, int NTW, int SC, int STAGES, bool GATED, int KSTEPS, int KSPLIT = 1, bool NTAIL = false,
          bool PIPE = false>
int launch_linear_wide(LinearParams prm, hipStream_t stream) {
  if ((NTAIL ? prm.N % 16 : prm.N % (64 * NTW)) || prm.K != 32 * KSTEPS * KSPLIT) return CDB_ERR_SHAPE;
  const int n_tiles = NTAIL ? (prm.N / 16 + 4 * NTW - 1) / (4 * NTW) : prm.N / (64 * NTW);  // as the kernel counts
  const int m_tiles = (prm.M + 16 * MT - 1) / (16 * MT);
  const int pairs = n_tiles * KSPLIT;
  hipLaunchKernelGGL((linear_wide_kernel<MT, NTW, SC, STAGES, GATED, KSTEPS, KSPLIT, NTAIL, PIPE>),
                     dim3((pairs + 7) / 8 * 8 * m_tiles), dim3(256), 0, stream, prm);
  return hipGetLastError() == hipSuccess ? CDB_OK : CDB_ERR_HIP;
}

// W [rows, K] (row stride ldw) -> packed MFMA operand order; one thread per 16 bytes.
__global__ void __launch_bounds__(256) linear_pack_kernel(const bf16_t* w, int64_t ldw, bf16_t* out, int64_t rows,
                                                          int32_t K) {
  const int64_t steps = K / 32;
  const int64_t total = rows / 16 * steps * kWave;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int lane = (int)(i & (kWave - 1));
    const int64_t blk = i / kWave;  // tile * steps + step
    const int64_t tile = blk / steps, step = blk - tile * steps;
    const bf16_t* src = w + (tile * 16 + (lane & 15)) * ldw + step * 32 + 8 * (lane >> 4);
    *reinterpret_cast<uint4*>(out + i * 8) = *reinterpret_cast<const uint4*>(src);
  }
}

// Second pass of the argmax form: one workgroup per row combines the row's tile
// candidates. Each thread loads its share of the candidates up front (16-byte
// vectors), so the row is one round of loads. The comparison is a total order,
// so the reduction order does not matter.
constexpr int kArgmaxMergeThreads = 256;
constexpr int kArgmaxMergeVecs = 4;  // 16-byte vectors (4 candidates) per thread per batch

// With an embedding table, a row whose bank_slots entry is >= 0 also has the
// embedding row of its token copied to that hidden-bank row: the next token's
// prelude (an embedding lookup) fused into the coda.
struct ArgmaxEmbed {
  const bf16_t* embed;       // [embed_rows, width] or null
  bf16_t* bank;              // [bank_rows, width]
  const int64_t* bank_slots; // [rows]; < 0: no successor
  int64_t embed_rows, bank_rows;
  int32_t width;
};

__global__ void __launch_bounds__(kArgmaxMergeThreads) linear_argmax_merge_kernel(const float* best_val,
                                                                                  const int32_t* best_idx,
                                                                                  int32_t tiles, int64_t* out,
                                                                                  int32_t rows, ArgmaxEmbed E) {
  __shared__ float sv[kArgmaxMergeThreads / kWave];
  __shared__ int si[kArgmaxMergeThreads / kWave];
  __shared__ int token_lds;
  const int row = blockIdx.x;
  if (row >= rows) return;
  const float* v = best_val + (int64_t)row * tiles;
  const int32_t* ix = best_idx + (int64_t)row * tiles;
  float best = -INFINITY;
  int bi = 0x7fffffff;
  // Whole vectors while the row's candidates are 16-byte aligned (tiles % 4 == 0 and
  // row bases aligned); the remainder one by one.
  const int nvec = (tiles % 4 == 0) ? tiles / 4 : 0;
  for (int base = threadIdx.x; base < nvec; base += kArgmaxMergeThreads * kArgmaxMergeVecs) {
    float4 vv[kArgmaxMergeVecs];
    int4 iv[kArgmaxMergeVecs];
#pragma unroll
    for (int u = 0; u < kArgmaxMergeVecs; ++u) {
      const int q = min(base + u * kArgmaxMergeThreads, nvec - 1);
      vv[u] = reinterpret_cast<const float4*>(v)[q];
      iv[u] = reinterpret_cast<const int4*>(ix)[q];
    }
#pragma unroll
    for (int u = 0; u < kArgmaxMergeVecs; ++u) {
      if (base + u * kArgmaxMergeThreads >= nvec) continue;
      if (argmax_better(vv[u].x, iv[u].x, best, bi)) { best = vv[u].x; bi = iv[u].x; }
      if (argmax_better(vv[u].y, iv[u].y, best, bi)) { best = vv[u].y; bi = iv[u].y; }
      if (argmax_better(vv[u].z, iv[u].z, best, bi)) { best = vv[u].z; bi = iv[u].z; }
      if (argmax_better(vv[u].w, iv[u].w, best, bi)) { best = vv[u].w; bi = iv[u].w; }
    }
  }
  for (int e = nvec * 4 + threadIdx.x; e < tiles; e += kArgmaxMergeThreads)
    if (argmax_better(v[e], ix[e], best, bi)) { best = v[e]; bi = ix[e]; }
#pragma unroll
  for (int mask = 32; mask >= 1; mask >>= 1) {
    const float ov = shfl_xor_f32(best, mask);
    const int oi = __shfl_xor(bi, mask, 64);
    if (argmax_better(ov, oi, best, bi)) { best = ov; bi = oi; }
  }
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) {
    sv[wave] = best;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kArgmaxMergeThreads / kWave; ++w)
      if (argmax_better(sv[w], si[w], best, bi)) { best = sv[w]; bi = si[w]; }
    out[row] = bi;
    token_lds = bi;
  }
  if (E.embed == nullptr) return;
  const int64_t slot = E.bank_slots[row];
  if (slot < 0 || slot >= E.bank_rows) return;  // block-uniform
  __syncthreads();
  const int64_t token = token_lds;
  if (token < 0 || token >= E.embed_rows) return;
  const uint4* src = reinterpret_cast<const uint4*>(E.embed + token * E.width);
  uint4* dst = reinterpret_cast<uint4*>(E.bank + slot * E.width);
  for (int v = threadIdx.x; v < E.width / 8; v += kArgmaxMergeThreads) dst[v] = src[v];
}

// Launch shape of one instantiation: threads per workgroup are capped so the
// accumulators and a batch of loads fit without spilling, and the LDS partial
// tiles (SLOTS x NT x MT x 1 KiB) stay within 64 KiB.
template <int MT, int NB, int S, bool GATED> struct LinearShape {
  static constexpr int kNT = GATED ? 2 * NB : NB;
  static constexpr int kRegs = 4 * (kNT * S + MT * S + kNT * MT);
  static constexpr int kThreads = kRegs <= 96 ? 1024 : 512;
  static constexpr int kSlots = 64 / (kNT * MT) < 8 ? 64 / (kNT * MT) : 8;
  static constexpr int kMaxWaves = kThreads / kWave < kLinearMaxWaves ? kThreads / kWave : kLinearMaxWaves;
};

// Steps per wave: an even share of K over at most max_waves waves, rounded up to
// whole batches of `batch` steps.
inline int linear_steps_per_wave(int32_t in_features, int batch, int max_waves) {
  const int total = in_features / 32;
  const int per_wave = (total + max_waves - 1) / max_waves;
  return (per_wave + batch - 1) / batch * batch;
}

template <int MT, int NB, int S, bool GATED, bool ARGMAX = false>
int launch_linear(LinearParams prm, hipStream_t stream, int max_waves = kLinearMaxWaves) {
  using Shape = LinearShape<MT, NB, S, GATED>;
  if (prm.N % (16 * NB)) return CDB_ERR_SHAPE;
  const int waves_cap = max_waves < Shape::kMaxWaves ? max_waves : Shape::kMaxWaves;
  prm.steps_per_wave = linear_steps_per_wave(prm.K, S, waves_cap);
  const int nwaves = (prm.K / 32 + prm.steps_per_wave - 1) / prm.steps_per_wave;
  hipLaunchKernelGGL((linear_kernel<MT, NB, S, Shape::kSlots, GATED, Shape::kThreads, ARGMAX>),
                     dim3(prm.N / (16 * NB)), dim3(nwaves * kWave), 0, stream, prm);
  return hipGetLastError() == hipSuccess ? CDB_OK : CDB_ERR_HIP;
}

}  // namespace cdb

using namespace cdb;

namespace {

// Tile choice, from a sweep over (NB, S, waves) at the Ouro-1.4B and Huginn-0125
// projection shapes with cold weights: two column tiles per workgroup once N is
// wide enough to keep more than 128 workgroups; otherwise one, so N = 2048
// still spreads over 128 CUs. Batches of 4 steps (2 at four row tiles, for
// registers); 8 waves per workgroup for one row tile, 4 above.
template <int MT, int S>
int dispatch_rows(const LinearParams& prm, bool gated, int max_waves, hipStream_t stream) {
  const bool wide = prm.N >= 4096 && prm.N % 32 == 0;
  if (wide) {
    return gated ? launch_linear<MT, 2, S, true>(prm, stream, max_waves)
                 : launch_linear<MT, 2, S, false>(prm, stream, max_waves);
  }
  return gated ? launch_linear<MT, 1, S, true>(prm, stream, max_waves)
               : launch_linear<MT, 1, S, false>(prm, stream, max_waves);
}

// Wide-tile path: batches of 33 to 256 rows over 2048-wide inputs with outputs
// of 4096+ columns (the Ouro-1.4B QKV and gate/up projections). Tiles from a
// sweep over (row tiles, column tiles, chunk, stages, pipelined x reads) with
// cold weights; the pipelined form wins only where a wave has 16 or more MFMAs
// per step to hide its reads behind (the gated projection above 64 rows).
bool wide_path(const LinearParams& prm) {
  // 5280-wide inputs (the Huginn QKV and gate/up projections) between 65 and 128 rows.
  if (prm.K == 5280) return prm.M > 64 && prm.M <= 128 && prm.N >= 4096 && prm.N % 16 == 0;
  return prm.M > 32 && prm.M <= kLinearWideMaxRows && prm.K == 2048 && prm.N >= 4096 && prm.N % 128 == 0;
}

int dispatch_wide(const LinearParams& prm, bool gated, hipStream_t stream) {
  if (prm.K == 5280) {  // 128-row tiles, from a cold-weight sweep at 64-128 rows
    return gated ? launch_linear_wide<8, 1, 2, 4, true, 165, 1, true>(prm, stream)
                 : launch_linear_wide<8, 1, 2, 4, false, 165, 1, true>(prm, stream);
  }
  if (prm.M <= 64) {
    return gated ? launch_linear_wide<2, 1, 4, 4, true, 64>(prm, stream)
                 : launch_linear_wide<2, 1, 4, 4, false, 64>(prm, stream);
  }
  if (prm.M <= 128) {
    return gated ? launch_linear_wide<4, 1, 2, 4, true, 64, 1, false, true>(prm, stream)
                 : launch_linear_wide<4, 1, 2, 4, false, 64>(prm, stream);
  }
  return gated ? launch_linear_wide<8, 1, 2, 4, true, 64, 1, false, true>(prm, stream)
               : launch_linear_wide<4, 2, 2, 4, false, 64>(prm, stream);
}

// Split-K form: 2048- and 5632-wide inputs into outputs of a multiple of 64
// columns (the Ouro O and down projections), fp32 partials per K range. Split
// counts and tiles from a sweep with cold weights, timed together with the
// residual RMSNorm that adds the partials: four ranges up to 64 rows; above,
// two for the 2048-wide input (whose partials would cost more than the
// parallelism buys) up to 128 rows, four for the 5632-wide one up to 256. The
// 5632-wide input takes eight ranges up to 16 rows: 2048 outputs are 32 column
// ranges, so eight ranges fill 256 CUs where four leave half of them idle.
// Returns 0 for shapes without a split form.
int parts_splits(int64_t rows, int32_t out_features, int32_t in_features) {
  if (rows < 1 || rows > kLinearWideMaxRows || out_features < 64 || out_features % 16) return 0;
  if (out_features % 64 == 0) {
    if (in_features == 2048) return rows <= 64 ? 4 : rows <= 128 ? 2 : 0;
    if (in_features == 5632) return rows <= 16 ? 8 : 4;
  }
  // The Huginn O (5280 -> 5280) and down (17920 -> 5280) projections: 5280 columns are
  // 82.5 column ranges of 64, so the last range is half full. Split counts from the same
  // cold-weight sweep: three ranges for the 5280-wide input; eight for the 17920-wide one
  // up to 64 rows, four above.
  if (in_features == 5280) return 3;
  if (in_features == 17920) return rows <= 64 ? 8 : 4;
  return 0;
}

int dispatch_parts(const LinearParams& prm, hipStream_t stream) {
  if (prm.K == 2048) {
    if (prm.M <= 32) return launch_linear_wide<1, 1, 4, 4, false, 16, 4>(prm, stream);
    if (prm.M <= 64) return launch_linear_wide<2, 1, 4, 4, false, 16, 4>(prm, stream);
    return launch_linear_wide<2, 1, 4, 4, false, 32, 2>(prm, stream);
  }
  if (prm.K == 5632) {
    if (prm.M <= 16) return launch_linear_wide<1, 1, 4, 4, false, 22, 8>(prm, stream);
    if (prm.M <= 32) return launch_linear_wide<1, 1, 4, 4, false, 44, 4>(prm, stream);
    if (prm.M <= 64) return launch_linear_wide<2, 1, 4, 4, false, 44, 4>(prm, stream);
    if (prm.M <= 128) return launch_linear_wide<4, 1, 2, 4, false, 44, 4>(prm, stream);
    return launch_linear_wide<8, 1, 2, 4, false, 44, 4, false, true>(prm, stream);  // two row ranges, pipelined
  }
  if (prm.K == 5280) {
    if (prm.M <= 16) return launch_linear_wide<1, 1, 4, 4, false, 55, 3, true>(prm, stream);
    return launch_linear_wide<4, 1, 2, 4, false, 55, 3, true>(prm, stream);
  }
  if (prm.K == 17920) {
    if (prm.M <= 16) return launch_linear_wide<1, 1, 4, 4, false, 70, 8, true>(prm, stream);
    if (prm.M <= 64) return launch_linear_wide<4, 1, 2, 4, false, 70, 8, true>(prm, stream);
    return launch_linear_wide<4, 1, 2, 4, false, 140, 4, true>(prm, stream);
  }
  return CDB_ERR_SHAPE;
}

int dispatch_linear(const LinearParams& prm, bool gated, hipStream_t stream) {
  if (wide_path(prm)) return dispatch_wide(prm, gated, stream);
  if (prm.M <= 16) return dispatch_rows<1, 4>(prm, gated, 8, stream);
  if (prm.M <= 32) return dispatch_rows<2, 4>(prm, gated, 4, stream);
  return dispatch_rows<4, 2>(prm, gated, 4, stream);
}

}  // namespace

extern "C" int cdb_linear_pack_weight(const void* w, int64_t ldw, void* w_packed, int64_t rows, int32_t in_features,
                                     int32_t dtype, hipStream_t stream) {
  if (!w || !w_packed) return CDB_ERR_NULL;
  if (dtype != CDB_DTYPE_BF16) return CDB_ERR_UNSUPPORTED;
  if (rows < 16 || rows % 16 || in_features < 32 || in_features % 32 || ldw < in_features || ldw % 8)
    return CDB_ERR_SHAPE;
  if (((uintptr_t)w & 15) || ((uintptr_t)w_packed & 15)) return CDB_ERR_SHAPE;
  const int64_t units = rows * (int64_t)in_features / 8;
  const int64_t blocks = (units + 255) / 256 < 65536 ? (units + 255) / 256 : 65536;
  hipLaunchKernelGGL(linear_pack_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     static_cast<const bf16_t*>(w), ldw, static_cast<bf16_t*>(w_packed), rows, in_features);
  return hipGetLastError() == hipSuccess ? CDB_OK : CDB_ERR_HIP;
}

extern "C" int cdb_linear(const void* x, int64_t ldx, const void* w_packed, void* y, int64_t ldy, int32_t rows,
                          int32_t out_features, int32_t in_features, int32_t gated, int32_t dtype,
                          hipStream_t stream) {
  if (!x || !w_packed || !y) return CDB_ERR_NULL;
  if (dtype != CDB_DTYPE_BF16) return CDB_ERR_UNSUPPORTED;
  if (rows < 1 || rows > kLinearWideMaxRows || out_features < 16 || out_features % 16 || in_features < 32 ||
      in_features % 32)
    return CDB_ERR_SHAPE;
  if (ldx < in_features || ldy < out_features || ldx % 8 || ldy % 4) return CDB_ERR_SHAPE;
  if (((uintptr_t)x & 15) || ((uintptr_t)w_packed & 15) || ((uintptr_t)y & 7)) return CDB_ERR_SHAPE;

  LinearParams prm;
  prm.x = static_cast<const bf16_t*>(x);
  prm.w = static_cast<const bf16_t*>(w_packed);
  prm.y = static_cast<bf16_t*>(y);
  prm.parts = nullptr;
  prm.ldx = ldx;
  prm.ldy = ldy;
  prm.M = rows;
  prm.N = out_features;
  prm.K = in_features;
  prm.steps_per_wave = 0;
  if (rows > kLinearMaxRows && !wide_path(prm)) return CDB_ERR_SHAPE;
  return dispatch_linear(prm, gated != 0, stream);
}

extern "C" int32_t cdb_linear_parts_splits(int64_t rows, int32_t out_features, int32_t in_features, int32_t dtype) {
  if (dtype != CDB_DTYPE_BF16) return 0;
  return parts_splits(rows, out_features, in_features);
}

extern "C" int cdb_linear_parts(const void* x, int64_t ldx, const void* w_packed, float* parts, int64_t parts_elems,
                                int32_t rows, int32_t out_features, int32_t in_features, int32_t dtype,
                                hipStream_t stream) {
  if (!x || !w_packed || !parts) return CDB_ERR_NULL;
  if (dtype != CDB_DTYPE_BF16) return CDB_ERR_UNSUPPORTED;
  const int splits = parts_splits(rows, out_features, in_features);
  if (splits == 0 || ldx < in_features || ldx % 8) return CDB_ERR_SHAPE;
  if (parts_elems < (int64_t)splits * rows * out_features) return CDB_ERR_SHAPE;
  if (((uintptr_t)x & 15) || ((uintptr_t)w_packed & 15) || ((uintptr_t)parts & 15)) return CDB_ERR_SHAPE;

  LinearParams prm;
  prm.x = static_cast<const bf16_t*>(x);
  prm.w = static_cast<const bf16_t*>(w_packed);
  prm.y = nullptr;
  prm.parts = parts;
  prm.ldx = ldx;
  prm.ldy = out_features;
  prm.M = rows;
  prm.N = out_features;
  prm.K = in_features;
  prm.steps_per_wave = 0;
  return dispatch_parts(prm, stream);
}

extern "C" int64_t cdb_linear_argmax_workspace_bytes(int32_t rows, int32_t out_features) {
  if (rows < 0 || out_features < 16 || out_features % 16) return -1;
  return (int64_t)rows * (out_features / 16) * 8;
}

extern "C" int cdb_linear_argmax(const void* x, int64_t ldx, const void* w_packed, int64_t* out, void* workspace,
                                 int64_t workspace_bytes, int32_t rows, int32_t out_features, int32_t in_features,
                                 const void* embed, void* bank, int64_t bank_rows, const int64_t* bank_slots,
                                 int32_t width, int32_t dtype, hipStream_t stream) {
  if (!x || !w_packed || !out || !workspace) return CDB_ERR_NULL;
  if (embed && (!bank || !bank_slots)) return CDB_ERR_NULL;
  if (embed && (width <= 0 || width % 8 || bank_rows <= 0 || ((uintptr_t)embed & 15) || ((uintptr_t)bank & 15)))
    return CDB_ERR_SHAPE;
  if (dtype != CDB_DTYPE_BF16) return CDB_ERR_UNSUPPORTED;
  if (rows < 1 || rows > kLinearMaxRows || out_features < 16 || out_features % 16 || in_features < 32 ||
      in_features % 32 || ldx < in_features || ldx % 8)
    return CDB_ERR_SHAPE;
  if (((uintptr_t)x & 15) || ((uintptr_t)w_packed & 15) || ((uintptr_t)workspace & 15)) return CDB_ERR_SHAPE;
  const int tiles = out_features / 16;
  if (workspace_bytes < (int64_t)rows * tiles * 8) return CDB_ERR_CAPACITY;

  LinearParams prm;
  prm.x = static_cast<const bf16_t*>(x);
  prm.w = static_cast<const bf16_t*>(w_packed);
  prm.best_val = static_cast<float*>(workspace);
  prm.best_idx = reinterpret_cast<int32_t*>(static_cast<float*>(workspace) + (int64_t)rows * tiles);
  prm.ldx = ldx;
  prm.ldy = out_features;
  prm.M = rows;
  prm.N = out_features;
  prm.K = in_features;
  prm.steps_per_wave = 0;
  static_assert(sizeof(LinearParams) == 64, "LinearParams is preloaded whole");
  // The projection kernel's tile choice (two column tiles per workgroup once N is wide).
  const bool two = out_features >= 4096 && out_features % 32 == 0;
  int rc;
  if (rows <= 16)
    rc = two ? launch_linear<1, 2, 4, false, true>(prm, stream, 8) : launch_linear<1, 1, 4, false, true>(prm, stream, 8);
  else if (rows <= 32)
    rc = two ? launch_linear<2, 2, 4, false, true>(prm, stream, 4) : launch_linear<2, 1, 4, false, true>(prm, stream, 4);
  else
    rc = two ? launch_linear<4, 2, 2, false, true>(prm, stream, 4) : launch_linear<4, 1, 2, false, true>(prm, stream, 4);
  if (rc != CDB_OK) return rc;
  ArgmaxEmbed emb{static_cast<const bf16_t*>(embed), static_cast<bf16_t*>(bank), bank_slots, out_features,
                  bank_rows, width};
  hipLaunchKernelGGL(linear_argmax_merge_kernel, dim3((unsigned)rows), dim3(kArgmaxMergeThreads), 0, stream,
                     prm.best_val, prm.best_idx, tiles, out, rows, emb);
  return hipGetLastError() == hipSuccess ? CDB_OK : CDB_ERR_HIP;
}
