// Device helpers shared by the CDB decode-step kernels (gfx950 / CDNA4).
//
// Storage types: activations and KV pages are either fp32 or bf16. bf16 is
// carried as raw uint16_t bits; all arithmetic happens in fp32 and is rounded
// back with round-to-nearest-even, which is what torch's bf16 ops do.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define CDB_DEVICE __device__ __forceinline__

namespace cdb {

constexpr int kWave = 64;

struct bf16_t {
  uint16_t bits;
};

CDB_DEVICE float bf16_to_f32(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

// fp32 -> bf16 with round-to-nearest-even: one v_cvt_pk_bf16_f32 on gfx950
// (no branch, so surrounding loads stay batched); NaN stays NaN.
CDB_DEVICE uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// Two fp32 values as one word of bf16 (lo in the low half), rounded as f32_to_bf16:
// a single v_cvt_pk_bf16_f32 for both.
typedef float cdb_f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 cdb_bf16x2_t __attribute__((ext_vector_type(2)));
CDB_DEVICE uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((cdb_f32x2_t){lo, hi}, cdb_bf16x2_t));
}

// Round an fp32 value to the nearest bf16 and return it as fp32.
CDB_DEVICE float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// SiLU of a bf16 value x, rounded to bf16: R(x / (1 + e^-x)) with e^-x from the
// hardware exponential and the IEEE division. For every one of the 65536 bf16
// inputs this gives the same bits as the libm expf form and as torch's bf16 SiLU
// (NaN inputs give NaN), which a GPU test checks input by input; so it is only
// for x that is itself a bf16 value.
CDB_DEVICE float silu_bf16(float x) { return round_bf16(x / (1.0f + __expf(-x))); }

// Element traits: load/store one scalar of the storage type as fp32.
template <typename T> struct Elem;
template <> struct Elem<float> {
  static CDB_DEVICE float load(const float* p) { return *p; }
  static CDB_DEVICE void store(float* p, float v) { *p = v; }
  // Rounding applied after every elementwise op of a torch tensor of this dtype.
  static CDB_DEVICE float round(float v) { return v; }
};
template <> struct Elem<bf16_t> {
  static CDB_DEVICE float load(const bf16_t* p) { return bf16_to_f32(p->bits); }
  static CDB_DEVICE void store(bf16_t* p, float v) { p->bits = f32_to_bf16(v); }
  static CDB_DEVICE float round(float v) { return round_bf16(v); }
};

// Vector of N storage elements loaded with the widest aligned loads available.
template <typename T, int N> struct Vec {
  static constexpr int kBytes = N * (int)sizeof(T);
  static_assert(kBytes % 4 == 0, "vector must be a whole number of dwords");
  static constexpr int kWords = kBytes / 4;
  uint32_t w[kWords];

  CDB_DEVICE void load(const T* p) {
    const uint32_t* src = reinterpret_cast<const uint32_t*>(p);
    if constexpr (kWords % 4 == 0) {
#pragma unroll
      for (int i = 0; i < kWords; i += 4) {
        uint4 v = *reinterpret_cast<const uint4*>(src + i);
        w[i] = v.x; w[i + 1] = v.y; w[i + 2] = v.z; w[i + 3] = v.w;
      }
    } else if constexpr (kWords % 2 == 0) {
#pragma unroll
      for (int i = 0; i < kWords; i += 2) {
        uint2 v = *reinterpret_cast<const uint2*>(src + i);
        w[i] = v.x; w[i + 1] = v.y;
      }
    } else {
#pragma unroll
      for (int i = 0; i < kWords; ++i) w[i] = src[i];
    }
  }
  // The same loads with the nontemporal hint: for data read once and streamed, so it
  // displaces less of what the caches hold.
  CDB_DEVICE void load_nt(const T* p) {
    typedef uint32_t u32x4_nt __attribute__((ext_vector_type(4)));
    typedef uint32_t u32x2_nt __attribute__((ext_vector_type(2)));
    const uint32_t* src = reinterpret_cast<const uint32_t*>(p);
    if constexpr (kWords % 4 == 0) {
#pragma unroll
      for (int i = 0; i < kWords; i += 4) {
        const u32x4_nt v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_nt*>(src + i));
        w[i] = v.x; w[i + 1] = v.y; w[i + 2] = v.z; w[i + 3] = v.w;
      }
    } else if constexpr (kWords % 2 == 0) {
#pragma unroll
      for (int i = 0; i < kWords; i += 2) {
        const u32x2_nt v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_nt*>(src + i));
        w[i] = v.x; w[i + 1] = v.y;
      }
    } else {
#pragma unroll
      for (int i = 0; i < kWords; ++i) w[i] = __builtin_nontemporal_load(src + i);
    }
  }
  CDB_DEVICE void store(T* p) const {
    uint32_t* dst = reinterpret_cast<uint32_t*>(p);
    if constexpr (kWords % 4 == 0) {
#pragma unroll
      for (int i = 0; i < kWords; i += 4)
        *reinterpret_cast<uint4*>(dst + i) = make_uint4(w[i], w[i + 1], w[i + 2], w[i + 3]);
    } else if constexpr (kWords % 2 == 0) {
#pragma unroll
      for (int i = 0; i < kWords; i += 2) *reinterpret_cast<uint2*>(dst + i) = make_uint2(w[i], w[i + 1]);
    } else {
#pragma unroll
      for (int i = 0; i < kWords; ++i) dst[i] = w[i];
    }
  }
  CDB_DEVICE float get(int i) const {
    if constexpr (sizeof(T) == 4) {
      return __uint_as_float(w[i]);
    } else {
      uint32_t word = w[i >> 1];
      return (i & 1) ? __uint_as_float(word & 0xffff0000u) : __uint_as_float(word << 16);
    }
  }
  // Elements i and i + 1 (i even) at once.
  CDB_DEVICE void set_pair(int i, float a, float b) {
    if constexpr (sizeof(T) == 4) {
      w[i] = __float_as_uint(a);
      w[i + 1] = __float_as_uint(b);
    } else {
      w[i >> 1] = pack_bf16x2(a, b);
    }
  }
  CDB_DEVICE void set(int i, float v) {
    if constexpr (sizeof(T) == 4) {
      w[i] = __float_as_uint(v);
    } else {
      uint32_t b = f32_to_bf16(v);
      uint32_t& word = w[i >> 1];
      word = (i & 1) ? ((word & 0x0000ffffu) | (b << 16)) : ((word & 0xffff0000u) | b);
    }
  }
};

// Workgroup barrier for LDS hand-offs that leaves global loads in flight:
// waits only for this wave's LDS operations (lgkmcnt) and then meets the other
// waves. __syncthreads() is a release/acquire fence plus barrier, which also
// waits for every outstanding global load (vmcnt 0) and so drains any
// prefetch pipeline at each barrier. The "memory" clobber keeps the compiler
// from moving LDS accesses across it.
CDB_DEVICE void lds_barrier() { __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// DPP row rotate by n within each 16-lane row. Used only for all-lane row reductions,
// which give every lane of the row the same result whichever way the rotation runs.
template <int kCtrl> CDB_DEVICE float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xf, 0xf, false));
}
constexpr int kRowRor1 = 0x121, kRowRor2 = 0x122, kRowRor4 = 0x124, kRowRor8 = 0x128;

// Sum across the 16 lanes of a DPP row; every lane of the row receives the total.
CDB_DEVICE float row16_sum(float v) {
  v += dpp_f32<kRowRor8>(v);
  v += dpp_f32<kRowRor4>(v);
  v += dpp_f32<kRowRor2>(v);
  v += dpp_f32<kRowRor1>(v);
  return v;
}
CDB_DEVICE float row16_max(float v) {
  v = fmaxf(v, dpp_f32<kRowRor8>(v));
  v = fmaxf(v, dpp_f32<kRowRor4>(v));
  v = fmaxf(v, dpp_f32<kRowRor2>(v));
  v = fmaxf(v, dpp_f32<kRowRor1>(v));
  return v;
}

// Greedy-argmax order (torch.argmax): a NaN counts as the maximum; among equal
// values (and among NaNs) the smaller index wins. True when (a, ia) beats (b, ib).
CDB_DEVICE bool argmax_better(float a, int ia, float b, int ib) {
  const bool na = a != a, nb = b != b;
  if (na || nb) return na && (!nb || ia < ib);
  return a > b || (a == b && ia < ib);
}

CDB_DEVICE float shfl_xor_f32(float v, int mask) {
  int lane = __lane_id();
  return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __float_as_int(v)));
}

CDB_DEVICE float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += shfl_xor_f32(v, m);
  return v;
}
CDB_DEVICE float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, shfl_xor_f32(v, m));
  return v;
}

// Exact fp32 product and sum without contraction into an FMA, matching two
// separately rounded torch elementwise ops.
// The pragma clears the contract flag on these instructions, so the backend
// cannot fuse a product into a following add after inlining.
CDB_DEVICE float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
CDB_DEVICE float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}
CDB_DEVICE float sub_rn(float a, float b) {
#pragma clang fp contract(off)
  return a - b;
}

}  // namespace cdb
