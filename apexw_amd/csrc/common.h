// Device helpers shared by the ApexW HIP kernels (gfx950 / CDNA4).
//
// Rounding helpers reproduce torch's CPU storage rounding: every value written to
// a bf16/fp16 tensor is rounded to nearest-even from fp32 (v_cvt_pk_bf16_f32 on
// gfx950).  Kernels are compiled with -ffp-contract=off, so a multiply followed by
// an add is only fused where fmaf() is written out, which is where torch's CPU
// kernels use an FMA (add with alpha, addcmul, lerp).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/apexw_hip.h"

#define APEXW_DEV static __device__ __forceinline__

typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;

// Pointers read out of the tensor table are generic; casting them to the global
// address space lets the compiler emit global_load/global_store instead of flat.
#define APEXW_GLOBAL(T, ptr) ((__attribute__((address_space(1))) T*)(ptr))

// ---------------------------------------------------------------------------
// dtype conversions
// ---------------------------------------------------------------------------
APEXW_DEV float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }
APEXW_DEV uint32_t f32_to_bf16_bits(float x) {
  __bf16 b = (__bf16)x;  // round to nearest even
  return (uint32_t)__builtin_bit_cast(uint16_t, b);
}
// Two fp32 values rounded to nearest-even bf16, packed (a in the low half).
APEXW_DEV uint32_t pack_bf16x2(float a, float b) {
  typedef __attribute__((ext_vector_type(2))) float f32x2;
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
}
APEXW_DEV float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
APEXW_DEV uint32_t f32_to_f16_bits(float x) {
  // x is a rounded fp32 value here: without this barrier the compiler folds a
  // preceding multiply or fma into the conversion (v_fma_mixlo_f16, a single
  // rounding of the exact result), which differs from torch's fp32 arithmetic
  // followed by the fp16 store on values that fall on an fp16 tie
  __asm__ volatile("" : "+v"(x));
  _Float16 h = (_Float16)x;
  return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

// Value of x after a round trip through the storage dtype.
template <int DT> APEXW_DEV float rnd(float x) {
  if constexpr (DT == APEXW_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(x));
  else if constexpr (DT == APEXW_F16) return f16_bits_to_f32(f32_to_f16_bits(x));
  else return x;
}

// torch's clamp to the fp16 range, which keeps NaN (fminf / fmaxf alone would not)
APEXW_DEV float clamp_f16_range(float x) { return x == x ? fminf(fmaxf(x, -65504.0f), 65504.0f) : x; }

// Stochastic rounding of fp32 to bf16 / fp16: add uniform random low bits to the
// fp32 bit pattern and truncate (the published "add noise then truncate" SR).
// r is 16 random bits for bf16 and 13 for fp16.  Returns the rounded value as fp32.
template <int DT> APEXW_DEV float sr_round(float x, uint32_t r) {
  if constexpr (DT == APEXW_BF16) {
    uint32_t u = __float_as_uint(x) + (r & 0xFFFFu);
    return __uint_as_float(u & 0xFFFF0000u);
  } else if constexpr (DT == APEXW_F16) {
    x = clamp_f16_range(x);
    uint32_t u = __float_as_uint(x) + (r & 0x1FFFu);
    float y = __uint_as_float(u & 0xFFFFE000u);
    y = clamp_f16_range(y);
    return rnd<APEXW_F16>(y);
  } else {
    return x;
  }
}

template <int DT> struct Elem;
template <> struct Elem<APEXW_F32> { static constexpr int bytes = 4; };
template <> struct Elem<APEXW_BF16> { static constexpr int bytes = 2; };
template <> struct Elem<APEXW_F16> { static constexpr int bytes = 2; };

// Load 8 consecutive elements starting at element index i (16-byte aligned for
// 16-bit types, 32-byte aligned for fp32) into fp32 registers.
template <int DT> APEXW_DEV void load8(const void* base, int64_t i, float (&x)[8]) {
  if constexpr (DT == APEXW_F32) {
    auto p = APEXW_GLOBAL(const u32x4, (const float*)base + i);
    u32x4 a = __builtin_nontemporal_load(p), b = __builtin_nontemporal_load(p + 1);
    x[0] = __uint_as_float(a.x); x[1] = __uint_as_float(a.y); x[2] = __uint_as_float(a.z); x[3] = __uint_as_float(a.w);
    x[4] = __uint_as_float(b.x); x[5] = __uint_as_float(b.y); x[6] = __uint_as_float(b.z); x[7] = __uint_as_float(b.w);
  } else {
    auto p = APEXW_GLOBAL(const u32x4, (const uint16_t*)base + i);
    u32x4 a = __builtin_nontemporal_load(p);
    uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if constexpr (DT == APEXW_BF16) {
        x[2 * k] = bf16_bits_to_f32(w[k] & 0xFFFFu);
        x[2 * k + 1] = __uint_as_float(w[k] & 0xFFFF0000u);
      } else {
        x[2 * k] = f16_bits_to_f32(w[k] & 0xFFFFu);
        x[2 * k + 1] = f16_bits_to_f32(w[k] >> 16);
      }
    }
  }
}

// Store 8 fp32 values that are already representable in DT.
template <int DT> APEXW_DEV void store8(void* base, int64_t i, const float (&x)[8]) {
  if constexpr (DT == APEXW_F32) {
    auto p = APEXW_GLOBAL(u32x4, (float*)base + i);
    u32x4 a = {__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]), __float_as_uint(x[3])};
    u32x4 b = {__float_as_uint(x[4]), __float_as_uint(x[5]), __float_as_uint(x[6]), __float_as_uint(x[7])};
    __builtin_nontemporal_store(a, p);
    __builtin_nontemporal_store(b, p + 1);
  } else {
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if constexpr (DT == APEXW_BF16) {
        w[k] = (__float_as_uint(x[2 * k]) >> 16) | (__float_as_uint(x[2 * k + 1]) & 0xFFFF0000u);
      } else {
        w[k] = f32_to_f16_bits(x[2 * k]) | (f32_to_f16_bits(x[2 * k + 1]) << 16);
      }
    }
    u32x4 a = {w[0], w[1], w[2], w[3]};
    __builtin_nontemporal_store(a, APEXW_GLOBAL(u32x4, (uint16_t*)base + i));
  }
}

template <int DT> APEXW_DEV float load1(const void* base, int64_t i) {
  if constexpr (DT == APEXW_F32) return APEXW_GLOBAL(const float, base)[i];
  else if constexpr (DT == APEXW_BF16) return bf16_bits_to_f32(APEXW_GLOBAL(const uint16_t, base)[i]);
  else return f16_bits_to_f32(APEXW_GLOBAL(const uint16_t, base)[i]);
}

template <int DT> APEXW_DEV void store1(void* base, int64_t i, float x) {
  if constexpr (DT == APEXW_F32) APEXW_GLOBAL(float, base)[i] = x;
  else if constexpr (DT == APEXW_BF16) APEXW_GLOBAL(uint16_t, base)[i] = (uint16_t)(__float_as_uint(x) >> 16);
  else APEXW_GLOBAL(uint16_t, base)[i] = (uint16_t)f32_to_f16_bits(x);
}

// ---------------------------------------------------------------------------
// Counter-based RNG: a keyed integer hash of the element index.
// mix32 is the "lowbias32" 32-bit finaliser (two multiply / xor-shift rounds).
// The key folds (seed, tensor index, step, stream) once per work unit.
// ---------------------------------------------------------------------------
APEXW_DEV uint32_t mix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

APEXW_DEV uint32_t rng_key(uint64_t seed, uint32_t tensor, uint32_t step, uint32_t stream, uint32_t hi_index) {
  uint32_t k = mix32((uint32_t)seed ^ 0x9e3779b9u);
  k = mix32(k ^ (uint32_t)(seed >> 32) ^ (tensor * 0x85ebca6bu));
  k = mix32(k ^ (step * 0xc2b2ae35u) ^ (stream << 24));
  return mix32(k ^ hi_index);
}

// one keyed hash per element: the key is already fully mixed, so a single
// finaliser round over key + index decorrelates neighbouring elements.
APEXW_DEV uint32_t rng_at(uint32_t key, uint32_t index) { return mix32(index + key); }

// ---------------------------------------------------------------------------
// Gradient sanitizing (NaN -> 0, +-Inf -> +-65504 after rounding to the grad dtype)
// ---------------------------------------------------------------------------
template <int GD> APEXW_DEV float sanitize(float g) {
  if (__builtin_isnan(g)) return 0.0f;
  if (__builtin_isinf(g)) return rnd<GD>(g > 0.0f ? 65504.0f : -65504.0f);
  return g;
}

// ---------------------------------------------------------------------------
// Wavefront (64 lanes) reductions
// ---------------------------------------------------------------------------
APEXW_DEV float wave_max(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off, 64));
  return x;
}
APEXW_DEV float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

APEXW_DEV int lane_id() { return (int)(threadIdx.x & 63u); }

// Grid for a 256-thread (4-wave) kernel that strides over `n_units` work units,
// one unit per wave: at most 16 workgroups per resident slot (blocks per CU from
// the kernel's occupancy on the current device).
// An AMP unscale factor the kernels take: finite and non-zero (negative with
// maximize=True, which negates the grads: exact, and commutes with every other
// grad preparation step).
inline bool apexw_inv_scale_ok(float x) { return x == x && x != 0.0f && x - x == 0.0f; }
int apexw_resident_grid(const void* kernel, int64_t n_units);
APEXW_DEV uint32_t uniform(uint32_t x) { return __builtin_amdgcn_readfirstlane(x); }
