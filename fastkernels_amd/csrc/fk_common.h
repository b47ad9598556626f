// Shared device helpers for the gfx950 (CDNA4) kernels of fastkernels_amd.
//
// Everything here is written for 64-lane wavefronts.  Weights and activations
// arrive either as bf16 (stored as raw uint16 bit patterns) or as fp32; all
// arithmetic is fp32.  Vector loads are 16 bytes wide (one `global_load_dwordx4`
// per lane), so every row handled by the streaming kernels must start on a
// 16-byte boundary and hold a multiple of 8 elements; the host entry points
// check both before launching.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/fastkernels_hip.h"

namespace fk {

constexpr int kWave = 64;

// Native 128-bit vector (usable with the nontemporal builtins).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Element conversion
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// Round-to-nearest-even fp32 -> bf16 (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Scalar load of element `i` from a tensor whose dtype is only known at run
// time.  Used for the small per-layer vectors (norm weights, gates, biases).
__device__ __forceinline__ float load_scalar(const void* p, int dtype, size_t i) {
  if (dtype == FK_DTYPE_BF16) return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
  return reinterpret_cast<const float*>(p)[i];
}

__device__ __forceinline__ void store_scalar(void* p, int dtype, size_t i, float v) {
  if (dtype == FK_DTYPE_BF16) {
    reinterpret_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(v);
  } else {
    reinterpret_cast<float*>(p)[i] = v;
  }
}

// Eight consecutive elements, raw.  For bf16 only `a` is used (8 x 16 bit);
// for fp32 `a` and `b` hold the 8 floats.  Keeping the raw registers separate
// from the conversion lets the compiler issue every load of a tile before the
// first use.
template <bool BF16>
struct Raw8 {
  u32x4 a;
  u32x4 b;
};

template <bool BF16>
__device__ __forceinline__ Raw8<BF16> load_raw8(const void* base, size_t elem_index) {
  Raw8<BF16> r;
  if constexpr (BF16) {
    r.a = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(base) + elem_index);
    r.b = u32x4{0, 0, 0, 0};
  } else {
    const u32x4* p = reinterpret_cast<const u32x4*>(reinterpret_cast<const float*>(base) + elem_index);
    r.a = p[0];
    r.b = p[1];
  }
  return r;
}

// Streaming (read-once) variant: non-temporal hint so weight tiles do not
// evict the small, reused activations from L2.
template <bool BF16>
__device__ __forceinline__ Raw8<BF16> load_raw8_stream(const void* base, size_t elem_index) {
  Raw8<BF16> r;
  if constexpr (BF16) {
    r.a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(base) + elem_index));
    r.b = u32x4{0, 0, 0, 0};
  } else {
    const u32x4* p = reinterpret_cast<const u32x4*>(reinterpret_cast<const float*>(base) + elem_index);
    r.a = __builtin_nontemporal_load(p);
    r.b = __builtin_nontemporal_load(p + 1);
  }
  return r;
}

template <bool BF16>
__device__ __forceinline__ void raw8_to_f32(const Raw8<BF16>& r, float out[8]) {
  if constexpr (BF16) {
    out[0] = __uint_as_float(r.a.x << 16);
    out[1] = __uint_as_float(r.a.x & 0xffff0000u);
    out[2] = __uint_as_float(r.a.y << 16);
    out[3] = __uint_as_float(r.a.y & 0xffff0000u);
    out[4] = __uint_as_float(r.a.z << 16);
    out[5] = __uint_as_float(r.a.z & 0xffff0000u);
    out[6] = __uint_as_float(r.a.w << 16);
    out[7] = __uint_as_float(r.a.w & 0xffff0000u);
  } else {
    out[0] = __uint_as_float(r.a.x);
    out[1] = __uint_as_float(r.a.y);
    out[2] = __uint_as_float(r.a.z);
    out[3] = __uint_as_float(r.a.w);
    out[4] = __uint_as_float(r.b.x);
    out[5] = __uint_as_float(r.b.y);
    out[6] = __uint_as_float(r.b.z);
    out[7] = __uint_as_float(r.b.w);
  }
}

template <bool BF16>
__device__ __forceinline__ void load8_f32(const void* base, size_t elem_index, float out[8]) {
  raw8_to_f32<BF16>(load_raw8<BF16>(base, elem_index), out);
}

// fp32 activations (8 consecutive floats, 32 bytes).
__device__ __forceinline__ void load8_act(const float* base, size_t elem_index, float out[8]) {
  const float4* p = reinterpret_cast<const float4*>(base + elem_index);
  float4 a = p[0];
  float4 b = p[1];
  out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
  out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
}

// ---------------------------------------------------------------------------
// Wavefront reductions (64 lanes).  Butterfly order is fixed, so results are
// bitwise reproducible run to run.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
  return v;
}

// Sum over aligned groups of `G` lanes (G a power of two <= 64).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int m = G / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    uint32_t lo = __shfl_xor((uint32_t)(v & 0xffffffffu), m, kWave);
    uint32_t hi = __shfl_xor((uint32_t)(v >> 32), m, kWave);
    uint64_t o = ((uint64_t)hi << 32) | lo;
    v = o > v ? o : v;
  }
  return v;
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }
__device__ __forceinline__ float sigmoid(float g) { return 1.0f / (1.0f + __expf(-g)); }

__host__ __device__ constexpr size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

}  // namespace fk
