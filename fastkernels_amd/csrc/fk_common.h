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

// Operand and accumulator types of v_mfma_f32_16x16x32_bf16.
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two floats to packed bf16 (a in the low half) by the hardware conversion
// (v_cvt_pk_bf16_f32, round to nearest even).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

// Eight floats split as hi = bf16(v) and lo = bf16(v - hi) (both round to
// nearest even), packed two per dword: MFMA operands whose products keep
// about 16 bits of each value.
__device__ __forceinline__ void split_hi_lo8(const float (&v)[8], u32x4& hi, u32x4& lo) {
  uint32_t h[4], l[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    h[p] = pack_bf16x2(v[2 * p], v[2 * p + 1]);
    l[p] = pack_bf16x2(v[2 * p] - __uint_as_float(h[p] << 16), v[2 * p + 1] - __uint_as_float(h[p] & 0xffff0000u));
  }
  hi = u32x4{h[0], h[1], h[2], h[3]};
  lo = u32x4{l[0], l[1], l[2], l[3]};
}

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

// Raw bits of N elements p[base + i * stride] of a bf16 (BF) or fp32 array;
// elements from n_valid on repeat element 0, so p[base] must exist and the
// caller ignores them.  The loads are straight-line, with no per-lane branch,
// no zeroed destination and no conversion beside them: any of those makes
// the compiler wait for every load in flight (the weight tiles included)
// right there.  Bits are turned into values where they are used.
template <bool BF, int N>
__device__ __forceinline__ void gather_raw(const void* p, size_t base, size_t stride, int n_valid, uint32_t (&out)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const size_t idx = base + (size_t)(i < n_valid ? i : 0) * stride;
    out[i] = BF ? (uint32_t)reinterpret_cast<const uint16_t*>(p)[idx] : reinterpret_cast<const uint32_t*>(p)[idx];
  }
}

// Element i of a bf16 or fp32 vector whose dtype is a run-time code, in two
// halves: elem_word() loads the aligned 32-bit word holding it with an
// address chosen arithmetically (no branch, so the load does not make the
// compiler wait for the loads before it), elem_value() decodes it where it
// is used.  For bf16 the word may start up to 2 bytes before the element
// (same aligned word, so the same page).
__device__ __forceinline__ uint32_t elem_word(const void* p, int dtype, size_t i) {
  const uintptr_t at = reinterpret_cast<uintptr_t>(p) + (dtype == FK_DTYPE_BF16 ? i * 2 : i * 4);
  return *reinterpret_cast<const uint32_t*>(at & ~(uintptr_t)3);
}
__device__ __forceinline__ float elem_value(uint32_t w, const void* p, int dtype, size_t i) {
  if (dtype != FK_DTYPE_BF16) return __uint_as_float(w);
  const bool high = ((reinterpret_cast<uintptr_t>(p) + i * 2) & 2) != 0;
  return __uint_as_float((high ? w >> 16 : w & 0xffffu) << 16);
}

template <bool BF>
__device__ __forceinline__ float raw_value(uint32_t r) {
  return __uint_as_float(BF ? r << 16 : r);
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

// Eight consecutive elements of a tensor whose dtype is a run-time code
// (uniform branch; both arms are 16-byte vector loads).  Needs 16-byte
// alignment of `base` and an element index that is a multiple of 8.
__device__ __forceinline__ void load8_any(const void* base, int dtype, size_t elem_index, float out[8]) {
  if (dtype == FK_DTYPE_BF16) {
    load8_f32<true>(base, elem_index, out);
  } else {
    load8_f32<false>(base, elem_index, out);
  }
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
// Wavefront all-reductions (64 lanes) built from DPP lane permutes and the
// gfx950 row swaps (v_permlane16_swap, v_permlane32_swap): no LDS round trip.
// Every lane ends with the full result; the combine order is fixed, so
// results are bitwise reproducible run to run.
//   step 1  quad_perm [1,0,3,2]    partner = lane ^ 1
//   step 2  quad_perm [2,3,0,1]    partner = lane ^ 2
//   step 3  row_half_mirror        partner = 7 - lane within 8 (other quad)
//   step 4  row_mirror             partner = 15 - lane within 16 (other 8)
//   step 5  v_permlane16_swap      partner = lane ^ 16
//   step 6  v_permlane32_swap      partner = lane ^ 32
// Steps 3 and 4 are not xor partners, but after steps 1-2 (resp. 1-3) all
// lanes of the source group hold the same partial, so any lane of the other
// group is an equivalent partner.
// ---------------------------------------------------------------------------
constexpr int kDppQuadXor1 = 0xB1;
constexpr int kDppQuadXor2 = 0x4E;
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}

// Value held by lane ^ 16: v_permlane16_swap exchanges the odd rows of its
// first operand with the even rows of its second, so with both operands v
// the first result holds rows (0,0,2,2) and the second rows (1,1,3,3).
__device__ __forceinline__ uint32_t xor16_u32(uint32_t v) {
  auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return ((__lane_id() >> 4) & 1) ? (uint32_t)r[0] : (uint32_t)r[1];
}

// Value held by lane ^ 32.
__device__ __forceinline__ uint32_t xor32_u32(uint32_t v) {
  auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return (__lane_id() < 32) ? (uint32_t)r[1] : (uint32_t)r[0];
}

template <typename Op>
__device__ __forceinline__ float wave_allreduce_f32(float v, Op op) {
  v = op(v, __uint_as_float(dpp_u32<kDppQuadXor1>(__float_as_uint(v))));
  v = op(v, __uint_as_float(dpp_u32<kDppQuadXor2>(__float_as_uint(v))));
  v = op(v, __uint_as_float(dpp_u32<kDppRowHalfMirror>(__float_as_uint(v))));
  v = op(v, __uint_as_float(dpp_u32<kDppRowMirror>(__float_as_uint(v))));
  v = op(v, __uint_as_float(xor16_u32(__float_as_uint(v))));
  v = op(v, __uint_as_float(xor32_u32(__float_as_uint(v))));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
  return wave_allreduce_f32(v, [](float a, float b) { return a + b; });
}

__device__ __forceinline__ float wave_max(float v) {
  return wave_allreduce_f32(v, [](float a, float b) { return fmaxf(a, b); });
}

// Eight wavefront sums at once, transposed: lane l ends with the sum over
// all 64 lanes of d[l >> 3] (lanes 8r .. 8r + 7 hold row r's total).  Each
// step halves the values per lane while pairing lanes:
//   v_permlane32_swap on (d[i], d[i+4]): lanes < 32 keep value i, lanes
//     >= 32 value i + 4, each summed over {l, l ^ 32};
//   v_permlane16_swap on (e[i], e[i+2]): value i + 2 (l >> 4), over
//     {l ^ 0, 16, 32, 48};
//   row_ror:8 (partner l ^ 8 within the 16-lane row) with each lane keeping
//     the value of its own bit 3: value l >> 3, over 8 lanes;
//   quad xor 1, quad xor 2, row half mirror: over the remaining 8 lanes.
// 22 instructions instead of eight 12-instruction reductions; fixed order.
constexpr int kDppRowRor8 = 0x128;
__device__ __forceinline__ float rows8_sum(const float (&d)[8]) {
  float e[4], f[2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(d[i]), __float_as_uint(d[i + 4]), false, false);
    e[i] = __uint_as_float((uint32_t)r[0]) + __uint_as_float((uint32_t)r[1]);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(e[i]), __float_as_uint(e[i + 2]), false, false);
    f[i] = __uint_as_float((uint32_t)r[0]) + __uint_as_float((uint32_t)r[1]);
  }
  const bool b3 = (__lane_id() >> 3) & 1;
  const float keep = b3 ? f[1] : f[0], give = b3 ? f[0] : f[1];
  float g = keep + __uint_as_float(dpp_u32<kDppRowRor8>(__float_as_uint(give)));
  g += __uint_as_float(dpp_u32<kDppQuadXor1>(__float_as_uint(g)));
  g += __uint_as_float(dpp_u32<kDppQuadXor2>(__float_as_uint(g)));
  g += __uint_as_float(dpp_u32<kDppRowHalfMirror>(__float_as_uint(g)));
  return g;
}

// Four wavefront sums at once, transposed the same way: lane l ends with
// the sum over all 64 lanes of d[l >> 4] (14 instructions instead of 48).
__device__ __forceinline__ float rows4_sum(const float (&d)[4]) {
  float e[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(d[i]), __float_as_uint(d[i + 2]), false, false);
    e[i] = __uint_as_float((uint32_t)r[0]) + __uint_as_float((uint32_t)r[1]);
  }
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(e[0]), __float_as_uint(e[1]), false, false);
  float g = __uint_as_float((uint32_t)r[0]) + __uint_as_float((uint32_t)r[1]);
  g += __uint_as_float(dpp_u32<kDppQuadXor1>(__float_as_uint(g)));
  g += __uint_as_float(dpp_u32<kDppQuadXor2>(__float_as_uint(g)));
  g += __uint_as_float(dpp_u32<kDppRowHalfMirror>(__float_as_uint(g)));
  g += __uint_as_float(dpp_u32<kDppRowMirror>(__float_as_uint(g)));
  return g;
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  auto step = [&](uint32_t lo, uint32_t hi) { v = max_u64(v, ((uint64_t)hi << 32) | lo); };
  step(dpp_u32<kDppQuadXor1>((uint32_t)v), dpp_u32<kDppQuadXor1>((uint32_t)(v >> 32)));
  step(dpp_u32<kDppQuadXor2>((uint32_t)v), dpp_u32<kDppQuadXor2>((uint32_t)(v >> 32)));
  step(dpp_u32<kDppRowHalfMirror>((uint32_t)v), dpp_u32<kDppRowHalfMirror>((uint32_t)(v >> 32)));
  step(dpp_u32<kDppRowMirror>((uint32_t)v), dpp_u32<kDppRowMirror>((uint32_t)(v >> 32)));
  step(xor16_u32((uint32_t)v), xor16_u32((uint32_t)(v >> 32)));
  step(xor32_u32((uint32_t)v), xor32_u32((uint32_t)(v >> 32)));
  return v;
}

// ---------------------------------------------------------------------------
// Cross-workgroup publication without cache-wide fences.
//
// A device-scope fence costs a chip-wide L2 write-back/invalidate (measured
// on MI355X: ~60 ns per workgroup, serialised).  Small values that other
// workgroups must read are instead written with device-scope atomic stores
// (write-through, `sc1`) and read with device-scope atomic loads (`sc1`,
// served from the coherent level); `publish_wait()` makes the storing
// wavefront wait until its stores are acknowledged before it signals with a
// device-scope atomic RMW.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_coherent(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int load_coherent(const int* p) {
  return __hip_atomic_load(const_cast<int*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void publish_wait() { __builtin_amdgcn_s_waitcnt(0); }
__device__ __forceinline__ uint32_t ticket_add(uint32_t* p) {
  return __hip_atomic_fetch_add(p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t load_coherent(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_coherent(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Tagged values: an fp32 value and a 32-bit launch tag in one naturally
// aligned 8-byte word, stored and loaded as single-copy-atomic coherent
// accesses.  A consumer that reads the tag of the current launch knows the
// value beside it is this launch's, with no counter or barrier between
// producer and consumer.
__device__ __forceinline__ void store_tagged(uint64_t* p, float v, uint32_t tag) {
  __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t load_tagged(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t tag_of(uint64_t w) { return (uint32_t)(w >> 32); }
__device__ __forceinline__ float value_of(uint64_t w) { return __uint_as_float((uint32_t)w); }

// Bounded poll of N tagged words of this lane (src[j] == nullptr: no word):
// re-reads every word that does not carry `tag` yet, all reads of one round
// in flight together, until all carry it or `limit` rounds have passed
// (limit 0: gives up at once).  Returns whether all carry the tag.
constexpr uint32_t kPollLimit = 1u << 16;
template <int N>
__device__ __forceinline__ bool poll_tagged(uint64_t (&w)[N], const uint64_t* const (&src)[N], uint32_t tag,
                                            uint32_t limit) {
  for (uint32_t i = 0; i < limit; ++i) {
    bool ready = true;
#pragma unroll
    for (int j = 0; j < N; ++j) ready = ready && (src[j] == nullptr || tag_of(w[j]) == tag);
    if (ready) return true;
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int j = 0; j < N; ++j)
      if (src[j] != nullptr && tag_of(w[j]) != tag) w[j] = load_tagged(src[j]);
  }
  return false;
}

// One tagged word whose first read `w` is already issued: its value once it
// carries `tag`.  The common case (the word was stored before the first read)
// is one compare with no loop, so the compiler waits for exactly that load;
// otherwise the word is re-read (every read checked before the next) until
// it carries the tag or `limit` rounds have passed, which clears `ok`.
__device__ __forceinline__ float settle_tagged(uint64_t w, const uint64_t* src, uint32_t tag, uint32_t limit,
                                               bool& ok) {
  if (tag_of(w) == tag) return value_of(w);
  for (uint32_t i = 0; i < limit; ++i) {
    __builtin_amdgcn_s_sleep(1);
    w = load_tagged(src);
    if (tag_of(w) == tag) return value_of(w);
  }
  ok = false;
  return value_of(w);
}

// poll_tagged over a contiguous run: word j of this thread is
// base[first + stride * j] when first + stride * j < n (else no word); the
// addresses are recomputed per round instead of held in registers.
template <int N>
__device__ __forceinline__ bool poll_run(uint64_t (&w)[N], const uint64_t* base, int first, int stride, int n,
                                         uint32_t tag, uint32_t limit) {
#pragma unroll
  for (int j = 0; j < N; ++j) w[j] = first + stride * j < n ? load_tagged(base + first + stride * j) : 0ull;
  for (uint32_t i = 0; i < limit; ++i) {
    bool ready = true;
#pragma unroll
    for (int j = 0; j < N; ++j) ready = ready && (first + stride * j >= n || tag_of(w[j]) == tag);
    if (ready) return true;
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int j = 0; j < N; ++j)
      if (first + stride * j < n && tag_of(w[j]) != tag) w[j] = load_tagged(base + first + stride * j);
  }
  return false;
}

// Grid-wide barrier for kernels whose grid the host has capped at the number
// of co-resident workgroups.  Called by one thread per workgroup after the
// workgroup's publishing stores have been waited for.  The wait is bounded
// (`limit` polls, see wait_limits): a wait that runs out records
// FK_DEVICE_ERR_BARRIER in `*error` and returns false, so a broken launch
// configuration gives flagged, poisoned results but never a hang.
constexpr uint32_t kSpinLimit = 1u << 20;
constexpr uint32_t FK_DEVICE_ERR_BARRIER = 1u;
// A device-held attention position whose step would pass the cache: the
// step's update is NaN and the position is left where it is.
constexpr uint32_t FK_DEVICE_ERR_POSITION = 2u;

__device__ __forceinline__ bool grid_arrive_and_wait(uint32_t* counter, uint32_t target, uint32_t* error,
                                                     uint32_t limit) {
  ticket_add(counter);
  for (uint32_t i = 0; i < limit; ++i) {
    if (load_coherent(counter) >= target) return true;
    __builtin_amdgcn_s_sleep(2);
  }
  __hip_atomic_fetch_or(error, FK_DEVICE_ERR_BARRIER, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return false;
}

// Wait bounds of a launch from its workspace header (16 words: epoch at
// `epoch_word`, host-set poll bound + 1 at word 14, error flag at word 15):
// 0 while the error flag is set (every wait gives up, outputs are NaN),
// else the host's bound, else the built-in one.  `spin` is the grid
// barrier's bound.  Also returns the launch tag, epoch + 1.
struct WaitLimits {
  uint32_t tag;
  uint32_t poll;
  uint32_t spin;
};
// The header words as loaded, turned into limits where they are first
// needed.  A kernel loads them before its other loads and calls limits()
// late: the compiler makes the uniform words scalar right after the load
// otherwise, and that wait (a round trip to the coherent level) would hold
// back every load issued after it.  Loads retire in order, so the late
// wait finds the header words long arrived.
struct WaitHeader {
  uint32_t epoch, set, err;
  __device__ __forceinline__ WaitLimits limits() {
    asm volatile("" : "+v"(epoch), "+v"(set), "+v"(err));
    WaitLimits w;
    w.tag = epoch + 1u;
    w.poll = err ? 0u : set ? set - 1u : kPollLimit;
    w.spin = err ? 0u : set ? set - 1u : kSpinLimit;
    return w;
  }
};
__device__ __forceinline__ WaitHeader load_wait_header(const uint32_t* header, int epoch_word) {
  WaitHeader h;
  h.epoch = load_coherent(&header[epoch_word]);
  h.set = load_coherent(&header[14]);
  h.err = load_coherent(&header[15]);
  return h;
}
__device__ __forceinline__ WaitLimits wait_limits(const uint32_t* header, int epoch_word) {
  return load_wait_header(header, epoch_word).limits();
}

// Workgroup barrier for hand-offs through LDS only: its fences cover LDS
// alone, so it waits for the wavefront's LDS operations and never for its
// global stores.  (On gfx950 without threadgroup split, __syncthreads()
// compiles to the same s_barrier behind an LDS wait; its workgroup-scope
// global fence would wait for the stores' acknowledgements only in a
// threadgroup-split build.)  For kernels whose wavefronts exchange data
// through LDS alone while their global words go to other workgroups, which
// read them by their launch tags.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Poisoned value of an output whose inputs a failed wait left invalid.
__device__ __forceinline__ float poison_if(bool bad, float v) { return bad ? __builtin_nanf("") : v; }

// Integer wave all-reductions (same lane schedule as wave_allreduce_f32).
template <typename Op>
__device__ __forceinline__ int wave_allreduce_i32(int v, Op op) {
  v = op(v, (int)dpp_u32<kDppQuadXor1>((uint32_t)v));
  v = op(v, (int)dpp_u32<kDppQuadXor2>((uint32_t)v));
  v = op(v, (int)dpp_u32<kDppRowHalfMirror>((uint32_t)v));
  v = op(v, (int)dpp_u32<kDppRowMirror>((uint32_t)v));
  v = op(v, (int)xor16_u32((uint32_t)v));
  v = op(v, (int)xor32_u32((uint32_t)v));
  return v;
}
__device__ __forceinline__ int wave_min_i32(int v) {
  return wave_allreduce_i32(v, [](int a, int b) { return a < b ? a : b; });
}
// Unsigned max (integer ops fold into the DPP moves; no float canonicalising).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  return (uint32_t)wave_allreduce_i32((int)v, [](int a, int b) { return (uint32_t)a > (uint32_t)b ? a : b; });
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }
__device__ __forceinline__ float sigmoid(float g) { return 1.0f / (1.0f + __expf(-g)); }

__host__ __device__ constexpr size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// ---------------------------------------------------------------------------
// Phase timeline of the single-launch kernels, in diagnostic builds only
// (-DFK_TIMELINE: `python -m fastkernels_amd.build --timeline` builds them
// into a library of their own).  FK_TIMELINE_DECL opens a kernel's marker
// registers; FK_MARK(k) keeps the wall clock (100 MHz) at marker k in the
// calling thread; FK_TIMELINE_COMMIT(unit, row) stores thread 0's markers in
// row `row` (one per workgroup) of the translation unit's device buffer,
// declared with FK_TIMELINE_BUFFER(unit) and read by the host through
// fk_timeline_read_<unit> / fk_timeline_clear_<unit>.  In ordinary builds
// they all expand to nothing.
constexpr int kTimelineMarks = 16;
constexpr int kTimelineRows = 1024;
#ifdef FK_TIMELINE
#define FK_TIMELINE_DECL unsigned long long fk_tl_[fk::kTimelineMarks] = {}
#define FK_MARK(k) (fk_tl_[(k)] = wall_clock64())
#define FK_TIMELINE_COMMIT(unit, row)                                                     \
  do {                                                                                    \
    if (threadIdx.x == 0 && (row) < fk::kTimelineRows)                                    \
      for (int i_ = 0; i_ < fk::kTimelineMarks; ++i_)                                     \
        fk_tl_buf_##unit[(size_t)(row) * fk::kTimelineMarks + i_] = fk_tl_[i_];           \
  } while (0)
#define FK_TIMELINE_BUFFER(unit)                                                                          \
  static __device__ unsigned long long fk_tl_buf_##unit[fk::kTimelineRows * fk::kTimelineMarks];          \
  extern "C" int fk_timeline_read_##unit(void* host, size_t bytes) {                                     \
    if (!host || bytes > sizeof(fk_tl_buf_##unit)) return FK_ERR_INVALID;                                 \
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(fk_tl_buf_##unit), bytes, 0, hipMemcpyDeviceToHost) ==    \
                   hipSuccess                                                                             \
               ? FK_OK                                                                                    \
               : FK_ERR_LAUNCH;                                                                           \
  }                                                                                                       \
  extern "C" int fk_timeline_clear_##unit() {                                                            \
    static const unsigned long long zeros[fk::kTimelineRows * fk::kTimelineMarks] = {};                  \
    return hipMemcpyToSymbol(HIP_SYMBOL(fk_tl_buf_##unit), zeros, sizeof(zeros), 0, hipMemcpyHostToDevice) == \
                   hipSuccess                                                                             \
               ? FK_OK                                                                                    \
               : FK_ERR_LAUNCH;                                                                           \
  }
#else
#define FK_TIMELINE_DECL \
  do {                   \
  } while (0)
#define FK_MARK(k) ((void)0)
#define FK_TIMELINE_COMMIT(unit, row) ((void)0)
#define FK_TIMELINE_BUFFER(unit)
#endif

}  // namespace fk
