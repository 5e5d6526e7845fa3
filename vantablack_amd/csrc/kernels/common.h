// Shared device helpers for the gfx950 attention kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vtb {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Storage tags for the KV cache element type.
struct kv_f32 { static constexpr int bytes = 4; };
struct kv_f16 { static constexpr int bytes = 2; };
struct kv_bf16 { static constexpr int bytes = 2; };

// One 16-byte load -> 16/bytes f32 values (exact upcast).
template <typename KV> struct Unpack;
template <> struct Unpack<kv_f32> {
  static constexpr int N = 4;
  // Bit-cast the whole vector: clang's __builtin_bit_cast on a single
  // ext-vector element (w.y) reads element 0.
  __device__ static inline void run(u32x4 w, float* o) {
    const f32x4 f = __builtin_bit_cast(f32x4, w);
    o[0] = f.x;
    o[1] = f.y;
    o[2] = f.z;
    o[3] = f.w;
  }
};
template <> struct Unpack<kv_bf16> {
  static constexpr int N = 8;
  // bf16 -> f32 is the 16 bits placed in the high half (exact).
  __device__ static inline void run(u32x4 w, float* o) {
    uint32_t a[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = __builtin_bit_cast(float, a[i] << 16);
      o[2 * i + 1] = __builtin_bit_cast(float, a[i] & 0xffff0000u);
    }
  }
};
template <> struct Unpack<kv_f16> {
  static constexpr int N = 8;
  __device__ static inline void run(u32x4 w, float* o) {
    f16x8 h = __builtin_bit_cast(f16x8, w);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = (float)h[i];
  }
};

// K/V are streamed once per launch: non-temporal loads keep them from
// displacing reusable lines (measured ~10% faster decode at 8K context).
__device__ inline u32x4 load16(const void* p) {
#ifndef VTB_NO_NT_LOADS
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
#else
  return *reinterpret_cast<const u32x4*>(p);
#endif
}

// Data that other workgroups re-read soon (prefill K/V tiles): ordinary
// cached load.
__device__ inline u32x4 load16_cached(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

// DPP lane moves within 16-lane rows (gfx9 encodings).
template <int CTRL>
__device__ inline float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}
constexpr int DPP_XOR1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int DPP_XOR2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int DPP_HALF_MIRROR = 0x141; // lane i <- 7-i within 8
constexpr int DPP_MIRROR = 0x140;      // lane i <- 15-i within 16

// Sum over aligned groups of N lanes; every lane of the group gets the sum.
template <int N>
__device__ inline float group_sum(float v) {
  if constexpr (N >= 2) v += dpp<DPP_XOR1>(v);
  if constexpr (N >= 4) v += dpp<DPP_XOR2>(v);
  if constexpr (N >= 8) v += dpp<DPP_HALF_MIRROR>(v);
  if constexpr (N >= 16) v += dpp<DPP_MIRROR>(v);
  if constexpr (N >= 32) v += __shfl_xor(v, 16, 64);
  if constexpr (N >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}

// Reduce across lanes that are STRIDE apart (STRIDE, 2*STRIDE, ... < 64):
// combines the row groups of a wave that share a column slot.
template <int STRIDE>
__device__ inline float stride_sum(float v) {
#pragma unroll
  for (int m = STRIDE; m < 64; m <<= 1) v += __shfl_xor(v, m, 64);
  return v;
}
template <int STRIDE>
__device__ inline float stride_max(float v) {
#pragma unroll
  for (int m = STRIDE; m < 64; m <<= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

__device__ inline float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// f32 -> cache dtype, round to nearest even (NaN stays a quiet NaN).
__device__ inline uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ inline uint16_t f32_to_f16_rne(float f) {
  _Float16 h = (_Float16)f;  // v_cvt_f16_f32 rounds to nearest even
  return __builtin_bit_cast(uint16_t, h);
}
template <typename KV>
__device__ inline void store_kv(void* base, long long i, float f) {
  if constexpr (KV::bytes == 4)
    ((float*)base)[i] = f;
  else if constexpr (__is_same(KV, kv_f16))
    ((uint16_t*)base)[i] = f32_to_f16_rne(f);
  else
    ((uint16_t*)base)[i] = f32_to_bf16_rne(f);
}

// Cross-workgroup hand-off without device-wide fences.  Agent-scope relaxed
// atomic stores/loads are coherent across the per-XCD L2 caches; ordering
// between a workgroup's data and its arrival counter comes from waiting for
// the stores to complete before the counter atomic is issued.
__device__ inline void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline float load_coherent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// Wait for all of this wave's vector-memory loads, including buffer->LDS
// transfers (their LDS writes have landed when vmcnt reaches zero).
__device__ inline void wait_loads() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

}  // namespace vtb
