// Shared device helpers for the gfx950 attention kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../kargs.h"

namespace vtb {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

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

constexpr int DPP_ROR8 = 0x128;        // lane i <- (i+8) mod 16 within 16, i.e. i ^ 8

// Lane exchange across 16 or 32 lanes without LDS (gfx950 v_permlane16_swap
// / v_permlane32_swap).  Called with x == y == v, the pair afterwards holds
// {v[l], v[l ^ 16]} (or {v[l], v[l ^ 32]}) in every lane l, in some order, so
// a symmetric combine of x and y is the butterfly step.  Inline asm because
// the compiler's builtins for these instructions return the first register
// for both results; the s_nop gives the two wait states a VALU write needs
// before a permlane reads it.  Every lane of the wave must be active.
__device__ inline void xchg16(float& x, float& y) {
  asm("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(x), "+v"(y));
}
__device__ inline void xchg32(float& x, float& y) {
  asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(x), "+v"(y));
}
// v[l] + v[l ^ M] (sum) or max of the two, for M in {8, 16, 32}.
template <int M>
__device__ inline float xor_sum(float v) {
  static_assert(M == 8 || M == 16 || M == 32, "xor_sum: M must be 8, 16 or 32");
  if constexpr (M == 8) return v + dpp<DPP_ROR8>(v);
  float x = v, y = v;
  if constexpr (M == 16) xchg16(x, y); else xchg32(x, y);
  return x + y;
}
template <int M>
__device__ inline float xor_max(float v) {
  static_assert(M == 8 || M == 16 || M == 32, "xor_max: M must be 8, 16 or 32");
  if constexpr (M == 8) return fmaxf(v, dpp<DPP_ROR8>(v));
  float x = v, y = v;
  if constexpr (M == 16) xchg16(x, y); else xchg32(x, y);
  return fmaxf(x, y);
}

// Sum over aligned groups of N lanes; every lane of the group gets the sum.
template <int N>
__device__ inline float group_sum(float v) {
  if constexpr (N >= 2) v += dpp<DPP_XOR1>(v);
  if constexpr (N >= 4) v += dpp<DPP_XOR2>(v);
  if constexpr (N >= 8) v += dpp<DPP_HALF_MIRROR>(v);
  if constexpr (N >= 16) v += dpp<DPP_MIRROR>(v);
  if constexpr (N >= 32) v = xor_sum<16>(v);
  if constexpr (N >= 64) v = xor_sum<32>(v);
  return v;
}

// Max over aligned groups of N lanes; every lane of the group gets it.
template <int N>
__device__ inline float group_max(float v) {
  if constexpr (N >= 2) v = fmaxf(v, dpp<DPP_XOR1>(v));
  if constexpr (N >= 4) v = fmaxf(v, dpp<DPP_XOR2>(v));
  if constexpr (N >= 8) v = fmaxf(v, dpp<DPP_HALF_MIRROR>(v));
  if constexpr (N >= 16) v = fmaxf(v, dpp<DPP_MIRROR>(v));
  if constexpr (N >= 32) v = xor_max<16>(v);
  if constexpr (N >= 64) v = xor_max<32>(v);
  return v;
}

// Reduce across lanes that are STRIDE apart (STRIDE, 2*STRIDE, ... < 64):
// combines the row groups of a wave that share a column slot.
template <int STRIDE>
__device__ inline float stride_sum(float v) {
  static_assert(STRIDE == 8 || STRIDE == 16 || STRIDE == 32 || STRIDE == 64, "stride_sum: unsupported stride");
  if constexpr (STRIDE <= 8) v = xor_sum<8>(v);
  if constexpr (STRIDE <= 16) v = xor_sum<16>(v);
  if constexpr (STRIDE <= 32) v = xor_sum<32>(v);
  return v;
}
template <int STRIDE>
__device__ inline float stride_max(float v) {
  static_assert(STRIDE == 8 || STRIDE == 16 || STRIDE == 32 || STRIDE == 64, "stride_max: unsupported stride");
  if constexpr (STRIDE <= 8) v = xor_max<8>(v);
  if constexpr (STRIDE <= 16) v = xor_max<16>(v);
  if constexpr (STRIDE <= 32) v = xor_max<32>(v);
  return v;
}

__device__ inline float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Power-of-two scaling.  scale_exp(m) is the e for which m * 2^-e lies in
// [2^14, 2^15), from the biased exponent of the magnitude m, clamped to
// [-100, 114] (m = 0 or an f32 subnormal gives 0; NaN or inf give 114 and stay
// NaN / inf); pow2f(e) = 2^e for -126 <= e <= 127.
__device__ inline int scale_exp(float m) {
  const int be = (int)((__builtin_bit_cast(uint32_t, m) >> 23) & 0xffu);
  if (be == 0) return 0;
  const int e = be - 127 - 14;
  return e < -100 ? -100 : e;
}
__device__ inline float pow2f(int e) { return __builtin_bit_cast(float, (uint32_t)(e + 127) << 23); }

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
// Raw buffer resource over [base, base + bytes): loads at offsets >= bytes
// return zero without a memory access (hardware range check).  Word 3 is the
// gfx9 raw-buffer format (32-bit data, no swizzle).
__device__ inline __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
// Agent-coherent (sc1) buffer loads: the counterpart of load_coherent for
// data written by other workgroups with store_coherent.  Built from 32-bit
// loads at consecutive offsets into separate float scalars, which the
// backend merges into one buffer_load_dwordx4 / dwordx2; scalars rather than
// a vector because a bit_cast of one ext-vector element reads element 0
// with this compiler (see Unpack<kv_f32>).
constexpr int kBufSc1 = 16;
__device__ inline float buffer_load_coherent(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kBufSc1));
}
__device__ inline void buffer_load16_coherent(__amdgpu_buffer_rsrc_t r, int off, float& x, float& y, float& z,
                                              float& w) {
  x = buffer_load_coherent(r, off);
  y = buffer_load_coherent(r, off + 4);
  z = buffer_load_coherent(r, off + 8);
  w = buffer_load_coherent(r, off + 12);
}
__device__ inline void buffer_load8_coherent(__amdgpu_buffer_rsrc_t r, int off, float& x, float& y) {
  x = buffer_load_coherent(r, off);
  y = buffer_load_coherent(r, off + 4);
}
// 16-byte agent-coherent (sc1) buffer load / store (whole-vector bit-casts:
// a bit_cast of one ext-vector element reads element 0 with this compiler).
__device__ inline f32x4 buffer_load_f4_coherent(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kBufSc1));
}
__device__ inline void buffer_store_f4_coherent(__amdgpu_buffer_rsrc_t r, int off, f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, kBufSc1);
}

// Split-merge hand-off, XL = true when writer and reader run on one XCD
// and so share its L2: stores stay in the L2 (sc0, group scope; the L2
// acknowledges them) and loads skip only the L1 (sc0).  XL = false: the
// agent-coherent (sc1) forms above, through to memory.  The arrival counter
// atomic is the same in both (atomics are performed past the L2s).
constexpr int kBufSc0 = 1;
template <bool XL>
__device__ inline f32x4 part_load_f4(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, XL ? kBufSc0 : kBufSc1));
}
template <bool XL>
__device__ inline void part_store_f4(__amdgpu_buffer_rsrc_t r, int off, f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, XL ? kBufSc0 : kBufSc1);
}
template <bool XL>
__device__ inline void part_load8(__amdgpu_buffer_rsrc_t r, int off, float& x, float& y) {
  x = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, XL ? kBufSc0 : kBufSc1));
  y = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off + 4, 0, XL ? kBufSc0 : kBufSc1));
}
template <bool XL>
__device__ inline void part_store(float* p, float v) {
  if constexpr (XL)
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  else
    store_coherent(p, v);
}

// Wait for all of this wave's vector-memory loads, including buffer->LDS
// transfers (their LDS writes have landed when vmcnt reaches zero).
__device__ inline void wait_loads() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// Wait until at most N of this wave's vector-memory operations are
// outstanding (they complete in issue order for loads).
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Wait for all of this wave's LDS operations.
__device__ inline void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Gated activations of the FFN (math.zig:154-175): silu(z) * u and the
// tanh-approximate gelu(z) * u, in the reference's operation order with no
// contraction into FMAs (hipcc contracts a*b+c by default; Zig's f32 does
// not).
__device__ inline float silu_mul(float z, float u) {
#pragma clang fp contract(off)
  return z / (1.0f + expf(-z)) * u;
}
__device__ inline float gelu_approx_mul(float z, float u) {
#pragma clang fp contract(off)
  const float inner = 0.7978845608028654f * (z + 0.044715f * z * z * z);
  return 0.5f * z * (1.0f + tanhf(inner)) * u;
}

// sin and cos of an f32 RoPE angle.  The angle (up to ~2^24 rad) is
// reduced in f64: theta / (2 pi) in revolutions, keeping the signed fraction
// (absolute error < 1e-9 rev), then rounded to f32 (< 3e-8 rev) and fed to
// the hardware v_sin / v_cos, which take revolutions.  About ten
// instructions against the library sincosf's large-argument reduction; the
// GPU RoPE tests hold the result to the host libm at 2e-6 of the row.
__device__ inline void rope_sincos(float theta, float* sn, float* cs) {
  const double rev = (double)theta * 0.15915494309189533577;  // 1 / (2 pi)
  const float r = (float)(rev - __builtin_rint(rev));
  *sn = __builtin_amdgcn_sinf(r);
  *cs = __builtin_amdgcn_cosf(r);
}

}  // namespace vtb
