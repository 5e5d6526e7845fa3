// KV-slot append and f32 copy (gfx950).
//
// vtb_kv_append_<kv>: dst[i] = round_to_kv_dtype(src[i]) for i < n.  This is
// the splice of k_cur / v_cur into the cache slot at `pos`
// (src/runtime/forward.zig:267-270 on CPU, :466-468 via the Metal copy_f32
// kernel at src/metal/bridge.m:477-488), widened to the f16/bf16 caches this
// build adds: f32 -> f16 and f32 -> bf16 both round to nearest even.  For a
// prefill of B tokens the B slots are contiguous in the layer-major layout,
// so one launch writes them all (prefill.zig:175-191).
//
// vtb_copy_f32: dst[i] = src[i], the plain Metal copy_f32.
// vtb_fill_u32: dst[i] = value (clears counters).
#include "common.h"

namespace vtb {


template <typename KV>
__device__ inline void append_body(const AppendArgs& a) {
  const long long i0 = ((long long)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i0 >= a.n) return;
  if (a.vec && i0 + 4 <= a.n) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(a.src + i0);
    if constexpr (KV::bytes == 4) {
      *reinterpret_cast<f32x4*>((float*)a.dst + i0) = v;
    } else {
      uint16_t h[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        h[j] = __is_same(KV, kv_f16) ? f32_to_f16_rne(v[j]) : f32_to_bf16_rne(v[j]);
      u32x2 w;
      w.x = (uint32_t)h[0] | ((uint32_t)h[1] << 16);
      w.y = (uint32_t)h[2] | ((uint32_t)h[3] << 16);
      *reinterpret_cast<u32x2*>((uint16_t*)a.dst + i0) = w;
    }
  } else {
    const long long i1 = i0 + 4 < a.n ? i0 + 4 : a.n;
    for (long long i = i0; i < i1; ++i) {
      const float f = a.src[i];
      if constexpr (KV::bytes == 4)
        ((float*)a.dst)[i] = f;
      else
        ((uint16_t*)a.dst)[i] = __is_same(KV, kv_f16) ? f32_to_f16_rne(f) : f32_to_bf16_rne(f);
    }
  }
}

}  // namespace vtb

extern "C" __global__ __launch_bounds__(256) void vtb_kv_append_f32(vtb::AppendArgs a) {
  vtb::append_body<vtb::kv_f32>(a);
}
extern "C" __global__ __launch_bounds__(256) void vtb_kv_append_f16(vtb::AppendArgs a) {
  vtb::append_body<vtb::kv_f16>(a);
}
extern "C" __global__ __launch_bounds__(256) void vtb_kv_append_bf16(vtb::AppendArgs a) {
  vtb::append_body<vtb::kv_bf16>(a);
}

// Unaligned-safe scalar copy: dst and src may be any 4-byte aligned offsets.
extern "C" __global__ __launch_bounds__(256) void vtb_copy_f32(vtb::CopyArgs a) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < a.n) a.dst[i] = a.src[i];
}

extern "C" __global__ __launch_bounds__(256) void vtb_fill_u32(vtb::FillArgs a) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < a.n) a.dst[i] = a.value;
}
