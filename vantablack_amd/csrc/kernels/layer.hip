// The small ops of a decode layer around the projections and attention, as
// vantablack's full-GPU layer encodes them (gpuLayerStep,
// src/runtime/forward.zig:419-513; Metal kernels src/metal/bridge.m:88-194):
//   vtb_rmsnorm_f32       out = in * w * inv, inv = 1 / sqrt(sum(in^2)/n + eps)
//                         (math.rmsNorm, src/kernels/math.zig:11-32)
//   vtb_swiglu_f32        gate = gate / (1 + exp(-gate)) * up   (math.zig:154-161)
//   vtb_gelu_approx_f32   gate = 0.5 g (1 + tanh(sqrt(2/pi) (g + 0.044715 g^3))) * up
//                         (math.zig:166-175)
//   vtb_residual_add_f32  a += b                              (math.addInto)
//   vtb_rope_rows_f32     RoPE of rows tokens x heads in place, token t at
//                         position pos0 + t (prefill.zig:180-189: math.rope /
//                         ropeHalf per (batch, head)), with the decode
//                         kernel's angle, sin/cos and operation order
//   vtb_add_rmsnorm_f32   x += b, then out = rmsnorm(x) * w: the residual add
//                         and the rmsnorm that follows it in the layer
//                         (forward.zig:487 and 490, 510 then the next layer's 441),
//                         one launch instead of two, same arithmetic
//
// rmsnorm is one workgroup: a model row is a few tens of KB (the CPU path
// stops at dim 8192, forward.zig:646-648), so the launch is latency-bound and
// a single workgroup avoids a second pass.  Each thread sums the squares of its
// float4 chunks, the waves reduce by DPP and the 16 wave sums meet in LDS in a
// fixed order.  The scale is an IEEE square root and division (not the
// hardware reciprocal square root), as the CPU path computes it.  The
// elementwise kernels take float4s and finish a ragged tail element by
// element.
#include "common.h"

namespace vtb {





}  // namespace vtb

extern "C" __global__ __launch_bounds__(1024) void vtb_rmsnorm_f32(vtb::RmsNormArgs a) {
  __shared__ float s_part[16];
  const int tid = (int)threadIdx.x;
  // Row blockIdx.x of a batch (the prefill's per-token norm).
  a.in += (size_t)blockIdx.x * a.n;
  a.out += (size_t)blockIdx.x * a.n;
  const int n4 = a.n4;
  float ss = 0.0f;
  for (int c = tid; c < n4; c += 1024) {
    const float4 v = reinterpret_cast<const float4*>(a.in)[c];
    ss = fmaf(v.x, v.x, ss);
    ss = fmaf(v.y, v.y, ss);
    ss = fmaf(v.z, v.z, ss);
    ss = fmaf(v.w, v.w, ss);
  }
  for (int i = 4 * n4 + tid; i < a.n; i += 1024) ss = fmaf(a.in[i], a.in[i], ss);
  ss = vtb::group_sum<64>(ss);
  if ((tid & 63) == 0) s_part[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int w = 0; w < 16; ++w) tot += s_part[w];
  const float inv = 1.0f / __builtin_sqrtf(tot / (float)a.n + a.eps);
  for (int c = tid; c < n4; c += 1024) {
    const float4 v = reinterpret_cast<const float4*>(a.in)[c];
    const float4 w = reinterpret_cast<const float4*>(a.w)[c];
    reinterpret_cast<float4*>(a.out)[c] = make_float4(v.x * w.x * inv, v.y * w.y * inv, v.z * w.z * inv, v.w * w.w * inv);
  }
  for (int i = 4 * n4 + tid; i < a.n; i += 1024) a.out[i] = a.in[i] * a.w[i] * inv;
}

// x += b (stored), then the rmsnorm of the new x into out.  Each thread
// re-reads in the second pass exactly the elements it wrote in the first.
extern "C" __global__ __launch_bounds__(1024) void vtb_add_rmsnorm_f32(vtb::AddNormArgs a) {
  __shared__ float s_part[16];
  const int tid = (int)threadIdx.x;
  const int n4 = a.n4;
  float ss = 0.0f;
  for (int c = tid; c < n4; c += 1024) {
    float4 v = reinterpret_cast<const float4*>(a.x)[c];
    const float4 d = reinterpret_cast<const float4*>(a.b)[c];
    v = make_float4(v.x + d.x, v.y + d.y, v.z + d.z, v.w + d.w);
    reinterpret_cast<float4*>(a.x)[c] = v;
    ss = fmaf(v.x, v.x, ss);
    ss = fmaf(v.y, v.y, ss);
    ss = fmaf(v.z, v.z, ss);
    ss = fmaf(v.w, v.w, ss);
  }
  for (int i = 4 * n4 + tid; i < a.n; i += 1024) {
    const float v = a.x[i] + a.b[i];
    a.x[i] = v;
    ss = fmaf(v, v, ss);
  }
  ss = vtb::group_sum<64>(ss);
  if ((tid & 63) == 0) s_part[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int w = 0; w < 16; ++w) tot += s_part[w];
  const float inv = 1.0f / __builtin_sqrtf(tot / (float)a.n + a.eps);
  for (int c = tid; c < n4; c += 1024) {
    const float4 v = reinterpret_cast<const float4*>(a.x)[c];
    const float4 w = reinterpret_cast<const float4*>(a.w)[c];
    reinterpret_cast<float4*>(a.out)[c] = make_float4(v.x * w.x * inv, v.y * w.y * inv, v.z * w.z * inv, v.w * w.w * inv);
  }
  for (int i = 4 * n4 + tid; i < a.n; i += 1024) a.out[i] = a.x[i] * a.w[i] * inv;
}

// One thread per rotated pair.
extern "C" __global__ __launch_bounds__(256) void vtb_rope_rows_f32(vtb::RopeRowsArgs a) {
#pragma clang fp contract(off)
  const int hd2 = a.head_dim >> 1;
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long long)a.rows * a.heads * hd2) return;
  const int j = (int)(i % hd2);
  const long long rh = i / hd2;  // row * heads + head
  const long long row = rh / a.heads;
  float* base = a.x + rh * a.head_dim;
  const int i0 = a.half ? j : 2 * j, i1 = a.half ? j + hd2 : 2 * j + 1;
  float sn, cs;
  vtb::rope_sincos((float)(a.pos0 + row) * a.inv_freq[j], &sn, &cs);
  const float x0 = base[i0], x1 = base[i1];
  base[i0] = x0 * cs - x1 * sn;
  base[i1] = x0 * sn + x1 * cs;
}

// Elementwise kernels: thread i takes float4 i; the elements past the float4
// chunks go to the first threads.
#define VTB_ELT(NAME, EXPR)                                                                  \
  extern "C" __global__ __launch_bounds__(256) void NAME(vtb::EltArgs a) {                  \
    const int i = (int)(blockIdx.x * 256 + threadIdx.x);                                     \
    const int n4 = a.n4;                                                                     \
    if (i < n4) {                                                                            \
      float4 x = reinterpret_cast<float4*>(a.a)[i];                                          \
      const float4 y = reinterpret_cast<const float4*>(a.b)[i];                              \
      x.x = EXPR(x.x, y.x);                                                                  \
      x.y = EXPR(x.y, y.y);                                                                  \
      x.z = EXPR(x.z, y.z);                                                                  \
      x.w = EXPR(x.w, y.w);                                                                  \
      reinterpret_cast<float4*>(a.a)[i] = x;                                                 \
    }                                                                                        \
    const int t = 4 * n4 + i;                                                                \
    if (t < a.n) a.a[t] = EXPR(a.a[t], a.b[t]);                                              \
  }

#define VTB_ADD(x, y) ((x) + (y))
VTB_ELT(vtb_swiglu_f32, vtb::silu_mul)
VTB_ELT(vtb_gelu_approx_f32, vtb::gelu_approx_mul)
VTB_ELT(vtb_residual_add_f32, VTB_ADD)
