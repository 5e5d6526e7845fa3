// Quantised matrix-vector product (gfx950): out[i] = W[i, :] . x for m rows
// of GGUF block-quantised weights and f32 activations.
//
// Replaces vantablack's Metal matmul_q8_0 / matmul_q4_k / matmul_q5_k /
// matmul_q6_k (src/metal/bridge.m:39-74, 329-475, dispatched by
// segMatmulQuant, src/runtime/forward.zig:400-417) and computes what the CPU
// matmul_* of src/kernels/simd.zig:159-433 compute: dequantise each weight
// exactly as dequantBlock* does, dot with x in f32.
//
// Work decomposition: a workgroup owns R consecutive rows and has one wave
// per 2048 columns of k (up to 16 waves, k <= 32768).  Within a wave's
// 2048-column slice every lane owns 32 weights of each row, as two runs of 16
// consecutive columns (Q8_0: one block; Q4_K / Q5_K: both nibbles of 16 quant
// bytes, i.e. 16 weights of two sub-blocks; Q6_K: both nibbles of 16 ql bytes,
// two quadrants).  Lanes are ordered so that the wave's loads of one field
// are contiguous across lanes, and every lane reads 16 bytes of quants (plus
// its block's header words) per row.
//
// The activations are read once per wave, coalesced (64 lanes x 16 bytes per
// load), and handed to their owner lanes through LDS: float4 number idx of
// lane L's runs is stored at [idx][L] (rows padded so that the reads of 16
// consecutive lanes never share a bank), then each lane reads its 8 float4
// back.  Each lane issues all its loads before it waits for any: the
// activations, then the raw words of every row.  (Measured against this: a
// persistent-wave variant that stages x once per workgroup and loops over
// row groups was slower on the Llama-2-7B projection shapes in all formats
// but Q6_K with k = 11008, its per-workgroup staging sitting in front of
// every first weight load.)
//
// Arithmetic.  Per row the part's dot is formed in factored form,
//   sum_l (s q_l - mn) x_l = s sum_l q_l x_l - mn sum_l x_l,
// with s and mn the reference's f32 products (d*sc, dmin*mn) and the x sums
// over one 16-column run.  The quant sums sum_l q_l x_l use v_fma_mix_f32: a
// small unsigned quant q placed in the low bits of a 16-bit half (below
// 0x400) is exactly the f16 subnormal q * 2^-24 (q * 2^-20 four bits up),
// so masking a quant word yields two weights at once and the mixed fma takes
// them without a conversion; the power of two is removed exactly at the end.
// The wave sums its lanes (DPP / permlane) and the waves' partials are added
// in wave order through LDS, so results do not depend on timing.  The
// factoring changes only the rounding order (the GPU bar is 1e-4 relative,
// the reference's own Metal bar, bridge.zig:466-470).
//
// Weights are read through a raw buffer resource over the m rows, its range
// rounded up to whole dwords: the aligned-dword reads that cover a 2-byte
// aligned field (Q8_0 blocks are 34 bytes, Q6_K 210) never fault, and a field
// ending two bytes into the last dword still reads its own bytes.  Rows past
// m and columns past k read from the end of the range, where buffer loads
// return zero without touching memory, so every load is branch-free.
#include "common.h"

namespace vtb {


// Activation staging: 8 rows of 64 lanes + kGemvXPad float4 per wave, in
// dynamic LDS that the host sizes with the same constants.
constexpr int kGemvXPad = 4;
constexpr int kGemvXRow = 64 + kGemvXPad;

__device__ inline uint32_t wload(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}

// N consecutive weight dwords from a 4-byte aligned offset; consecutive
// 32-bit buffer loads are merged by the backend into dwordx4 / x2 loads.
// Loads and use are split so that every load of a lane is in flight before
// any result is waited for.  Cached loads: with the nontemporal policy the
// 34- and 210-byte blocks, whose neighbouring lanes share cache lines, ran
// 20-40% slower on MI355X (Q4_K unchanged).
template <int N> struct Words {
  uint32_t t[N];
  __device__ void load(__amdgpu_buffer_rsrc_t r, int off) {
#pragma unroll
    for (int i = 0; i < N; ++i) t[i] = wload(r, off + 4 * i);
  }
};

// v_perm_b32 over {hi, lo}: selector byte n < 4 picks byte n of lo, 4..7
// byte n - 4 of hi, 0x0c a zero byte.
__device__ inline uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) { return __builtin_amdgcn_perm(hi, lo, sel); }
constexpr uint32_t kPerm0 = 0x03020100u, kPerm2 = 0x05040302u;
// Bytes (0, 2) and (1, 3) of a dword as two 16-bit halves.
constexpr uint32_t kSplit02 = 0x0c020c00u, kSplit13 = 0x0c030c01u;

// Halves of v as f16, converted to f32 (exact).
__device__ inline float h_lo(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xffffu)); }
__device__ inline float h_hi(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16)); }

// acc + lo(p) * xa + hi(p) * xb, as two v_fma_mix_f32: with quant patterns
// below 0x400 in the halves this adds 2^-24 * (qa * xa + qb * xb).
__device__ inline float mix2(uint32_t p, float xa, float xb, float acc) {
  return fmaf(h_hi(p), xb, fmaf(h_lo(p), xa, acc));
}
constexpr float kTwo24 = 16777216.0f, kTwo20 = 1048576.0f;

// Byte j of v as f32 (one v_cvt_f32_ubyte<j>).
__device__ inline float ubyte_f(uint32_t v, int j) { return (float)((v >> (8 * j)) & 0xffu); }

// 2^-24 * sum over a 16-weight run whose quants are the bytes (all below
// 0x400 as 16-bit values) of u[0..4), against x[0..16).
__device__ inline float byte_run(const uint32_t (&u)[4], const float* x) {
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc = mix2(perm(0u, u[i], kSplit02), x[4 * i], x[4 * i + 2], acc);
    acc = mix2(perm(0u, u[i], kSplit13), x[4 * i + 1], x[4 * i + 3], acc);
  }
  return acc;
}

// A lane's 32 activations (run 0 then run 1) and the sum of each run.
struct XPart {
  float v[32];
  float s0, s1;
};

enum { GQ8_0 = 0, GQ4_K = 1, GQ5_K = 2, GQ6_K = 3 };

template <int KIND> struct Fmt;

// Each format defines, for a lane of a wave's 2048-column slice:
//   first(lane)      the slice column of its run 0 (run 1 starts RUN1 later),
//   owner(g), idx(g) the inverse: which lane needs slice float4 g, and as its
//                    float4 number 4 * run + i (checked against first() at
//                    compile time, staging_ok below),
//   block(lane, c0)  the row's block index holding its weights,
//   load / dot       its raw words of one row and their dot with its XPart.

// simd.zig:145-157.  Lane = one 34-byte block: f16 d, then qs[0..32).
template <> struct Fmt<GQ8_0> {
  static constexpr int BE = 32, BB = 34, RUN1 = 16;
  __host__ __device__ static constexpr int first(int lane) { return 32 * lane; }
  __host__ __device__ static constexpr int owner(int g) { return g >> 3; }
  __host__ __device__ static constexpr int idx(int g) { return g & 7; }
  __device__ static int block(int lane, int c0) { return c0 / BE + lane; }
  struct Raw {
    Words<9> w;
    uint32_t s02, s13;  // selectors: qs bytes (4i, 4i+2) / (4i+1, 4i+3) from {w[i+1], w[i]}
    int dsh;            // bit offset of d in w[0]
  };
  __device__ static void load(__amdgpu_buffer_rsrc_t r, int blk, int, Raw& raw) {
    raw.w.load(r, blk & ~3);
    // qs starts 2 bytes into w[0] when the block is 4-aligned, else 4.
    const bool sh = (blk & 2) != 0;
    raw.s02 = sh ? 0x0c060c04u : 0x0c040c02u;
    raw.s13 = sh ? 0x0c070c05u : 0x0c050c03u;
    raw.dsh = sh ? 16 : 0;
  }
  __device__ static float dot(const Raw& raw, int, const XPart& x) {
    const float d = h_lo(raw.w.t[0] >> raw.dsh);
    // Flipping each byte's sign bit gives u = q + 128 (0..255), so
    // sum q x = sum u x - 128 sum x.
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float* xv = x.v + 4 * i;
      acc = mix2(perm(raw.w.t[i + 1], raw.w.t[i], raw.s02) ^ 0x00800080u, xv[0], xv[2], acc);
      acc = mix2(perm(raw.w.t[i + 1], raw.w.t[i], raw.s13) ^ 0x00800080u, xv[1], xv[3], acc);
    }
    return d * (acc * kTwo24 - 128.0f * (x.s0 + x.s1));
  }
};

// simd.zig:211-219: the 6-bit scales and mins of sub-blocks 2j and 2j + 1 as
// bytes [sc0, sc1, mn0, mn1], from the 12 packed bytes at block bytes 4..16
// (header dwords 1..3).  With s' = 2 (j & 1) + t and bytes A = scales[s'],
// B = scales[s' + 4], C = scales[s' + 8]:
//   j < 2  (sub-block s'):     sc = A & 63, mn = B & 63
//   j >= 2 (sub-block s' + 4): sc = (C & 15) | (A >> 6) << 4,
//                              mn = (C >> 4) | (B >> 6) << 4
__device__ inline uint32_t k4_scale_min_pair(int j, const uint32_t (&h)[4]) {
  const bool odd = (j & 1) != 0;
  const uint32_t p = perm(h[2], h[1], odd ? 0x07060302u : 0x05040100u);  // [A0 A1 B0 B1]
  const uint32_t q = perm(h[3], h[3], odd ? 0x03020302u : 0x01000100u);  // [C0 C1 C0 C1]
  const uint32_t lo = p & 0x3F3F3F3Fu;
  const uint32_t hi = ((q >> 4) & 0x0F0F0000u) | (q & 0x00000F0Fu) | ((p >> 2) & 0x30303030u);
  return j < 2 ? lo : hi;
}

// simd.zig:192-243 (Q4_K), 275-317 (Q5_K).  Lane c = 0..7 of a block reads
// qs bytes [16c, 16c + 16): with j = c / 2, l0 = 16 (c % 2), their low
// nibbles are sub-block 2j, weights 64j + l0 + l, and their high nibbles
// sub-block 2j + 1, weights 64j + 32 + l0 + l (l < 16); Q5_K adds bit 2j
// (resp. 2j + 1) of qh[l0 + l] as 16.
template <bool FIVE> struct FmtK45 {
  static constexpr int BE = 256, BB = FIVE ? 176 : 144, RUN1 = 32;
  __host__ __device__ static constexpr int first(int lane) {
    return 256 * (lane >> 3) + 64 * ((lane & 7) >> 1) + 16 * (lane & 1);
  }
  // slice float4 g = 64 b + 16 j + 8 run + 4 (c % 2) + i
  __host__ __device__ static constexpr int owner(int g) {
    return ((g >> 6) << 3) | (((g >> 4) & 3) << 1) | ((g >> 2) & 1);
  }
  __host__ __device__ static constexpr int idx(int g) { return (((g >> 3) & 1) << 2) | (g & 3); }
  __device__ static int block(int lane, int c0) { return c0 / BE + (lane >> 3); }
  struct Raw {
    Words<4> h;
    Words<4> q;
    Words<FIVE ? 4 : 1> qh;
  };
  __device__ static void load(__amdgpu_buffer_rsrc_t r, int blk, int c, Raw& raw) {
    raw.h.load(r, blk);
    raw.q.load(r, blk + (FIVE ? 48 : 16) + 16 * c);
    if constexpr (FIVE) raw.qh.load(r, blk + 16 + 16 * (c & 1));
  }
  __device__ static float dot(const Raw& raw, int c, const XPart& x) {
    const int j = c >> 1;
    float a0, a1;  // run sums, as 2^-24 (Q4_K run 1: 2^-20) * sum q x
    if constexpr (FIVE) {
      uint32_t lo[4], hi[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        lo[i] = (raw.q.t[i] & 0x0F0F0F0Fu) | (((raw.qh.t[i] >> (2 * j)) & 0x01010101u) << 4);
        hi[i] = ((raw.q.t[i] >> 4) & 0x0F0F0F0Fu) | (((raw.qh.t[i] >> (2 * j + 1)) & 0x01010101u) << 4);
      }
      a0 = byte_run(lo, x.v) * kTwo24;
      a1 = byte_run(hi, x.v + 16) * kTwo24;
    } else {
      // q & 0x000F000F: low nibbles of bytes 0 and 2 (weights 4i, 4i + 2 of
      // run 0); & 0x00F000F0: their high nibbles (run 1), four bits up; the
      // same of q >> 8 for bytes 1 and 3.
      float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t w = raw.q.t[i], w8 = w >> 8;
        const float* x0 = x.v + 4 * i;
        const float* x1 = x.v + 16 + 4 * i;
        s0 = mix2(w & 0x000F000Fu, x0[0], x0[2], s0);
        s0 = mix2(w8 & 0x000F000Fu, x0[1], x0[3], s0);
        s1 = mix2(w & 0x00F000F0u, x1[0], x1[2], s1);
        s1 = mix2(w8 & 0x00F000F0u, x1[1], x1[3], s1);
      }
      a0 = s0 * kTwo24;
      a1 = s1 * kTwo20;
    }
    const uint32_t v = k4_scale_min_pair(j, raw.h.t);
    const float d = h_lo(raw.h.t[0]), dmin = h_hi(raw.h.t[0]);
    return (d * ubyte_f(v, 0)) * a0 - (dmin * ubyte_f(v, 2)) * x.s0 + (d * ubyte_f(v, 1)) * a1 -
           (dmin * ubyte_f(v, 3)) * x.s1;
  }
};
template <> struct Fmt<GQ4_K> : FmtK45<false> {};
template <> struct Fmt<GQ5_K> : FmtK45<true> {};

// simd.zig:349-404.  Lane c = 4h + 2a + lh of a block reads ql bytes
// 64h + 32a + 16lh + [0, 16) and qh bytes 32h + 16lh + [0, 16): for
// l = 16lh + [0, 16) the low nibbles are quadrant a (weights 128h + 32a + l,
// qh bits 2a..2a+1), the high nibbles quadrant a + 2 (weights
// 128h + 32(a+2) + l, qh bits 2a+4..2a+5); value - 32, scaled by
// d * sc[8h + lh + 2 * quadrant].
template <> struct Fmt<GQ6_K> {
  static constexpr int BE = 256, BB = 210, RUN1 = 64;
  __host__ __device__ static constexpr int first(int lane) {
    return 256 * (lane >> 3) + 128 * ((lane >> 2) & 1) + 32 * ((lane >> 1) & 1) + 16 * (lane & 1);
  }
  // slice float4 g = 64 b + 32 h + 16 run + 8 a + 4 lh + i
  __host__ __device__ static constexpr int owner(int g) {
    return ((g >> 6) << 3) | (((g >> 5) & 1) << 2) | (((g >> 3) & 1) << 1) | ((g >> 2) & 1);
  }
  __host__ __device__ static constexpr int idx(int g) { return (((g >> 4) & 1) << 2) | (g & 3); }
  __device__ static int block(int lane, int c0) { return c0 / BE + (lane >> 3); }
  // The block is 2-byte aligned, and so is every field in it: each is read
  // as aligned dwords from 2 bytes before it when the block is not 4-aligned,
  // and realigned with v_perm.
  struct Raw {
    Words<5> ql, qh;
    Words<3> sc;
    Words<1> d;
    uint32_t sel;
    int dsh;
  };
  __device__ static void load(__amdgpu_buffer_rsrc_t r, int blk, int c, Raw& raw) {
    const int h = c >> 2, a = (c >> 1) & 1, lh = c & 1;
    const int b4 = blk & ~3;
    raw.ql.load(r, b4 + 64 * h + 32 * a + 16 * lh);
    raw.qh.load(r, b4 + 128 + 32 * h + 16 * lh);
    raw.sc.load(r, b4 + 192 + 8 * h);
    raw.d.load(r, b4 + 208);
    const bool sh = (blk & 2) != 0;
    raw.sel = sh ? kPerm2 : kPerm0;
    raw.dsh = sh ? 16 : 0;
  }
  __device__ static float dot(const Raw& raw, int c, const XPart& x) {
    const int a = (c >> 1) & 1, lh = c & 1;
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t w = perm(raw.ql.t[i + 1], raw.ql.t[i], raw.sel);
      const uint32_t q = perm(raw.qh.t[i + 1], raw.qh.t[i], raw.sel);
      lo[i] = (w & 0x0F0F0F0Fu) | (((q >> (2 * a)) & 0x03030303u) << 4);
      hi[i] = ((w >> 4) & 0x0F0F0F0Fu) | (((q >> (2 * a + 4)) & 0x03030303u) << 4);
    }
    const float a0 = byte_run(lo, x.v) * kTwo24, a1 = byte_run(hi, x.v + 16) * kTwo24;
    const float d = h_lo(raw.d.t[0] >> raw.dsh);
    // sc[8h + t] and sc[8h + t + 4], t = lh + 2a: byte t of the two realigned
    // scale dwords.
    const int t = lh + 2 * a;
    const uint32_t s_lo = perm(raw.sc.t[1], raw.sc.t[0], raw.sel) >> (8 * t);
    const uint32_t s_hi = perm(raw.sc.t[2], raw.sc.t[1], raw.sel) >> (8 * t);
    const float sc0 = (float)(int8_t)(s_lo & 0xffu), sc1 = (float)(int8_t)(s_hi & 0xffu);
    // sum (u - 32) x = sum u x - 32 sum x over each 16-weight scale group
    return (d * sc0) * (a0 - 32.0f * x.s0) + (d * sc1) * (a1 - 32.0f * x.s1);
  }
};

// first(), owner() and idx() agree for every lane and float4 of its runs.
template <class F> constexpr bool staging_ok() {
  for (int lane = 0; lane < 64; ++lane)
    for (int run = 0; run < 2; ++run)
      for (int i = 0; i < 4; ++i) {
        const int g = (F::first(lane) + run * F::RUN1) / 4 + i;
        if (g < 0 || g >= 512 || F::owner(g) != lane || F::idx(g) != 4 * run + i) return false;
      }
  return true;
}
static_assert(staging_ok<Fmt<GQ8_0>>(), "Q8_0 staging map");
static_assert(staging_ok<Fmt<GQ4_K>>(), "Q4_K / Q5_K staging map");
static_assert(staging_ok<Fmt<GQ6_K>>(), "Q6_K staging map");

constexpr int kGemvMaxWaves = 16;  // k <= 16 * 2048 (8 * 2048 for R = 4)

template <int KIND, int R>
__device__ __forceinline__ void gemv_body(const GemvArgs& a) {
  using F = Fmt<KIND>;
  __shared__ float s_part[kGemvMaxWaves][R];
  extern __shared__ float4 s_x[];  // [waves][8][kGemvXRow]
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nw = (int)(blockDim.x >> 6);
  // This workgroup's row block (wave-uniform selects).
  int wg = (int)blockIdx.x;
  const uint8_t* wp = a.w;
  float* outp = a.out;
  unsigned wbytes = a.w_bytes;
  int m = a.m;
  if (a.nblk > 2 && wg >= a.wg2) {
    wp = a.w2, outp = a.out2, wbytes = a.w_bytes2, m = a.m2, wg -= a.wg2;
  } else if (a.nblk > 1 && wg >= a.wg1) {
    wp = a.w1, outp = a.out1, wbytes = a.w_bytes1, m = a.m1, wg -= a.wg1;
  }
  constexpr int RH = R > 1 ? R / 2 : 1;
  const bool gated = R > 1 && a.gated != 0;
  const int row0 = gated ? wg * RH : wg * R;
  const int c0 = wave * 2048;  // the wave's slice
  const int c = lane & 7;      // lane within its block (K-quants)
  const auto rsrc = buffer_rsrc(wp, wbytes);
  const auto rsrc_up = buffer_rsrc(a.w1, a.w_bytes1);
  const auto xrsrc = buffer_rsrc(a.x, 4u * (unsigned)a.k);
  const bool active = c0 + F::first(lane) < a.k;

  // All loads first, branch-free so that none waits on another: the slice's
  // activations (coalesced), then every row's raw words.  Columns past k and
  // rows past m read from the end of the buffer ranges, where buffer loads
  // return zero without touching memory, so their dots are zero.
  float4 xg[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int off = 4 * (c0 + 4 * (64 * t + lane));
    xg[t].x = __builtin_bit_cast(float, wload(xrsrc, off));
    xg[t].y = __builtin_bit_cast(float, wload(xrsrc, off + 4));
    xg[t].z = __builtin_bit_cast(float, wload(xrsrc, off + 8));
    xg[t].w = __builtin_bit_cast(float, wload(xrsrc, off + 12));
  }
  typename F::Raw raw[R];
  const int boff = F::block(lane, c0) * F::BB;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    // Gated: rows 0 .. RH-1 of the workgroup are gate rows, RH .. R-1 the
    // same rows of up.
    const bool up = gated && i >= RH;
    const int row = row0 + (gated ? i % RH : i);
    F::load(up ? rsrc_up : rsrc, active && row < m ? row * a.row_bytes + boff : (int)(up ? a.w_bytes1 : wbytes), c,
            raw[i]);
  }

  // Hand each float4 to its owner lane through this wave's LDS rows.  LDS
  // operations of one wave execute in order, so the reads below see every
  // lane's writes; the fences only keep the compiler from reordering them.
  float4* sx = s_x + wave * (8 * kGemvXRow);
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int g = 64 * t + lane;
    sx[F::idx(g) * kGemvXRow + F::owner(g)] = xg[t];
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  XPart x;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const float4 v = sx[q * kGemvXRow + lane];
    x.v[4 * q] = v.x;
    x.v[4 * q + 1] = v.y;
    x.v[4 * q + 2] = v.z;
    x.v[4 * q + 3] = v.w;
  }

  x.s0 = 0.0f;
  x.s1 = 0.0f;
#pragma unroll
  for (int l = 0; l < 16; ++l) {
    x.s0 += x.v[l];
    x.s1 += x.v[16 + l];
  }
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const float t = group_sum<64>(F::dot(raw[i], c, x));
    if (lane == 0) s_part[wave][i] = t;
  }
  __syncthreads();
  if (gated) {
    if ((int)threadIdx.x < RH && row0 + (int)threadIdx.x < m) {
      float g = 0.0f, u = 0.0f;
      for (int w = 0; w < nw; ++w) {
        g += s_part[w][threadIdx.x];
        u += s_part[w][threadIdx.x + RH];
      }
      outp[row0 + threadIdx.x] = a.gated == 1 ? silu_mul(g, u) : gelu_approx_mul(g, u);
    }
  } else if ((int)threadIdx.x < R && row0 + (int)threadIdx.x < m) {
    float t = 0.0f;
    for (int w = 0; w < nw; ++w) t += s_part[w][threadIdx.x];
    outp[row0 + threadIdx.x] = t;
  }
}

}  // namespace vtb

// Entry points: vtb_gemv_<q8_0|q4_k|q5_k|q6_k>_r<R> (R rows per workgroup;
// 64 * ceil(k / 2048) threads: up to 1024, k <= 32768, for R = 1, 2; up to
// 512, k <= 16384, for R = 4, whose registers do not fit 4 waves per SIMD).
// Dynamic LDS: waves * 8 * kGemvXRow float4.
#define VTB_GEMV(NAME, KIND, R)                                                          \
  extern "C" __global__ __launch_bounds__(R == 4 ? 512 : 1024) void vtb_gemv_##NAME##_r##R(vtb::GemvArgs a) { \
    vtb::gemv_body<vtb::KIND, R>(a);                                                   \
  }
#define VTB_GEMV_R(NAME, KIND) \
  VTB_GEMV(NAME, KIND, 1)      \
  VTB_GEMV(NAME, KIND, 2)      \
  VTB_GEMV(NAME, KIND, 4)

VTB_GEMV_R(q8_0, GQ8_0)
VTB_GEMV_R(q4_k, GQ4_K)
VTB_GEMV_R(q5_k, GQ5_K)
VTB_GEMV_R(q6_k, GQ6_K)
