// Batched quantised matmul on CDNA4 MFMA (gfx950): out[b, i] = W[i, :] . x[b, :]
// for B tokens, m rows of GGUF block-quantised weights and f32 activations.
//
// Replaces the prefill projections of vantablack's CPU prefill,
// matmulBatched (src/runtime/prefill.zig:325-378, called at :170-226):
// every weight row dequantised as dequantToF32 does
// (src/runtime/forward.zig:654-730) and dotted with each token in f32.
//
// Precision.  Every quant is a small integer, exact in f16.  Each token's
// activations are scaled by a power of two 2^e that puts the token's largest
// |x| in [2^14, 2^15), then cut into two f16 pieces rounded to nearest
// (pre-pass vtb_xsplit): h1 = f16(x 2^e), h2 = f16(x 2^e - h1).  h1 + h2
// holds x 2^e to 22 significant bits (to an absolute 2^-25 where the
// remainder falls below f16's normal range, i.e. 2^-40 of the token's
// largest |x|), so the GPU sum differs from the reference's f32 one by
// ~2^-22 of sum |W||x| at most, far inside the parity bar.  Products of
// f16 operands are exact and v_mfma_f32_32x32x16_f16 accumulates them in
// f32; the token's 2^-e comes back out exactly in the epilogue.  (Three
// truncated bf16 pieces would be exact, at 3/2 the MFMA work and operand
// traffic: measured 4-16% slower over the Llama-3-8B shapes.)  Quants enter
// as the f16 of the integer the reference scales: q (Q4_K, Q5_K, signed
// Q8_0) and q - 32 (Q6_K), converted once per workgroup as they are staged.
//
// Per scale unit (Q4_K/Q5_K sub-block and Q8_0 block of 32 columns, Q6_K
// group of 16) the MFMAs give T = sum q x over the unit, and
//   sum_unit W x = s * T - corr * sum_unit x,
// with s the reference's scale product (d*sc; d for Q8_0) and corr the
// K-quants' dmin*mn (zero for Q6_K and Q8_0).  These FMAs, one or two per
// output and unit, run on the VALU beside the MFMAs.
//
// Tiling.  A workgroup computes 128 tokens x 128 rows; four waves each own
// 64 tokens x 64 rows as 2 x 2 MFMA tiles (D = x . W^T: lane column = one
// weight row, 16 tokens per lane, so a lane needs one scale per tile).  The
// K loop steps 32 columns: the next step's activation pieces, x sums and raw
// weight words are loaded into registers while the current step's MFMAs run
// from LDS; weights are converted to f16 as they are stored.  LDS rows are
// padded to 40 halves (80 bytes) so that 16 lanes' 16-byte fragment reads
// never share a bank.  Workgroup ids are remapped so that each XCD works
// through contiguous (token block, row block) ranges, token block major:
// the activation pieces of a token block stay in that XCD's L2.
#include "common.h"

namespace vtb {


__device__ inline float wave_max(float v) {
  v = fmaxf(v, dpp<DPP_XOR1>(v));
  v = fmaxf(v, dpp<DPP_XOR2>(v));
  v = fmaxf(v, dpp<DPP_HALF_MIRROR>(v));
  v = fmaxf(v, dpp<DPP_MIRROR>(v));
  v = xor_max<16>(v);
  return xor_max<32>(v);
}

// One workgroup (256 threads) per token: the row's largest |x| fixes the
// token's power of two, then each thread splits 16-column groups.
extern "C" __global__ __launch_bounds__(256) void vtb_xsplit(XSplitArgs a) {
  __shared__ float s_max[4];
  const int t = (int)blockIdx.x, tid = (int)threadIdx.x;
  const int gpr = a.k >> 4;
  const bool live = t < a.B;
  const float* row = a.x + (size_t)t * a.k;
  float mx = 0.0f;
  if (live)
    for (int c = 4 * tid; c < a.k; c += 1024) {
      const float4 v = *reinterpret_cast<const float4*>(row + c);
      mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
  mx = wave_max(mx);
  if ((tid & 63) == 0) s_max[tid >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
  // 2^e with mx 2^e in [2^14, 2^15); e clamped so that 2^e and 2^-e stay
  // normal f32 (a row that small is then scaled less, not wrongly).
  int e = mx > 0.0f ? 14 - ilogbf(mx) : 0;
  e = e > 100 ? 100 : (e < -100 ? -100 : e);
  const float scale = ldexpf(1.0f, e);
  if (tid == 0) a.inv_scale[t] = ldexpf(1.0f, -e);
  const size_t plane = (size_t)a.Bp * a.k;
  for (int g = tid; g < gpr; g += 256) {
    const int c = 16 * g;
    float v[16];
    if (live) {
      const float4* p = reinterpret_cast<const float4*>(row + c);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 q = p[i];
        v[4 * i] = q.x;
        v[4 * i + 1] = q.y;
        v[4 * i + 2] = q.z;
        v[4 * i + 3] = q.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) v[i] = 0.0f;
    }
    uint32_t w1[8], w2[8];
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float xs = v[j] * scale;  // exact (power of two)
      sum += xs;
      const _Float16 h1 = (_Float16)xs;                 // round to nearest even
      const _Float16 h2 = (_Float16)(xs - (float)h1);  // the difference is exact in f32
      const uint32_t b1 = __builtin_bit_cast(uint16_t, h1), b2 = __builtin_bit_cast(uint16_t, h2);
      if (j & 1) {
        w1[j >> 1] |= b1 << 16;
        w2[j >> 1] |= b2 << 16;
      } else {
        w1[j >> 1] = b1;
        w2[j >> 1] = b2;
      }
    }
    uint4* d1 = reinterpret_cast<uint4*>(a.planes + (size_t)t * a.k + c);
    uint4* d2 = reinterpret_cast<uint4*>(a.planes + plane + (size_t)t * a.k + c);
    d1[0] = make_uint4(w1[0], w1[1], w1[2], w1[3]);
    d1[1] = make_uint4(w1[4], w1[5], w1[6], w1[7]);
    d2[0] = make_uint4(w2[0], w2[1], w2[2], w2[3]);
    d2[1] = make_uint4(w2[4], w2[5], w2[6], w2[7]);
    a.sums[(size_t)t * gpr + g] = sum;
  }
}


constexpr int kQgTile = 128;  // tokens and rows per workgroup
constexpr int kQgLd = 40;     // LDS row stride in 16-bit elements (80 bytes)

__device__ inline uint32_t qload(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ inline uint32_t qperm(uint32_t hi, uint32_t lo, uint32_t sel) { return __builtin_amdgcn_perm(hi, lo, sel); }
__device__ inline float qh_lo(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xffffu)); }
__device__ inline float qh_hi(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16)); }

// Two f32 holding small integers as one f16 pair (exact).
__device__ inline uint32_t f16_pair(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
}

// Eight f16 pairs (16 weights) of the byte fields of u[0..4), minus `bias`:
// small integers, so every value is exact in f16.
__device__ inline void byte_pairs(const uint32_t (&u)[4], float bias, uint32_t (&o)[8]) {
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    float f[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) f[e] = (float)((u[d] >> (8 * e)) & 0xffu) - bias;
    o[2 * d] = f16_pair(f[0], f[1]);
    o[2 * d + 1] = f16_pair(f[2], f[3]);
  }
}

// Per-thread staging of the weights of one K step (32 columns): thread
// (row, half) owns columns [16 half, 16 half + 16) of the step in one row.
// load() issues the raw loads (rows past m read zeros from the end of the
// range); store() converts to 16 f16 and the row's scale pair(s).
enum { QG8_0 = 0, QG4_K = 1, QG5_K = 2, QG6_K = 3 };
template <int KIND> struct QgFmt;

// simd.zig:145-157.  One 34-byte block per step; half = qs [16 half, +16).
template <> struct QgFmt<QG8_0> {
  static constexpr int BE = 32, BB = 34;
  static constexpr bool GROUPS16 = false, CORR = false;
  struct Raw {
    uint32_t t[5];  // aligned dwords covering qs[16 half .. +16)
    uint32_t dw;    // dword holding d
    int sh;         // block offset mod 4 (0 or 2)
  };
  __device__ static void load(__amdgpu_buffer_rsrc_t r, int row_off, int k0, int half, Raw& raw) {
    const int blk = row_off + (k0 / BE) * BB;
    const int q0 = blk + 2 + 16 * half;
    const int a0 = q0 & ~3;
#pragma unroll
    for (int i = 0; i < 5; ++i) raw.t[i] = qload(r, a0 + 4 * i);
    raw.dw = qload(r, blk & ~3);
    raw.sh = blk & 2;
  }
  // Signed quants as f16(q).
  __device__ static void store(const Raw& raw, int half, uint32_t (&o)[8], float& s, float& corr, int&) {
    const uint32_t sel = raw.sh ? kPerm0 : kPerm2;  // qs starts 2 bytes into t[0] when the block is 4-aligned
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t u = qperm(raw.t[d + 1], raw.t[d], sel);
      float f[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) f[e] = (float)(int)(int8_t)((u >> (8 * e)) & 0xffu);
      o[2 * d] = f16_pair(f[0], f[1]);
      o[2 * d + 1] = f16_pair(f[2], f[3]);
    }
    s = qh_lo(raw.dw >> (raw.sh ? 16 : 0));
    corr = 0.0f;
    (void)half;
  }
  static constexpr uint32_t kPerm0 = 0x03020100u, kPerm2 = 0x05040302u;
};

// simd.zig:211-219: the 6-bit scale and min of sub-block s (0..7) from the
// header dwords h[1..3] (packed bytes 4..16 of the block).
__device__ inline void qg_scale_min(int s, const uint32_t (&h)[4], uint32_t& sc, uint32_t& mn) {
  auto b = [&](int i) { return (h[1 + (i >> 2)] >> (8 * (i & 3))) & 0xffu; };
  if (s < 4) {
    sc = b(s) & 0x3Fu;
    mn = b(s + 4) & 0x3Fu;
  } else {
    sc = (b(s + 4) & 0x0Fu) | ((b(s - 4) >> 6) << 4);
    mn = (b(s + 4) >> 4) | ((b(s) >> 6) << 4);
  }
}

// simd.zig:192-243 (Q4_K), 275-317 (Q5_K).  Step = sub-block s of a block;
// half's 16 weights are nibble (s & 1) of qs[32 (s / 2) + 16 half + l], plus
// bit s of qh[16 half + l] as 16 for Q5_K (l < 16).
template <bool FIVE> struct QgFmtK45 {
  static constexpr int BE = 256, BB = FIVE ? 176 : 144;
  static constexpr bool GROUPS16 = false, CORR = true;
  struct Raw {
    uint32_t h[4];
    uint32_t q[4];
    uint32_t qh[FIVE ? 4 : 1];
  };
  __device__ static void load(__amdgpu_buffer_rsrc_t r, int row_off, int k0, int half, Raw& raw) {
    const int blk = row_off + (k0 / BE) * BB;
    const int s = (k0 % BE) / 32;
#pragma unroll
    for (int i = 0; i < 4; ++i) raw.h[i] = qload(r, blk + 4 * i);
    const int qs = blk + (FIVE ? 48 : 16) + 32 * (s >> 1) + 16 * half;
#pragma unroll
    for (int i = 0; i < 4; ++i) raw.q[i] = qload(r, qs + 4 * i);
    if constexpr (FIVE) {
#pragma unroll
      for (int i = 0; i < 4; ++i) raw.qh[i] = qload(r, blk + 16 + 16 * half + 4 * i);
    }
  }
  __device__ static void store(const Raw& raw, int k0, uint32_t (&o)[8], float& s_out, float& corr, int&) {
    const int s = (k0 % BE) / 32;
    uint32_t u[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      u[d] = (raw.q[d] >> (4 * (s & 1))) & 0x0F0F0F0Fu;
      if constexpr (FIVE) u[d] |= ((raw.qh[d] >> s) & 0x01010101u) << 4;
    }
    byte_pairs(u, 0.0f, o);
    uint32_t sc, mn;
    qg_scale_min(s, raw.h, sc, mn);
    s_out = qh_lo(raw.h[0]) * (float)sc;  // d * sc
    corr = qh_hi(raw.h[0]) * (float)mn;   // dmin * mn
  }
};
template <> struct QgFmt<QG4_K> : QgFmtK45<false> {};
template <> struct QgFmt<QG5_K> : QgFmtK45<true> {};

// simd.zig:349-404.  Step t (0..7) of a block = quadrant qd = t % 4 of half
// hb = t / 4: for l < 32, weight 128 hb + 32 qd + l is nibble (qd / 2) of
// ql[64 hb + 32 (qd % 2) + l] | bits 2qd..2qd+1 of qh[32 hb + l] << 4,
// minus 32, scaled by d * sc[8 hb + l / 16 + 2 qd].  Thread half takes
// l = 16 half + [0, 16): one scale group.  Blocks are 210 bytes (2-byte
// aligned): fields are read as aligned dwords and realigned.
template <> struct QgFmt<QG6_K> {
  static constexpr int BE = 256, BB = 210;
  static constexpr bool GROUPS16 = true, CORR = false;
  struct Raw {
    uint32_t ql[5], qh[5];
    uint32_t scw, dw;
    int sh;
  };
  __device__ static void load(__amdgpu_buffer_rsrc_t r, int row_off, int k0, int half, Raw& raw) {
    const int blk = row_off + (k0 / BE) * BB;
    const int t = (k0 % BE) / 32, hb = t >> 2, qd = t & 3;
    const int b4 = blk & ~3;
    const int ql = b4 + 64 * hb + 32 * (qd & 1) + 16 * half;
    const int qh = b4 + 128 + 32 * hb + 16 * half;
#pragma unroll
    for (int i = 0; i < 5; ++i) {
      raw.ql[i] = qload(r, ql + 4 * i);
      raw.qh[i] = qload(r, qh + 4 * i);
    }
    raw.scw = qload(r, (blk + 192 + 8 * hb + half + 2 * qd) & ~3);
    raw.dw = qload(r, (blk + 208) & ~3);
    raw.sh = blk & 2;
  }
  __device__ static void store(const Raw& raw, int k0, uint32_t (&o)[8], float& s, float& corr, int& half_io) {
    const int t = (k0 % BE) / 32, hb = t >> 2, qd = t & 3, half = half_io;
    const uint32_t sel = raw.sh ? 0x05040302u : 0x03020100u;
    uint32_t u[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t wl = qperm(raw.ql[d + 1], raw.ql[d], sel);
      const uint32_t wh = qperm(raw.qh[d + 1], raw.qh[d], sel);
      u[d] = ((wl >> (4 * (qd >> 1))) & 0x0F0F0F0Fu) | (((wh >> (2 * qd)) & 0x03030303u) << 4);
    }
    byte_pairs(u, 32.0f, o);  // q - 32, as dequantBlockQ6_K forms it
    const int blk_lo = raw.sh;  // block offset mod 4
    const int sc_byte = (blk_lo + 192 + 8 * hb + half + 2 * qd) & 3;
    const float sc = (float)(int8_t)((raw.scw >> (8 * sc_byte)) & 0xffu);
    const float d = qh_lo(raw.dw >> (raw.sh ? 16 : 0));
    s = d * sc;
    corr = 0.0f;
  }
};

template <int KIND>
__device__ __forceinline__ void qgemm_body(const QGemmArgs& a) {
  using F = QgFmt<KIND>;
  __shared__ __attribute__((aligned(16))) uint16_t s_x[2][kQgTile][kQgLd];
  __shared__ float s_inv[kQgTile];
  __shared__ __attribute__((aligned(16))) uint16_t s_w[kQgTile][kQgLd];
  __shared__ float s_scale[2][2][kQgTile];  // [group][s, corr][row]
  __shared__ __attribute__((aligned(16))) float s_sum[3][kQgTile];  // [group 0, group 1, both][token]

  const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // XCD-aware block order: consecutive ids go to different XCDs, so give
  // each XCD a contiguous range of the (token block, row block) list.
  const int total = a.n_rb * a.n_tb;
  const int per = total >> 3;
  int wi = (int)blockIdx.x;
  if (wi < 8 * per) wi = (wi & 7) * per + (wi >> 3);
  const int tb = wi / a.n_rb, rb = wi % a.n_rb;
  const int tok0 = tb * kQgTile, row0 = rb * kQgTile;

  const auto rsrc = buffer_rsrc(a.w, a.w_bytes);
  // Staging roles.
  const int srow = tid >> 1, shalf = tid & 1;
  const int row_off = row0 + srow < a.m ? (row0 + srow) * a.row_bytes : (int)a.w_bytes;
  const size_t plane = (size_t)a.Bp * a.k;
  const int gpr = a.k >> 4;

  typename F::Raw raw;
  u32x4 xr[4];
  float2 sr = make_float2(0.0f, 0.0f);
  auto load_step = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = tid + 256 * j;
      const int piece = c >> 9, token = (c & 511) >> 2, part = c & 3;
      xr[j] = *reinterpret_cast<const u32x4*>(a.planes + piece * plane + (size_t)(tok0 + token) * a.k + k0 + 8 * part);
    }
    if (tid < kQgTile) sr = *reinterpret_cast<const float2*>(a.sums + (size_t)(tok0 + tid) * gpr + (k0 >> 4));
    F::load(rsrc, row_off, k0, shalf, raw);
  };
  auto store_step = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = tid + 256 * j;
      const int piece = c >> 9, token = (c & 511) >> 2, part = c & 3;
      *reinterpret_cast<u32x4*>(&s_x[piece][token][8 * part]) = xr[j];
    }
    if (tid < kQgTile) {
      s_sum[0][tid] = sr.x;
      s_sum[1][tid] = sr.y;
      s_sum[2][tid] = sr.x + sr.y;
    }
    uint32_t o[8];
    float s, corr;
    int hh = shalf;
    if constexpr (KIND == QG8_0)
      F::store(raw, shalf, o, s, corr, hh);
    else
      F::store(raw, k0, o, s, corr, hh);
    *reinterpret_cast<u32x4*>(&s_w[srow][16 * shalf]) = u32x4{o[0], o[1], o[2], o[3]};
    *reinterpret_cast<u32x4*>(&s_w[srow][16 * shalf + 8]) = u32x4{o[4], o[5], o[6], o[7]};
    if (F::GROUPS16 || shalf == 0) {
      s_scale[F::GROUPS16 ? shalf : 0][0][srow] = s;
      s_scale[F::GROUPS16 ? shalf : 0][1][srow] = corr;
    }
  };

  // Wave tiles: tokens [64 tw, +64) x rows [64 rw, +64) of the block.
  const int tw = wave & 1, rw = wave >> 1;
  const int fl = lane & 31, fk = 8 * (lane >> 5);  // fragment row / column within the 16-wide K half
  f32x16 acc[2][2];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[tt][rt][i] = 0.0f;

  // T over the K halves in `khs`, then acc += s * T - corr * sum x.
  auto unit = [&](int kh_lo, int kh_hi, int grp) __attribute__((always_inline)) {
    f32x16 T[2][2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int i = 0; i < 16; ++i) T[tt][rt][i] = 0.0f;
    for (int kh = kh_lo; kh < kh_hi; ++kh) {
      f16x8 b[2];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
        b[rt] = *reinterpret_cast<const f16x8*>(&s_w[64 * rw + 32 * rt + fl][16 * kh + fk]);
#pragma unroll
      for (int p = 0; p < 2; ++p) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const f16x8 av = *reinterpret_cast<const f16x8*>(&s_x[p][64 * tw + 32 * tt + fl][16 * kh + fk]);
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) T[tt][rt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, b[rt], T[tt][rt], 0, 0, 0);
        }
      }
    }
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int row = 64 * rw + 32 * rt + fl;
      const float s = s_scale[grp][0][row], corr = s_scale[grp][1][row];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          // tokens 8q + 4 (lane / 32) + [0, 4) of the tile
          const int tok = 64 * tw + 32 * tt + 8 * q + 4 * (lane >> 5);
          float4 sx = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
          if constexpr (F::CORR) sx = *reinterpret_cast<const float4*>(&s_sum[F::GROUPS16 ? grp : 2][tok]);
          const float sxv[4] = {sx.x, sx.y, sx.z, sx.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float v = fmaf(s, T[tt][rt][4 * q + e], acc[tt][rt][4 * q + e]);
            if constexpr (F::CORR) v = fmaf(-corr, sxv[e], v);
            acc[tt][rt][4 * q + e] = v;
          }
        }
      }
    }
  };

  const int nks = a.k / 32;
  if (tid < kQgTile) s_inv[tid] = a.inv_scale[tok0 + tid];
  load_step(0);
  for (int ks = 0; ks < nks; ++ks) {
    __syncthreads();
    store_step(32 * ks);
    __syncthreads();
    // (the last step reloads step 0, unused: an unconditional load keeps
    // the staging registers out of scratch)
    load_step(32 * (ks + 1 < nks ? ks + 1 : 0));
    if constexpr (F::GROUPS16) {
      unit(0, 1, 0);
      unit(1, 2, 1);
    } else {
      unit(0, 2, 0);
    }
  }

  // out[token][row]: lanes 0..31 of one register hold 32 consecutive rows of
  // one token.
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int row = row0 + 64 * rw + 32 * rt + fl;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int tl = 64 * tw + 32 * tt + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
        if (row < a.m && tok0 + tl < a.B) a.out[(size_t)(tok0 + tl) * a.m + row] = acc[tt][rt][i] * s_inv[tl];
      }
    }
}

}  // namespace vtb

// Two workgroups per CU (at most 256 registers per lane): 4-16% faster than
// one, measured over the Llama-3-8B projection shapes in all four formats.
#define VTB_QGEMM(NAME, KIND)                                                                 \
  extern "C" __global__ __launch_bounds__(256, 2) void vtb_qgemm_##NAME(vtb::QGemmArgs a) { \
    vtb::qgemm_body<vtb::KIND>(a);                                                       \
  }
VTB_QGEMM(q8_0, QG8_0)
VTB_QGEMM(q4_k, QG4_K)
VTB_QGEMM(q5_k, QG5_K)
VTB_QGEMM(q6_k, QG6_K)
