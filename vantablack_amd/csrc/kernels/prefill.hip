// Causal prefill attention on CDNA4 MFMA (gfx950).
//
// Computes, for every query b of a prompt (position pos0 + b) and head h,
// exactly the attention of prefill.attentionCausal
// (src/runtime/prefill.zig:237-287):
//   out[b,h] = sum_t softmax_t(q[b,h].K[t,kv_h] / sqrt(D)) V[t,kv_h]
// over t in [window_start(pos0+b), pos0+b], kv_h = (h*n_kv)/n_heads.
//
// Flash-attention formulation, transposed so that every lane owns one query:
//   S^T = K Q^T        v_mfma_f32_32x32x16_{bf16,f16}; A = K rows from LDS,
//                      B = Q^T kept in registers for the whole key loop.
//   online softmax     the 32x32 accumulator layout puts one query per lane
//                      column (lane % 32) and 16 keys per lane, so row max /
//                      row sum need one cross-lane step (lane ^ 32).
//   O^T += V^T P^T     v_mfma_f32_32x32x16_f16; B = P^T straight from the S^T
//                      accumulators (rounded to f16), A = V^T from LDS.  The
//                      V^T tile is stored with its key columns permuted so the
//                      8 keys a lane holds in P^T are 8 contiguous f16 in LDS.
// P is rounded to f16 (not bf16: 11 vs 8 significant bits), and a bf16 V is
// converted to f16 while it is transposed into LDS (exact for |v| in f16's
// normal range; the cache dtype's values are carried over unchanged).
//
// Workgroup = 4 waves x 32 queries = BM queries of one head; key tiles of BN
// rows stream through LDS with the next tile prefetched into registers.
// Tiles entirely above a wave's diagonal or before its window are skipped.
#include "common.h"
#include "../tiles.h"

namespace vtb {

struct PrefillArgs {
  const void* q;       // [n_q][n_heads][D] of DT
  const void* k;       // layer base: row t at k + t*n_kv*D elements
  const void* v;
  float* out;          // [n_q][n_heads][D] f32
  int n_q;
  int n_heads;
  int n_kv;
  int pad0;
  long long pos0;      // absolute position of query 0
  long long window;    // sliding window in rows; <= 0 disables it
  float scale_log2;    // (1/sqrt(D)) * log2(e)
  int pad1;
};

template <typename DT> struct Mfma;
template <> struct Mfma<kv_bf16> {
  typedef bf16x8 frag;
  __device__ static inline f32x16 qk(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  // bf16 bits -> f16 value (via the exact f32 upcast).
  __device__ static inline _Float16 to_f16(uint16_t bits) {
    return (_Float16)__builtin_bit_cast(float, (uint32_t)bits << 16);
  }
};
template <> struct Mfma<kv_f16> {
  typedef f16x8 frag;
  __device__ static inline f32x16 qk(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  __device__ static inline _Float16 to_f16(uint16_t bits) { return __builtin_bit_cast(_Float16, bits); }
};

__device__ inline f32x16 mfma_pv(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Column of key x (0..15 within a 16-key step) in the V^T tile: swaps the
// middle two 4-key groups, so lane half hi reads keys {4hi..4hi+3,
// 8+4hi..8+4hi+3} -- the keys its P^T fragment holds -- as 8 contiguous f16.
__device__ inline int vt_col(int x) { return 8 * ((x >> 2) & 1) + 4 * (x >> 3) + (x & 3); }

template <typename DT, int D>
__device__ __forceinline__ void prefill_body(const PrefillArgs& a) {
  constexpr int BM = prefill_block_m(D);      // queries per workgroup (4 waves x 32)
  constexpr int BN = prefill_block_n(D);      // keys per tile
  constexpr int KP = D + 8;                   // K tile row pitch (f16/bf16 elements)
  constexpr int VP = BN + 8;                  // V^T tile row pitch
  constexpr int KCH = BN * D / 8;             // 16-byte chunks per K (or V) tile
  constexpr int KPT = (KCH + 255) / 256;      // K chunks per thread
  constexpr int VBLK = (BN / 4) * (D / 8);    // 4-row x 8-col V blocks per tile
  constexpr int NS = BN / 32;                 // 32-key S^T tiles per key tile
  constexpr int ND = D / 32;                  // 32-dim O^T tiles
  constexpr int KS = D / 16;                  // k-steps of the QK product
  static_assert(BM == 128, "4 waves x 32 queries");
  static_assert(VBLK <= 256 && KCH % 256 == 0, "tile does not match 256 threads");
  typedef typename Mfma<DT>::frag frag;

  __shared__ __attribute__((aligned(16))) uint16_t k_lds[BN * KP];
  __shared__ __attribute__((aligned(16))) _Float16 vt_lds[D * VP];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int hi = lane >> 5;   // lane half
  const int lc = lane & 31;   // lane column: the query this lane owns
  const int h = blockIdx.x;
  const int nblk = gridDim.y;
  const int qb = nblk - 1 - (int)blockIdx.y;  // longest (last) query blocks first
  const int kvh = (int)(((long long)h * a.n_kv) / a.n_heads);

  const int m0 = qb * BM;
  const int mq = m0 + wave * 32 + lc;  // this lane's query (may be >= n_q: padding)
  const long long qpos = a.pos0 + mq;
  const long long q_lo = a.pos0 + m0;  // first query position of the workgroup
  const int m_last = (m0 + BM < a.n_q ? m0 + BM : a.n_q) - 1;
  const long long q_hi = a.pos0 + m_last;
  const long long kend = q_hi + 1;  // keys [.., kend) may be attended
  long long kbeg = 0;
  if (a.window > 0 && q_lo >= a.window) kbeg = q_lo - a.window + 1;
  const long long kt_first = kbeg / BN * BN;

  // Wave-level query range, for tile skipping.
  const long long wq_lo = a.pos0 + m0 + wave * 32;
  const long long wq_hi = a.pos0 + (m0 + wave * 32 + 31 < a.n_q ? m0 + wave * 32 + 31 : a.n_q - 1);
  const bool wave_live = m0 + wave * 32 < a.n_q;

  const long long row_stride = (long long)a.n_kv * D;  // elements
  const uint16_t* kg = (const uint16_t*)a.k + (long long)kvh * D;
  const uint16_t* vg = (const uint16_t*)a.v + (long long)kvh * D;

  // Q^T fragments (B operand): lane holds Q[mq][16ks + 8hi .. +8].
  frag qf[KS];
  {
    const int mr = mq < a.n_q ? mq : a.n_q - 1;
    const uint16_t* qp = (const uint16_t*)a.q + ((long long)mr * a.n_heads + h) * D + 8 * hi;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = __builtin_bit_cast(frag, load16(qp + 16 * ks));
  }

  f32x16 o[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i) o[i] = f32x16{};
  float m_run = -INFINITY, l_run = 0.0f;

  // Register prefetch of one tile: K as 16-byte chunks, V as one 4x8 block.
  u32x4 kpre[KPT];
  u32x4 vpre[4];
  const int vblk = tid;                       // V block owned by this thread
  const int vb_r = (vblk / (D / 8)) * 4;      // first of 4 key rows
  const int vb_c = (vblk % (D / 8)) * 8;      // first of 8 dims
  auto prefetch = [&](long long kt0) {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int c = tid + 256 * i;
      const int r = c / (D / 8), cc = (c % (D / 8)) * 8;
      long long row = kt0 + r;
      row = row < kend ? row : kend - 1;
      kpre[i] = load16(kg + row * row_stride + cc);
    }
    if (vblk < VBLK) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        long long row = kt0 + vb_r + j;
        row = row < kend ? row : kend - 1;
        vpre[j] = load16(vg + row * row_stride + vb_c);
      }
    }
  };
  auto stage = [&]() {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int c = tid + 256 * i;
      const int r = c / (D / 8), cc = (c % (D / 8)) * 8;
      *reinterpret_cast<u32x4*>(&k_lds[r * KP + cc]) = kpre[i];
    }
    if (vblk < VBLK) {
      // Transpose the 4 (keys) x 8 (dims) block to 8 x 4 and store each dim's
      // 4 keys as one 8-byte write at the permuted key column.
      uint16_t e[4][8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const u32x4 w = vpre[j];
        const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int c = 0; c < 8; ++c) e[j][c] = (uint16_t)(ww[c >> 1] >> (16 * (c & 1)));
      }
      const int xcol = 16 * (vb_r / 16) + vt_col(vb_r % 16);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        f16x4 t;
#pragma unroll
        for (int j = 0; j < 4; ++j) t[j] = Mfma<DT>::to_f16(e[j][c]);
        *reinterpret_cast<f16x4*>(&vt_lds[(vb_c + c) * VP + xcol]) = t;
      }
    }
  };

  const float sl = a.scale_log2;
  long long kt0 = kt_first;
  if (kt0 < kend) prefetch(kt0);
  for (; kt0 < kend; kt0 += BN) {
    __syncthreads();  // previous tile's LDS reads are done
    stage();
    __syncthreads();
    if (kt0 + BN < kend) prefetch(kt0 + BN);

    // Skip tiles entirely above this wave's diagonal or before its windows.
    bool live = wave_live && kt0 <= wq_hi;
    if (a.window > 0 && kt0 + BN - 1 < wq_lo - a.window + 1) live = false;
    if (!live) continue;

    // S^T = K Q^T.
    f32x16 s[NS];
#pragma unroll
    for (int nt = 0; nt < NS; ++nt) {
      s[nt] = f32x16{};
      const uint16_t* kr = &k_lds[(32 * nt + lc) * KP + 8 * hi];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const frag kf = __builtin_bit_cast(frag, *reinterpret_cast<const u32x4*>(kr + 16 * ks));
        s[nt] = Mfma<DT>::qk(kf, qf[ks], s[nt]);
      }
    }

    // Scale to the log2 domain, mask, and the online softmax update.
    const bool need_mask =
        (kt0 + BN - 1 > wq_lo) || (a.window > 0 && kt0 < wq_hi - a.window + 1);
    float mt = -INFINITY;
#pragma unroll
    for (int nt = 0; nt < NS; ++nt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float v = s[nt][r] * sl;
        if (need_mask) {
          const long long kp = kt0 + 32 * nt + 8 * (r >> 2) + 4 * hi + (r & 3);
          const bool ok = kp <= qpos && (a.window <= 0 || kp > qpos - a.window);
          v = ok ? v : -INFINITY;
        }
        s[nt][r] = v;
        mt = fmaxf(mt, v);
      }
    }
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float m_new = fmaxf(m_run, mt);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;  // all masked so far
    const float corr = exp2_fast(m_run - m_use);
    m_run = m_new;

    f16x8 pf[NS * 2];
    float ls = 0.0f;
#pragma unroll
    for (int nt = 0; nt < NS; ++nt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const _Float16 p = (_Float16)exp2_fast(s[nt][r] - m_use);
        ls += (float)p;
        pf[2 * nt + (r >> 3)][r & 7] = p;
      }
    }
    l_run = l_run * corr + ls;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) o[dt] *= corr;

    // O^T += V^T P^T.
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) {
      const _Float16* vr = &vt_lds[(32 * dt + lc) * VP + 8 * hi];
#pragma unroll
      for (int ks = 0; ks < BN / 16; ++ks) {
        const f16x8 vf = *reinterpret_cast<const f16x8*>(vr + 16 * ks);
        o[dt] = mfma_pv(vf, pf[ks], o[dt]);
      }
    }
  }

  // out[mq][h][d] = O^T[d][mq] / l.  The lane holds d = 32dt + 8(r/4) +
  // 4hi + (r%4): four consecutive dims per r/4, written as one 16-byte store.
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  if (mq < a.n_q) {
    const float inv = 1.0f / l_tot;
    float* op = a.out + ((long long)mq * a.n_heads + h) * D + 4 * hi;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f32x4 w;
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = o[dt][4 * g + j] * inv;
        *reinterpret_cast<f32x4*>(op + 32 * dt + 8 * g) = w;
      }
    }
  }
}

}  // namespace vtb

#define VTB_PREFILL(DTN, DTT, D)                                                          \
  extern "C" __global__ __launch_bounds__(256) void vtb_prefill_##DTN##_d##D(vtb::PrefillArgs a) { \
    vtb::prefill_body<vtb::DTT, D>(a);                                                    \
  }

VTB_PREFILL(bf16, kv_bf16, 64)
VTB_PREFILL(bf16, kv_bf16, 128)
VTB_PREFILL(bf16, kv_bf16, 256)
VTB_PREFILL(f16, kv_f16, 64)
VTB_PREFILL(f16, kv_f16, 128)
VTB_PREFILL(f16, kv_f16, 256)
