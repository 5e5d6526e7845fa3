// Causal prefill attention on CDNA4 MFMA (gfx950).
//
// Computes, for every query b of a prompt (position pos0 + b) and head h,
// exactly the attention of prefill.attentionCausal
// (src/runtime/prefill.zig:237-287):
//   out[b,h] = sum_t softmax_t(q[b,h].K[t,kv_h] / sqrt(D)) V[t,kv_h]
// over t in [window_start(pos0+b), pos0+b], kv_h = (h*n_kv)/n_heads.
//
// Two kernels per call:
//   vtb_vt_<dt>_d<D>       V pre-pass: writes V^T as f16, [kv_h][d][key],
//                          keys permuted inside each 16-key group (vt_col),
//                          zero-padded to a whole number of key tiles.  A bf16
//                          V is converted to f16 here (exact for |v| in f16's
//                          normal range).  One pass over V: ~5 us at 8K keys.
//   vtb_prefill_<dt>_d<D>  flash attention, transposed so that every lane
//                          owns one query:
//     S^T = K Q^T          v_mfma_f32_32x32x16_{bf16,f16}; A = K rows from LDS,
//                          B = Q^T kept in registers for the whole key loop.
//     online softmax       the 32x32 accumulator puts one query per lane
//                          column (lane % 32) and 16 keys per lane, so the row
//                          max / sum need one cross-lane step (lane ^ 32).
//                          Rescaling of O is lazy: the running max is only
//                          raised when a row's max grows by more than 2^8, so
//                          P stays <= 256 (well inside f16) and most tiles skip
//                          the O multiply.
//     O^T += V^T P^T       v_mfma_f32_32x32x16_f16; B = P^T straight from the
//                          S^T accumulators (rounded to f16), A = V^T from LDS.
//                          The pre-pass permutation makes the 8 keys a lane
//                          holds in P^T 8 contiguous f16 of a V^T row.
// P is rounded to f16 (11 significant bits; bf16's 8 bits would give ~2e-3
// relative error, at the parity bar).
//
// Workgroup = 4 waves x 32 queries = 128 queries of one head; key tiles of BN
// rows stream through LDS (K row-major, V^T row-major, both padded so the
// 16-byte MFMA operand reads and the tile stores are bank-conflict free),
// with the next tile prefetched into registers.  Tiles entirely above a
// wave's diagonal or before its window are skipped.
#include "common.h"
#include "../tiles.h"

namespace vtb {



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

// Column of key x (0..15 within a 16-key group) in V^T: swaps the middle two
// 4-key groups, so lane half hi reads keys {4hi..4hi+3, 8+4hi..8+4hi+3} --
// exactly the keys its P^T fragment holds -- as 8 contiguous f16.  The map is
// its own inverse.
__device__ inline int vt_col(int x) { return 8 * ((x >> 2) & 1) + 4 * (x >> 3) + (x & 3); }

// v of lane l ^ 32 via v_permlane32_swap_b32, which swaps lanes 32..63 of
// its first register with lanes 0..31 of its second: with both holding v,
// the first ends up holding v of lane l % 32 and the second v of lane
// l % 32 + 32, in every lane.  Inline asm because the compiler's builtin for
// this instruction returns the first register for both results; the s_nop
// gives the two wait states a VALU write needs before a permlane reads it.
__device__ inline void lane_halves(float v, float& lo_half, float& hi_half) {
  float x = v, y = v;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(x), "+v"(y));
  lo_half = x;
  hi_half = y;
}

// ---------------------------------------------------------------- pre-pass
template <typename DT, int D>
__device__ __forceinline__ void vt_body(const VtArgs& a) {
  constexpr int TK = 64;            // keys per workgroup
  constexpr int TP = D + 8;         // LDS pitch (f16)
  __shared__ __attribute__((aligned(16))) _Float16 tile[TK * TP];
  const int tid = threadIdx.x;
  const int kvh = blockIdx.y;
  const long long key0 = (long long)blockIdx.x * TK;
  const long long row_stride = (long long)a.n_kv * D;
  const uint16_t* vg = (const uint16_t*)a.v + (long long)kvh * D;
  // Load 64 keys x D dims (16-byte chunks), convert to f16, stage row-major.
  for (int c = tid; c < TK * D / 8; c += 256) {
    const int key = c / (D / 8), dc = (c % (D / 8)) * 8;
    u32x4 w = {0u, 0u, 0u, 0u};
    if (key0 + key < a.n_rows) w = load16(vg + (key0 + key) * row_stride + dc);
    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
    f16x8 h;
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = Mfma<DT>::to_f16((uint16_t)(ww[e >> 1] >> (16 * (e & 1))));
    *reinterpret_cast<f16x8*>(&tile[key * TP + dc]) = h;
  }
  __syncthreads();
  // Write V^T rows: output column o of a 16-key group holds key vt_col(o).
  for (int c = tid; c < D * TK / 8; c += 256) {
    const int d = c / (TK / 8), o0 = (c % (TK / 8)) * 8;
    f16x8 h;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int o = o0 + e;
      h[e] = tile[(16 * (o >> 4) + vt_col(o & 15)) * TP + d];
    }
    *reinterpret_cast<f16x8*>((_Float16*)a.vt + ((long long)kvh * D + d) * a.vt_ld + key0 + o0) = h;
  }
}

// ---------------------------------------------------------------- attention
template <typename DT, int D, int NW>
__device__ __forceinline__ void prefill_body(const PrefillArgs& a) {
  constexpr int NT = 64 * NW;                 // threads per workgroup
  constexpr int BM = 32 * NW;                 // queries per workgroup (NW waves x 32)
  constexpr int BN = prefill_block_n(D);      // keys per tile
  constexpr int KCH = D / 8;                  // 16-byte chunks per K row
  constexpr int VCH = BN / 8;                 // 16-byte chunks per V^T row
  constexpr int KPB = (KCH + 1) * 16;         // LDS pitch of a K row: one pad chunk
  constexpr int VPB = (VCH + 1) * 16;         // LDS pitch of a V^T row
  constexpr int CPT = BN * KCH / NT;          // 16-byte chunks per thread per tile (K; V^T alike)
  static_assert(BN * KCH % NT == 0 && D * (BN / 8) == BN * KCH, "tile does not match the workgroup");
  constexpr int NS = BN / 32;                 // 32-key S^T tiles per key tile
  constexpr int ND = D / 32;                  // 32-dim O^T tiles
  constexpr int KS = D / 16;                  // k-steps of the QK product
  constexpr int PS = BN / 16;                 // k-steps of the PV product
#ifndef VTB_PF_KB
#define VTB_PF_KB 1
#endif
#ifndef VTB_PF_VB
#define VTB_PF_VB 2
#endif
  constexpr int KB = NS < VTB_PF_KB ? NS : VTB_PF_KB;  // S^T tiles per K-fragment batch
  constexpr int VB = ND < VTB_PF_VB ? ND : VTB_PF_VB;  // O^T tiles per V-fragment batch
  static_assert(NS % KB == 0 && ND % VB == 0, "batches must divide the tiles");
  typedef typename Mfma<DT>::frag frag;

  // Two K and two V^T stages: tile j is read from stage j%2 while tile j+1
  // is written into the other, so one barrier per tile suffices.
  __shared__ __attribute__((aligned(16))) char k_lds0[BN * KPB];
  __shared__ __attribute__((aligned(16))) char k_lds1[BN * KPB];
  __shared__ __attribute__((aligned(16))) char v_lds0[D * VPB];
  __shared__ __attribute__((aligned(16))) char v_lds1[D * VPB];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int hi = lane >> 5;   // lane half
  const int lc = lane & 31;   // lane column: the query this lane owns
  const int nblk = gridDim.y;
  int h, qb;
  {
    // Workgroups are dispatched round-robin over the 8 XCDs in linear order.
    // When the heads split evenly, XCD x gets heads [x*hpx, (x+1)*hpx) --
    // with GQA these share KV heads, so each XCD's L2 holds fewer K/V tiles
    // -- and every XCD takes its longest (last) query blocks first.
    const int i = blockIdx.y * gridDim.x + blockIdx.x;
    if (a.n_heads % 8 == 0) {
      const int hpx = a.n_heads / 8, j = i / 8;
      h = (i % 8) * hpx + j % hpx;
      qb = nblk - 1 - j / hpx;
    } else {
      h = blockIdx.x;
      qb = nblk - 1 - (int)blockIdx.y;
    }
  }
  const int kvh = (int)(((long long)h * a.n_kv) / a.n_heads);

  const int m0 = qb * BM;
  const int mq = m0 + wave * 32 + lc;  // this lane's query (may be >= n_q: padding)
  const long long qpos = a.pos0 + mq;
  const long long q_lo = a.pos0 + m0;  // first query position of the workgroup
  const int m_last = (m0 + BM < a.n_q ? m0 + BM : a.n_q) - 1;
  const long long kend = a.pos0 + m_last + 1;  // keys [.., kend) may be attended
  long long kbeg = 0;
  if (a.window > 0 && q_lo >= a.window) kbeg = q_lo - a.window + 1;
  const long long kt_first = kbeg / BN * BN;

  // Wave-level query range, for tile skipping.
  const long long wq_lo = a.pos0 + m0 + wave * 32;
  const long long wq_hi = a.pos0 + (m0 + wave * 32 + 31 < a.n_q ? m0 + wave * 32 + 31 : a.n_q - 1);
  const bool wave_live = m0 + wave * 32 < a.n_q;

  const long long row_stride = (long long)a.n_kv * D;  // elements
  const uint16_t* kg = (const uint16_t*)a.k + (long long)kvh * D;
  const _Float16* vtg = (const _Float16*)a.vt + (long long)kvh * D * a.vt_ld;

  // Tile staging through registers: thread chunk i of a tile is K row
  // (tid + NT i) / KCH, chunk (tid + NT i) % KCH, and V^T row (tid + NT i) /
  // VCH, chunk (tid + NT i) % VCH.  K rows at or past kend are clamped to
  // kend - 1 (those keys are masked for every query here).
  u32x4 kpre[CPT], vpre[CPT];
  auto fetch = [&](long long kt0) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + NT * i;
      long long row = kt0 + c / KCH;
      row = row < kend ? row : kend - 1;
      kpre[i] = load16_cached(kg + row * row_stride + 8 * (c % KCH));
    }
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + NT * i;
      vpre[i] = load16_cached(vtg + (long long)(c / VCH) * a.vt_ld + kt0 + 8 * (c % VCH));
    }
  };
  auto stage = [&](char* kl, char* vl) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + NT * i;
      *reinterpret_cast<u32x4*>(kl + (c / KCH) * KPB + 16 * (c % KCH)) = kpre[i];
    }
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + NT * i;
      *reinterpret_cast<u32x4*>(vl + (c / VCH) * VPB + 16 * (c % VCH)) = vpre[i];
    }
  };

  // Q^T fragments (B operand): lane holds Q[mq][16ks + 8hi .. +8].
  frag qf[KS];
  {
    const int mr = mq < a.n_q ? mq : a.n_q - 1;
    const uint16_t* qp = (const uint16_t*)a.q + ((long long)mr * a.n_heads + h) * D + 8 * hi;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = __builtin_bit_cast(frag, load16_cached(qp + 16 * ks));
  }

  f32x16 o[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i) o[i] = f32x16{};
  float m_ref = -INFINITY;  // running reference max (log2 domain, scaled)
  float l_run = 0.0f;
  const float sl = a.scale_log2;
  // The window as a 32-bit bound (positions stay below 2^30; a larger or
  // absent window keeps every causal key).
  const int wcap = (a.window > 0 && a.window < (1 << 30)) ? (int)a.window : (1 << 30);

  auto compute = [&](const char* kl, const char* vl, long long kt0) {
    // Skip tiles entirely above this wave's diagonal or before its windows.
    bool live = wave_live && kt0 <= wq_hi;
    if (a.window > 0 && kt0 + BN - 1 < wq_lo - a.window + 1) live = false;
    if (!live) return;

    // S^T = K Q^T.  K fragments (row 32nt + lc, chunk 2ks + hi) are read in
    // batches of KB S^T tiles so their LDS latency overlaps the MFMAs.
    const char* kr = kl + lc * KPB + 16 * hi;
    f32x16 s[NS];
#pragma unroll
    for (int nt = 0; nt < NS; ++nt) s[nt] = f32x16{};
#pragma unroll
    for (int n0 = 0; n0 < NS; n0 += KB) {
      u32x4 kf[KS][KB];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int nb = 0; nb < KB; ++nb)
          kf[ks][nb] = *reinterpret_cast<const u32x4*>(kr + 32 * (n0 + nb) * KPB + 32 * ks);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int nb = 0; nb < KB; ++nb)
          s[n0 + nb] = Mfma<DT>::qk(__builtin_bit_cast(frag, kf[ks][nb]), qf[ks], s[n0 + nb]);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(0);
    }

    // First V^T batch (dims 0 .. 32VB) for the PV product, in flight during
    // the softmax.
    const char* vr = vl + lc * VPB + 16 * hi;
    u32x4 vf[PS][VB];
#pragma unroll
    for (int ks = 0; ks < PS; ++ks)
#pragma unroll
      for (int db = 0; db < VB; ++db) vf[ks][db] = *reinterpret_cast<const u32x4*>(vr + 32 * db * VPB + 32 * ks);

    // Mask (diagonal / window tiles only: a wave-uniform branch).  Key
    // 32nt + 8(r/4) + 4hi + r%4 of the tile is kept iff it lies in
    // (qpos - window, qpos]; lim is qpos relative to this lane's first key.
    const bool need_mask = (kt0 + BN - 1 > wq_lo) || (a.window > 0 && kt0 < wq_hi - a.window + 1);
    if (need_mask) {
      const int lim = (int)(qpos - kt0) - 4 * hi;
#pragma unroll
      for (int nt = 0; nt < NS; ++nt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int ko = 32 * nt + 8 * (r >> 2) + (r & 3);
          const bool ok = ko <= lim && ko > lim - wcap;
          s[nt][r] = ok ? s[nt][r] : -INFINITY;
        }
      }
    }
    float mt = -INFINITY;
#pragma unroll
    for (int nt = 0; nt < NS; ++nt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[nt][r]);
    }
    {
      float m0, m1;
      lane_halves(mt, m0, m1);
      mt = fmaxf(m0, m1) * sl;
    }

    // Lazy rescale: raise the reference only if some row's max exceeds it by
    // more than 8 (log2), keeping P <= 2^8.
    const bool grow = mt > m_ref + 8.0f;
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {
      // Rows that do not grow keep their reference (corr 1; also avoids
      // -inf - -inf for rows still fully masked); m_ref = -inf -> corr 0.
      const float corr = grow ? exp2_fast(m_ref - mt) : 1.0f;
      m_ref = grow ? mt : m_ref;
      l_run *= corr;
#pragma unroll
      for (int dt = 0; dt < ND; ++dt) o[dt] *= corr;
    }
    const float m_use = m_ref == -INFINITY ? 0.0f : m_ref;  // row masked so far

    f16x8 pf[PS];
#pragma unroll
    for (int nt = 0; nt < NS; ++nt) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        pf[2 * nt + (r >> 3)][r & 7] = (_Float16)exp2_fast(fmaf(s[nt][r], sl, -m_use));
    }
    // Row sum over the f16-rounded P, the values the PV MFMAs consume:
    // v_dot2_f32_f16 against (1, 1) adds two of them per instruction.
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 ones = {(_Float16)1.0f, (_Float16)1.0f};
    float ls = 0.0f;
#pragma unroll
    for (int i = 0; i < PS; ++i)
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const h2 pr = {pf[i][e], pf[i][e + 1]};
        ls = __builtin_amdgcn_fdot2(pr, ones, ls, false);
      }
    l_run += ls;

    // O^T += V^T P^T, VB dim tiles per batch; the next batch's fragments are
    // read while the current batch's MFMAs run.
#pragma unroll
    for (int d0 = 0; d0 < ND; d0 += VB) {
      if (d0 > 0) {
#pragma unroll
        for (int ks = 0; ks < PS; ++ks)
#pragma unroll
          for (int db = 0; db < VB; ++db)
            vf[ks][db] = *reinterpret_cast<const u32x4*>(vr + 32 * (d0 + db) * VPB + 32 * ks);
      }
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int ks = 0; ks < PS; ++ks)
#pragma unroll
        for (int db = 0; db < VB; ++db)
          o[d0 + db] = mfma_pv(__builtin_bit_cast(f16x8, vf[ks][db]), pf[ks], o[d0 + db]);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(0);
    }
  };

  // Key loop, two tiles per trip so each stage is a fixed LDS object.  Per
  // tile: barrier (the stage to read is complete; every wave is done with the
  // other stage), fetch the next tile into registers, compute, then store the
  // fetched tile into the other stage.
  if (kt_first < kend) {
    fetch(kt_first);
    stage(k_lds0, v_lds0);
  }
  for (long long kt0 = kt_first; kt0 < kend; kt0 += 2 * BN) {
    __syncthreads();
    const bool more1 = kt0 + BN < kend;
    if (more1) fetch(kt0 + BN);
    compute(k_lds0, v_lds0, kt0);
    if (!more1) break;
    stage(k_lds1, v_lds1);
    __syncthreads();
    const bool more2 = kt0 + 2 * BN < kend;
    if (more2) fetch(kt0 + 2 * BN);
    compute(k_lds1, v_lds1, kt0 + BN);
    if (!more2) break;
    stage(k_lds0, v_lds0);
  }

  // out[mq][h][d] = O^T[d][mq] / l.  The lane holds d = 32dt + 8(r/4) +
  // 4hi + (r%4): four consecutive dims per r/4, written as one 16-byte store.
  float l0, l1;
  lane_halves(l_run, l0, l1);
  const float l_tot = l0 + l1;
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

#define VTB_PREFILL(DTN, DTT, D)                                                           \
  extern "C" __global__ __launch_bounds__(256, vtb::prefill_waves_per_simd(D))                  \
  void vtb_prefill_##DTN##_d##D(vtb::PrefillArgs a) {                                         \
    vtb::prefill_body<vtb::DTT, D, 4>(a);                                                  \
  }                                                                                        \
  extern "C" __global__ __launch_bounds__(256) void vtb_vt_##DTN##_d##D(vtb::VtArgs a) {   \
    vtb::vt_body<vtb::DTT, D>(a);                                                          \
  }

// Wide variant (d <= 128): 8 waves x 32 queries share one set of staged
// K / V^T tiles.  The body needs ~214 VGPRs, so a CU holds one such
// workgroup: the same 8 waves (2 per SIMD) as two 4-wave workgroups, with
// each staged byte feeding twice the queries.
#define VTB_PREFILL_WIDE(DTN, DTT, D)                                                      \
  extern "C" __global__ __launch_bounds__(512, 2)                                          \
  void vtb_prefill8_##DTN##_d##D(vtb::PrefillArgs a) {                                        \
    vtb::prefill_body<vtb::DTT, D, 8>(a);                                                  \
  }

VTB_PREFILL_WIDE(bf16, kv_bf16, 64)
VTB_PREFILL_WIDE(bf16, kv_bf16, 128)
VTB_PREFILL_WIDE(f16, kv_f16, 64)
VTB_PREFILL_WIDE(f16, kv_f16, 128)

VTB_PREFILL(bf16, kv_bf16, 64)
VTB_PREFILL(bf16, kv_bf16, 128)
VTB_PREFILL(bf16, kv_bf16, 256)
VTB_PREFILL(f16, kv_f16, 64)
VTB_PREFILL(f16, kv_f16, 128)
VTB_PREFILL(f16, kv_f16, 256)
