// Causal prefill attention on CDNA4 MFMA (gfx950).
//
// Computes, for every query b of a prompt (position pos0 + b) and head h,
// exactly the attention of prefill.attentionCausal
// (src/runtime/prefill.zig:237-287):
//   out[b,h] = sum_t softmax_t(q[b,h].K[t,kv_h] / sqrt(D)) V[t,kv_h]
// over t in [window_start(pos0+b), pos0+b], kv_h = (h*n_kv)/n_heads.
//
// Kernels per call:
//   vtb_kvt_<dt>_d<D>      pre-pass, one workgroup per (64-key tile, KV
//                          head) over the tiles some query attends: V^T as
//                          f16, [kv_h][d][key], keys permuted inside each
//                          16-key group (vt_col), zero-padded to whole tiles;
//                          for bf16 caches also the keys as f16
//                          [kv_h][key][d].  A bf16 key tile is scaled by the
//                          power of two 2^-ek that brings its largest |k|
//                          into [2^14, 2^15), a value tile by 2^-ev with ev
//                          that exponent rounded up to a multiple of 4: exact
//                          for every value within 2^25 of the tile's maximum
//                          (f16's normal range holds every 8-bit bf16
//                          mantissa), whatever the absolute range; (ek, ev)
//                          go to texp.  f16 caches are f16 already.  Each
//                          tile's statistics (largest |k|, sum of k^2,
//                          largest key-row |k_t|^2, keys, largest |v|, sum
//                          of v^2) go to tstat for the precision choice.
//   vtb_prefill_d<D>       flash attention, transposed so that every lane
//                          owns one query:
//     q                    read as f32 (prefill.zig's s.q), scaled per wave
//                          (32 queries of one head) by the power of two that
//                          brings the largest magnitude into [2^14, 2^15),
//                          rounded to f16 (11 significant bits); the score
//                          multiplier takes the scales of q and K back.
//     S^T = K Q^T          v_mfma_f32_32x32x16_f16; A = K rows from LDS,
//                          B = Q^T kept in registers for the whole key loop;
//                          the tile's key exponent joins the score multiplier.
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
//                          holds in P^T 8 contiguous f16 of a V^T row.  O is
//                          held in units of 2^E, E the value exponent of the
//                          tiles accumulated (a tile with another one
//                          rescales O first); 2^E comes back out with the
//                          final 1/l.
// P is rounded to f16 (11 significant bits; bf16's 8 bits would give ~2e-3
// relative error, at the parity bar).
//
// Precision.  With 11-bit q and P the output error grows with the score
// magnitude (q's rounding error is weighted by |k|) and with the crest
// factor of V (P's rounding error is weighted by |v - out|).  N(0,1) data
// stays near 7e-4 of max|out|; channel outliers x20 (crest ~27) reach
// ~7e-3 with one piece.  A work item whose key tiles allow large scores
// therefore enters q as two f16 pieces (hi + lo, 22 significant bits), one
// whose value tiles have a large crest factor P likewise (prefill_entry):
// twice the QK or the PV products for those items only.
//
// Workgroup = 4 waves x 32 queries = 128 queries of one head; key tiles of BN
// rows stream through LDS (K row-major, V^T row-major, both padded so the
// 16-byte MFMA operand reads are bank-conflict free), the next tile written
// by LDS DMA (buffer_load ... lds) while the current one is computed.  Tiles
// entirely above a wave's diagonal or before its window are skipped.
#include "common.h"
#include "../tiles.h"

namespace vtb {



__device__ inline f32x16 mfma_qk(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
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
// Power-of-two scaling: scale_exp / pow2f (common.h).

// Max over the 64 lanes of a wave (every lane gets it).
__device__ inline float wave_max(float v) {
  v = fmaxf(v, dpp<DPP_XOR1>(v));
  v = fmaxf(v, dpp<DPP_XOR2>(v));
  v = fmaxf(v, dpp<DPP_HALF_MIRROR>(v));
  v = fmaxf(v, dpp<DPP_MIRROR>(v));
  v = xor_max<16>(v);
  return xor_max<32>(v);
}

// |x| maximum over the eight 16-bit values of w; returns their sum of
// squares.
template <typename DT>
__device__ inline float stat8(u32x4 w, float& mx) {
  float f[8];
  Unpack<DT>::run(w, f);
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    mx = fmaxf(mx, fabsf(f[e]));
    ss = fmaf(f[e], f[e], ss);
  }
  return ss;
}

// Value exponent of a bf16 tile: scale_exp of its largest |v| rounded up to
// a multiple of 4 (largest scaled magnitude in [2^11, 2^15)), so tiles of
// similar range share it; kEvAny for an all-zero tile (any scale holds it).
constexpr int kEvAny = -1000;
__device__ inline int value_exp(float vmx) {
  if (vmx == 0.0f) return kEvAny;
  return ((scale_exp(vmx) + 3) >> 2) << 2;  // arithmetic shift: floor, so ceil to 4
}

// One pass per (64-key tile, KV head): statistics, exponents and the f16
// operands of the tile.  Keys at or past n_rows are zero.
template <typename DT, int D>
__device__ __forceinline__ void kvt_body(const KvtArgs& a) {
  constexpr int TK = 64;                 // keys per workgroup
  constexpr int TP = D + 8;              // LDS pitch (16-bit elements)
  constexpr int CPR = D / 8;             // 16-byte chunks per row
  constexpr int CH = TK * D / 8 / 256;   // 16-byte chunks per thread
  constexpr bool kBf = __is_same(DT, kv_bf16);
  static_assert(CH * 256 * 8 == TK * D, "tile does not match the workgroup");
  __shared__ __attribute__((aligned(16))) uint16_t tile[TK * TP];
  __shared__ float s_st[4][5];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int kvh = blockIdx.y;
  const int tix = blockIdx.x + a.tile_lo;
  const int n_tiles = a.vt_ld / TK;
  const long long key0 = (long long)tix * TK;
  const long long row_stride = (long long)a.n_kv * D;
  const uint16_t* vg = (const uint16_t*)a.v + (long long)kvh * D;
  const uint16_t* kg = (const uint16_t*)a.k + (long long)kvh * D;
  // 64 keys x D dims of K and V, CH 16-byte chunks of each per thread
  // (chunk c: key c / CPR, dims 8 (c % CPR) ..); a row's CPR chunks sit in
  // CPR consecutive lanes.  V goes to LDS as it is for the transpose; K
  // stays in registers until the tile's key exponent is known.
  u32x4 kw[CH], vw[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int c = tid + 256 * i;
    const int key = c / CPR, dc = (c % CPR) * 8;
    const bool in = key0 + key < a.n_rows;
    const long long off = (key0 + key) * row_stride + dc;
    kw[i] = in ? load16(kg + off) : u32x4{0u, 0u, 0u, 0u};
    vw[i] = in ? load16(vg + off) : u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int c = tid + 256 * i;
    *reinterpret_cast<u32x4*>(&tile[(c / CPR) * TP + (c % CPR) * 8]) = vw[i];
  }
  // Statistics: largest |k|, sum of k^2, largest |k_t|^2 of a key row,
  // largest |v|, sum of v^2 (zero rows add nothing).
  float kmx = 0.0f, kss = 0.0f, kn2 = 0.0f, vmx = 0.0f, vss = 0.0f;
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const float kc = stat8<DT>(kw[i], kmx);
    kss += kc;
    kn2 = fmaxf(kn2, group_sum<CPR>(kc));
    vss += stat8<DT>(vw[i], vmx);
  }
  kmx = wave_max(kmx);
  kn2 = wave_max(kn2);
  vmx = wave_max(vmx);
  kss = group_sum<64>(kss);
  vss = group_sum<64>(vss);
  if (lane == 0) {
    s_st[wave][0] = kmx;
    s_st[wave][1] = kss;
    s_st[wave][2] = kn2;
    s_st[wave][3] = vmx;
    s_st[wave][4] = vss;
  }
  __syncthreads();
  // The tile's maxima, the same in every thread (the exponents must agree
  // with what thread 0 records).
  kmx = s_st[0][0];
  vmx = s_st[0][3];
#pragma unroll
  for (int w = 1; w < 4; ++w) {
    kmx = fmaxf(kmx, s_st[w][0]);
    vmx = fmaxf(vmx, s_st[w][3]);
  }
  if (tid == 0) {
    f32x4 r0 = {s_st[0][0], s_st[0][1], s_st[0][2], 0.0f}, r1 = {s_st[0][3], s_st[0][4], 0.0f, 0.0f};
#pragma unroll
    for (int w = 1; w < 4; ++w) {
      r0[0] = fmaxf(r0[0], s_st[w][0]);
      r0[1] += s_st[w][1];
      r0[2] = fmaxf(r0[2], s_st[w][2]);
      r1[0] = fmaxf(r1[0], s_st[w][3]);
      r1[1] += s_st[w][4];
    }
    const long long valid = a.n_rows - key0;
    r0[3] = (float)(valid < TK ? valid : TK);
    float* dst = a.tstat + ((long long)kvh * n_tiles + tix) * 8;
    *reinterpret_cast<f32x4*>(dst) = r0;
    *reinterpret_cast<f32x4*>(dst + 4) = r1;
  }
  float vscale = 1.0f;
  if constexpr (kBf) {
    const int ek = scale_exp(kmx), ev = value_exp(vmx);
    vscale = pow2f(ev == kEvAny ? 0 : -ev);
    const float kscale = pow2f(-ek);
    if (tid == 0) *reinterpret_cast<int2*>(a.texp + ((long long)kvh * n_tiles + tix) * 2) = int2{ek, ev};
    // f16 keys [kv_h][key][d], scaled by 2^-ek.
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = tid + 256 * i;
      const int key = c / CPR, dc = (c % CPR) * 8;
      const uint32_t ww[4] = {kw[i].x, kw[i].y, kw[i].z, kw[i].w};
      f16x8 h;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        h[2 * e] = (_Float16)(__builtin_bit_cast(float, ww[e] << 16) * kscale);
        h[2 * e + 1] = (_Float16)(__builtin_bit_cast(float, ww[e] & 0xffff0000u) * kscale);
      }
      *reinterpret_cast<f16x8*>((_Float16*)a.k16 + ((long long)kvh * a.vt_ld + key0 + key) * D + dc) = h;
    }
  }
  // Write V^T rows: output column o of a 16-key group holds key vt_col(o).
  for (int c = tid; c < D * TK / 8; c += 256) {
    const int d = c / (TK / 8), o0 = (c % (TK / 8)) * 8;
    f16x8 h;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int o = o0 + e;
      const uint16_t bits = tile[(16 * (o >> 4) + vt_col(o & 15)) * TP + d];
      if constexpr (kBf)
        h[e] = (_Float16)(__builtin_bit_cast(float, (uint32_t)bits << 16) * vscale);
      else
        h[e] = __builtin_bit_cast(_Float16, bits);
    }
    *reinterpret_cast<f16x8*>((_Float16*)a.vt + ((long long)kvh * D + d) * a.vt_ld + key0 + o0) = h;
  }
}

// ---------------------------------------------------------------- attention
// XQ / XP: q / P enter their MFMAs as two f16 pieces (hi + lo, 22
// significant bits), twice the products of the single-piece form.
// The K and V^T tile stages of one workgroup: two of each, so tile j is read
// from stage j%2 while tile j+1 is written into the other and one barrier
// per tile suffices.  K rows are padded by one 16-byte chunk, V^T rows
// likewise (bank spread).  Declared once per kernel in the entry and shared
// by both precision paths, so a workgroup holds one set.  Four separate
// __shared__ arrays rather than one object: the compiler then knows a DMA
// into one stage cannot write the stage being read, and does not wait for
// the DMA before those reads.
// LDS-typed bytes: stage pointers stay in the local address space, so
// reads are ds_reads and DMA targets need no address-space conversion.
typedef __attribute__((address_space(3))) char lchar;
template <typename T>
__device__ __forceinline__ T lds_load(const lchar* p) {
  return *reinterpret_cast<const __attribute__((address_space(3))) T*>(p);
}

template <int D>
struct PrefillLds {
  static constexpr int BN = prefill_block_n(D);
  static constexpr int KBYTES = BN * (D / 8 + 1) * 16;
  static constexpr int VBYTES = D * (BN / 8 + 1) * 16;
  lchar* k0;
  lchar* k1;
  lchar* v0;
  lchar* v1;
  // Key-split form only: the second key tile of each step (stage sets
  // {k0, v0, k2, v2} and {k1, v1, k3, v3}).
  lchar* k2;
  lchar* k3;
  lchar* v2;
  lchar* v3;
};

// Tile staging by LDS DMA (buffer_load_dwordx4 ... lds): a stage is filled
// in 1 KB blocks, each one instruction of one wave whose 64 lanes write 16
// bytes each, in lane order, from the block's LDS offset on.  Slot s = 64 b +
// lane of a stage is 16-byte chunk s % (C + 1) of row s / (C + 1) of the
// padded layout (C chunks per row, one pad chunk); the pad slot's lane loads
// chunk 0 of its row (never read).  Block b belongs to wave b % NW.  K rows
// at or past kend lie outside the tile's buffer resource and read as zero
// (those keys are masked for every query here); V^T tiles are whole (the
// conversion pass zero-pads the last).  No registers hold a tile in flight;
// completion is counted by vmcnt (wait_loads() before the barrier that
// publishes a stage).  Offsets are 32-bit: the host keeps a K tile and a
// V^T head below 2 GiB.
template <int D, int NW>
struct TileDma {
  static constexpr int BN = prefill_block_n(D);
  static constexpr int KCH = D / 8;
  static constexpr int VCH = BN / 8;
  static constexpr int KSL = BN * (KCH + 1);   // 16-byte slots per K stage
  static constexpr int VSL = D * (VCH + 1);    // per V^T stage
  static constexpr int KBL = (KSL + 63) / 64;  // 1 KB blocks
  static constexpr int VBL = (VSL + 63) / 64;
  static constexpr int KPW = (KBL + NW - 1) / NW;
  static constexpr int VPW = (VBL + NW - 1) / NW;
  int wave, lane;
  int koff[KPW], voff[VPW];  // this lane's source byte offsets inside a tile
  __device__ __forceinline__ TileDma(int wave_, int lane_, int krow_bytes, int vrow_bytes) : wave(wave_), lane(lane_) {
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      const int sl = 64 * (wave + NW * i) + lane, row = sl / (KCH + 1), ch = sl % (KCH + 1);
      koff[i] = row * krow_bytes + 16 * (ch == KCH ? 0 : ch);
    }
#pragma unroll
    for (int i = 0; i < VPW; ++i) {
      const int sl = 64 * (wave + NW * i) + lane, row = sl / (VCH + 1), ch = sl % (VCH + 1);
      voff[i] = row * vrow_bytes + 16 * (ch == VCH ? 0 : ch);
    }
  }
  // Keys [kt0, kt0 + BN) of a head's K rows (kbase, krow_bytes apart; rows
  // from kend on excluded) into the K stage kl.
  __device__ __forceinline__ void issue_k(const char* kbase, long long krow_bytes, long long kend, long long kt0,
                                          lchar* kl) const {
    const long long rows = kend - kt0 < BN ? kend - kt0 : BN;
    const auto r = buffer_rsrc(kbase + kt0 * krow_bytes, (unsigned)(rows * krow_bytes));
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      const int blk = wave + NW * i;
      // Rounds in which every wave has a block need no wave check (a
      // compile-time fact the compiler cannot see from wave < NW).
      if (((i + 1) * NW <= KBL || blk < KBL) && (KSL % 64 == 0 || 64 * blk + lane < KSL))
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, reinterpret_cast<__attribute__((address_space(3))) void*>(kl + 1024 * blk), 16,
                                                 koff[i], 0, 0, 0);
    }
  }
  // Keys [kt0, kt0 + BN) of a head's V^T (vbase; rows of vrow_bytes) into the
  // V^T stage vl.
  __device__ __forceinline__ void issue_v(const char* vbase, int vrow_bytes, long long kt0, lchar* vl) const {
    const auto r = buffer_rsrc(vbase + kt0 * 2, (unsigned)((D - 1) * vrow_bytes + BN * 2));
#pragma unroll
    for (int i = 0; i < VPW; ++i) {
      const int blk = wave + NW * i;
      if (((i + 1) * NW <= VBL || blk < VBL) && (VSL % 64 == 0 || 64 * blk + lane < VSL))
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, reinterpret_cast<__attribute__((address_space(3))) void*>(vl + 1024 * blk), 16,
                                                 voff[i], 0, 0, 0);
    }
  }
};

// Kernels built with balanced pairs of query blocks (prefill_entry).  Only
// d256, whose one-wave-per-SIMD workgroups fill the CUs once (C5: 256
// workgroups): there the longest causal block set the launch time.  The
// d <= 128 kernels spilled 21-28 VGPRs with the extra work-item state; the
// 4-wave d128 kernel measured 34-35 against 31 us at 512 tokens balanced.
template <int D>
constexpr bool kBalanced = D >= 256;

// 2^e for an exponent difference e, clamped to pow2f's range: O rescaled by
// more than 2^126 either way has left f32 anyway.
__device__ inline float pow2_diff(int e) { return pow2f(e < -126 ? -126 : (e > 126 ? 126 : e)); }

// A piece of a split query block (balanced launches): publish this
// workgroup's unnormalised partial (o, m, l per thread, o in units of 2^E)
// with coherent stores and count it in; the second piece to arrive loads
// the first's and merges them, always as piece 0's terms plus piece 1's, so
// the result does not depend on the arrival order.  Returns true in the
// workgroup that then writes the block's output.  Layout: part_o[slot]
// [piece][j][thread] float4 (j < D/8: the thread's o, consecutive threads
// adjacent), part_ml[slot][piece][thread] float4 (m, l, E, 0); slot =
// head * nblk/2 + pair.
template <int D, int NW>
__device__ __forceinline__ bool prefill_merge_pieces(const PrefillArgs& a, int h, int qb, int piece,
                                                    f32x16 (&o)[D / 32], float& m_ref, float& l_run, int& E) {
  constexpr int NT = 64 * NW, ND = D / 32, J = D / 8;
  __shared__ int s_last;
  const int tid = threadIdx.x;
  const int nblk = gridDim.y;
  const long long slot = (long long)h * (nblk / 2) + (nblk - 1 - qb);
  const long long mine = slot * 2 + piece, other = slot * 2 + (1 - piece);
  {
    const auto rw = buffer_rsrc(a.part_o + mine * J * NT * 4, J * NT * 16);
#pragma unroll
    for (int dt = 0; dt < ND; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4)
        buffer_store_f4_coherent(rw, ((4 * dt + q4) * NT + tid) * 16,
                                 f32x4{o[dt][4 * q4], o[dt][4 * q4 + 1], o[dt][4 * q4 + 2], o[dt][4 * q4 + 3]});
    const auto rm = buffer_rsrc(a.part_ml + mine * NT * 4, NT * 16);
    buffer_store_f4_coherent(rm, tid * 16, f32x4{m_ref, l_run, (float)E, 0.0f});
  }
  wait_stores();
  __syncthreads();
  if (tid == 0) {
    unsigned* ctr = a.part_ctr + slot * 32;
    const unsigned prev = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = prev == 1u;
    if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last;
  }
  __syncthreads();
  if (!s_last) return false;
  const auto rr = buffer_rsrc(a.part_o + other * J * NT * 4, J * NT * 16);
  const f32x4 mlo = buffer_load_f4_coherent(buffer_rsrc(a.part_ml + other * NT * 4, NT * 16), tid * 16);
  const float mo = mlo[0], lo = mlo[1];
  const int Eo = (int)mlo[2];
  const float M = fmaxf(m_ref, mo);
  const float fm = m_ref == -INFINITY ? 0.0f : exp2_fast(m_ref - M);
  const float fo = mo == -INFINITY ? 0.0f : exp2_fast(mo - M);
  // o terms also move from their own value exponent to the larger one.
  const int Em = E > Eo ? E : Eo;
  const float gm = fm * pow2_diff(E - Em), go = fo * pow2_diff(Eo - Em);
  const float f0 = piece == 0 ? fm : fo, f1 = piece == 0 ? fo : fm;
  const float g0 = piece == 0 ? gm : go, g1 = piece == 0 ? go : gm;
#pragma unroll
  for (int dt = 0; dt < ND; ++dt) {
    f32x4 ov[4];
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) ov[q4] = buffer_load_f4_coherent(rr, ((4 * dt + q4) * NT + tid) * 16);
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float mv = o[dt][4 * q4 + e], xv = ov[q4][e];
        const float v0 = piece == 0 ? mv : xv, v1 = piece == 0 ? xv : mv;
        o[dt][4 * q4 + e] = v0 * g0 + v1 * g1;
      }
  }
  const float l0v = piece == 0 ? l_run : lo, l1v = piece == 0 ? lo : l_run;
  l_run = l0v * f0 + l1v * f1;
  m_ref = M;
  E = Em;
  return true;
}

// out[mq][h][d] = O^T[d][mq] * 2^E / l.  The lane holds d = 32dt + 8(r/4) +
// 4hi + (r%4): four consecutive dims per r/4, written as one 16-byte store.
// The row sum is split over the lane pair (hi = 0, 1); E is the value
// exponent O is held in.
template <int D>
__device__ __forceinline__ void prefill_write_out(const PrefillArgs& a, int h, int mq, int hi,
                                                  const f32x16 (&o)[D / 32], float l_run, int E) {
  float l0, l1;
  lane_halves(l_run, l0, l1);
  const float l_tot = l0 + l1;
  if (mq < a.n_q) {
    const float inv = (1.0f / l_tot) * pow2_diff(E);
    float* op = a.out + ((long long)mq * a.n_heads + h) * D + 4 * hi;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
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

// A work item's keys: [kbeg, kend) = [k_lo, k_hi) intersected with the keys
// some query of block qb may attend (its causal end, its first query's
// window start).
template <int BM>
__device__ __forceinline__ void item_keys(const PrefillArgs& a, int qb, long long k_lo, long long k_hi,
                                          long long& kbeg, long long& kend) {
  const int m0 = qb * BM;
  const int m_last = (m0 + BM < a.n_q ? m0 + BM : a.n_q) - 1;
  kend = a.pos0 + m_last + 1;
  if (k_hi < kend) kend = k_hi;
  kbeg = k_lo;
  const long long q_lo = a.pos0 + m0;
  if (a.window > 0 && q_lo >= a.window && q_lo - a.window + 1 > kbeg) kbeg = q_lo - a.window + 1;
}

// A KV head's f16 key rows and V^T rows, as the tile DMA reads them.
struct TileSrc {
  const char* kbase;
  const char* vbase;
  long long krow_bytes;
  int vrow_bytes;
};
template <int D>
__device__ __forceinline__ TileSrc tile_src(const PrefillArgs& a, int kvh) {
  return TileSrc{(const char*)((const _Float16*)a.k + (long long)kvh * a.k_head_stride),
                 (const char*)((const _Float16*)a.vt + (long long)kvh * D * a.vt_ld), a.k_row_stride * 2,
                 a.vt_ld * 2};
}

// One work item: queries of block qb against keys [k_lo, k_hi) (intersected
// with each query's causal and window range); piece < 0: the whole block
// (write the output), else a piece of a split block (prefill_merge_pieces).
// The entry has issued the DMA of the item's first key tile into stage 0
// (key-split: its first two tiles, into k0/v0 and k2/v2) and the load of
// that tile's exponents (x_first; key-split: the wave's own tile's).
template <int D, int NW, bool XQ, bool XP, bool KSPLIT>
__device__ __forceinline__ void prefill_body(const PrefillArgs& a, const int h, const int qb, const int kvh,
                                             const f16x8 (&qf)[D / 16], const f16x8 (&ql)[D / 16],
                                             const int eq, PrefillLds<D>& lds, const long long k_lo,
                                             const long long k_hi, const int piece, const int2 x_first) {
  constexpr int NT = 64 * NW;                 // threads per workgroup
  constexpr int BM = prefill_item_queries(NW, KSPLIT);  // queries per work item
  constexpr int BN = prefill_block_n(D);      // keys per tile
  constexpr int KCH = D / 8;                  // 16-byte chunks per K row
  constexpr int VCH = BN / 8;                 // 16-byte chunks per V^T row
  constexpr int KPB = (KCH + 1) * 16;         // LDS pitch of a K row: one pad chunk
  constexpr int VPB = (VCH + 1) * 16;         // LDS pitch of a V^T row
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
  // O^T tiles per V-fragment batch (one in the two-piece forms, whose second
  // q or P pieces take the registers).
  constexpr int VB = (XQ || XP) ? 1 : (ND < VTB_PF_VB ? ND : VTB_PF_VB);
  static_assert(NS % KB == 0 && ND % VB == 0, "batches must divide the tiles");
  // The register-tight case: two-piece q in the 4-wave d128 kernel.
  constexpr bool LATE = XQ && NW == 4 && D == 128;

  static_assert(PrefillLds<D>::KBYTES == BN * KPB && PrefillLds<D>::VBYTES == D * VPB, "LDS stage size");
  lchar* const k_lds0 = lds.k0;
  lchar* const k_lds1 = lds.k1;
  lchar* const v_lds0 = lds.v0;
  lchar* const v_lds1 = lds.v1;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int hi = lane >> 5;   // lane half
  const int lc = lane & 31;   // lane column: the query this lane owns
  // The wave's 32 queries (sub-block wsb of the item) and, in the key-split
  // form, its key half kh: of each step's two key tiles it computes tile kh.
  const int wsb = KSPLIT ? wave >> 1 : wave;
  const int kh = KSPLIT ? wave & 1 : 0;

  const int m0 = qb * BM;
  const int mq = m0 + wsb * 32 + lc;  // this lane's query (may be >= n_q: padding)
  const long long qpos = a.pos0 + mq;
  const long long q_lo = a.pos0 + m0;  // first query position of the workgroup
  long long kbeg, kend;  // keys [kbeg, kend) may be attended
  item_keys<BM>(a, qb, k_lo, k_hi, kbeg, kend);
  const long long kt_first = kbeg / BN * BN;

  // Wave-level query range, for tile skipping.
  const long long wq_lo = a.pos0 + m0 + wsb * 32;
  const long long wq_hi = a.pos0 + (m0 + wsb * 32 + 31 < a.n_q ? m0 + wsb * 32 + 31 : a.n_q - 1);
  const bool wave_live = m0 + wsb * 32 < a.n_q;

  const TileSrc src = tile_src<D>(a, kvh);
  const char* const kbase = src.kbase;
  const char* const vbase = src.vbase;
  const long long krow_bytes = src.krow_bytes;
  const int vrow_bytes = src.vrow_bytes;
  const TileDma<D, NW> dma(wave, lane, (int)krow_bytes, vrow_bytes);
  auto fetch = [&](long long kt0, lchar* kl, lchar* vl) {
    dma.issue_k(kbase, krow_bytes, kend, kt0, kl);
    dma.issue_v(vbase, vrow_bytes, kt0, vl);
  };

  // Q^T fragments (B operand) from the entry: qf (and the second pieces ql,
  // read only by the two-piece q form), scaled by 2^-eq.
  // The pre-pass's (key, value) exponents of each 64-key tile (null: f16
  // cache, both 0): a tile's score multiplier is scale_log2 * 2^(eq + ek),
  // the exponent sum clamped so the product stays a normal f32 (beyond it
  // every score is ~0 or overflows, as in f32); its V^T is in units of 2^ev.
  const int* texp_h = a.texp ? a.texp + (long long)kvh * (a.vt_ld >> 6) * 2 : nullptr;

  f32x16 o[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i) o[i] = f32x16{};
  float m_ref = -INFINITY;  // running reference max (log2 domain, scaled)
  float l_run = 0.0f;
  // O is held in units of 2^E, E the value exponent of the last tile this
  // wave accumulated (wave-uniform); a tile with another exponent first
  // rescales O by a power of two (exact).
  int E = 0;
  int acc = 0;  // some tile was accumulated (wave-uniform)
  // The window as a 32-bit bound (positions stay below 2^30; a larger or
  // absent window keeps every causal key).
  const int wcap = (a.window > 0 && a.window < (1 << 30)) ? (int)a.window : (1 << 30);
  // The per-tile checks in 32-bit scalar arithmetic (positions stay below
  // 2^30; a window of 2^30 or more excludes no key, like none): wave-uniform
  // values in SGPRs, so the checks are SALU compares rather than 64-bit
  // vector ones.
  const int iwin = __builtin_amdgcn_readfirstlane(wcap < (1 << 30) ? wcap : 0);
  const int iwq_lo = __builtin_amdgcn_readfirstlane((int)wq_lo);
  const int iwq_hi = __builtin_amdgcn_readfirstlane((int)wq_hi);
  const int iqpos = (int)qpos;

  auto compute = [&](const lchar* kl, const lchar* vl, long long kt0, int ek, int evt) {
    // Skip tiles entirely above this wave's diagonal or before its windows.
    const int t0 = __builtin_amdgcn_readfirstlane((int)kt0);
    bool live = wave_live && t0 <= iwq_hi;
    if (iwin > 0 && t0 + BN - 1 < iwq_lo - iwin + 1) live = false;
    if (!live) return;
    acc = 1;
    evt = evt == kEvAny ? E : evt;  // an all-zero tile fits any unit
    int es = eq + ek;
    es = es < -120 ? -120 : (es > 120 ? 120 : es);
    const float sl = a.scale_log2 * pow2f(es);


    // S^T = K Q^T.  K fragments (row 32nt + lc, chunk 2ks + hi) are read in
    // batches of KB S^T tiles so their LDS latency overlaps the MFMAs (in
    // KH parts of the k-steps in the register-tight two-piece form).
    constexpr int KH = LATE ? 2 : 1;
    constexpr int KSH = KS / KH;
    const lchar* kr = kl + lc * KPB + 16 * hi;
    f32x16 s[NS];
#pragma unroll
    for (int nt = 0; nt < NS; ++nt) s[nt] = f32x16{};
#pragma unroll
    for (int n0 = 0; n0 < NS; n0 += KB) {
#pragma unroll
      for (int k0 = 0; k0 < KS; k0 += KSH) {
        u32x4 kf[KSH][KB];
#pragma unroll
        for (int ks = 0; ks < KSH; ++ks)
#pragma unroll
          for (int nb = 0; nb < KB; ++nb)
            kf[ks][nb] = lds_load<u32x4>(kr + 32 * (n0 + nb) * KPB + 32 * (k0 + ks));
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int ks = 0; ks < KSH; ++ks)
#pragma unroll
          for (int nb = 0; nb < KB; ++nb)
            s[n0 + nb] = mfma_qk(__builtin_bit_cast(f16x8, kf[ks][nb]), qf[k0 + ks], s[n0 + nb]);
        if constexpr (XQ) {
#pragma unroll
          for (int ks = 0; ks < KSH; ++ks)
#pragma unroll
            for (int nb = 0; nb < KB; ++nb)
              s[n0 + nb] = mfma_qk(__builtin_bit_cast(f16x8, kf[ks][nb]), ql[k0 + ks], s[n0 + nb]);
        }
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
      }
    }

    // First V^T batch (dims 0 .. 32VB) for the PV product, in flight during
    // the softmax.
    const lchar* vr = vl + lc * VPB + 16 * hi;
    u32x4 vf[PS][VB];
#pragma unroll
    for (int ks = 0; ks < PS; ++ks)
#pragma unroll
      for (int db = 0; db < VB; ++db) vf[ks][db] = lds_load<u32x4>(vr + 32 * db * VPB + 32 * ks);

    // Mask (diagonal / window tiles only: a wave-uniform branch).  Key
    // 32nt + 8(r/4) + 4hi + r%4 of the tile is kept iff it lies in
    // (qpos - window, qpos]; lim is qpos relative to this lane's first key.
    const bool need_mask = (t0 + BN - 1 > iwq_lo) || (iwin > 0 && t0 < iwq_hi - iwin + 1);
    if (need_mask) {
      const int lim = iqpos - t0 - 4 * hi;
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
    // more than 8 (log2), keeping P <= 2^8.  A change of value exponent
    // rescales O in the same multiply.
    const bool grow = mt > m_ref + 8.0f;
    if (__builtin_amdgcn_ballot_w64(grow) != 0 || evt != E) {
      // Rows that do not grow keep their reference (corr 1; also avoids
      // -inf - -inf for rows still fully masked); m_ref = -inf -> corr 0.
      const float corr = grow ? exp2_fast(m_ref - mt) : 1.0f;
      m_ref = grow ? mt : m_ref;
      l_run *= corr;
      const float oc = corr * pow2_diff(E - evt);
      E = evt;
#pragma unroll
      for (int dt = 0; dt < ND; ++dt) o[dt] *= oc;
    }
    const float m_use = m_ref == -INFINITY ? 0.0f : m_ref;  // row masked so far

    f16x8 pf[PS], pl[XP ? PS : 1];
#pragma unroll
    for (int nt = 0; nt < NS; ++nt) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
      {
        const float pv = exp2_fast(fmaf(s[nt][r], sl, -m_use));
        pf[2 * nt + (r >> 3)][r & 7] = (_Float16)pv;
        if constexpr (XP) pl[2 * nt + (r >> 3)][r & 7] = (_Float16)(pv - (float)pf[2 * nt + (r >> 3)][r & 7]);
      }
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
        if constexpr (XP) {
          const h2 pr2 = {pl[i][e], pl[i][e + 1]};
          ls = __builtin_amdgcn_fdot2(pr2, ones, ls, false);
        }
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
            vf[ks][db] = lds_load<u32x4>(vr + 32 * (d0 + db) * VPB + 32 * ks);
      }
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int ks = 0; ks < PS; ++ks)
#pragma unroll
        for (int db = 0; db < VB; ++db)
          o[d0 + db] = mfma_pv(__builtin_bit_cast(f16x8, vf[ks][db]), pf[ks], o[d0 + db]);
      if constexpr (XP) {
#pragma unroll
        for (int ks = 0; ks < PS; ++ks)
#pragma unroll
          for (int db = 0; db < VB; ++db)
            o[d0 + db] = mfma_pv(__builtin_bit_cast(f16x8, vf[ks][db]), pl[ks], o[d0 + db]);
      }
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(0);
    }
  };

  // Key loop, two tiles per trip so each stage is a fixed LDS object.  Per
  // tile: barrier (the stage to read is complete; every wave is done with the
  // other stage), DMA of the next tile into the other stage, compute, wait
  // for this wave's DMA.  The next tile's exponents are read with its DMA,
  // as a vector load that the same wait covers: a scalar load would be
  // waited for together with the tile's LDS fragment reads (one counter).
  // (Moved to scalar registers right after that wait, so no later
  // instruction waits on them.)
  auto texp_of = [&](long long kt0) -> int2 {
    return texp_h ? *reinterpret_cast<const int2*>(texp_h + (kt0 >> 6) * 2) : int2{0, 0};
  };
  int2 x0 = {0, 0}, x1 = {0, 0};
  const int ikend = __builtin_amdgcn_readfirstlane((int)kend);
  const int ikt_first = __builtin_amdgcn_readfirstlane((int)kt_first);
  auto uniform2 = [](int2 x) { return int2{__builtin_amdgcn_readfirstlane(x.x), __builtin_amdgcn_readfirstlane(x.y)}; };
  if constexpr (!KSPLIT) {
    if (ikt_first < ikend) {
      x0 = x_first;
      wait_loads();
      x0 = uniform2(x0);
      E = x0.y == kEvAny ? 0 : x0.y;
    }
    for (int kt0 = ikt_first; kt0 < ikend; kt0 += 2 * BN) {
      __syncthreads();
      const bool more1 = kt0 + BN < ikend;
      if (more1) {
        fetch(kt0 + BN, k_lds1, v_lds1);
        x1 = texp_of(kt0 + BN);
      }
      compute(k_lds0, v_lds0, kt0, x0.x, x0.y);
      if (!more1) break;
      wait_loads();
      x1 = uniform2(x1);
      __syncthreads();
      const bool more2 = kt0 + 2 * BN < ikend;
      if (more2) {
        fetch(kt0 + 2 * BN, k_lds0, v_lds0);
        x0 = texp_of(kt0 + 2 * BN);
      }
      compute(k_lds1, v_lds1, kt0 + BN, x1.x, x1.y);
      if (!more2) break;
      wait_loads();
      x0 = uniform2(x0);
    }
  } else {
    // Key-split form: each step stages two key tiles, t (for the kh = 0
    // waves) and t + BN (kh = 1), in one stage set while the other set is
    // computed: sets {k0, v0, k2, v2} and {k1, v1, k3, v3}.  A tile at or
    // past the item's last key is neither fetched nor read (no wave is live
    // for it) and its exponents are not loaded.
    lchar* const k_lds2 = lds.k2;
    lchar* const k_lds3 = lds.k3;
    lchar* const v_lds2 = lds.v2;
    lchar* const v_lds3 = lds.v3;
    auto fetch2 = [&](int t, lchar* ka, lchar* va, lchar* kb, lchar* vb) {
      fetch(t, ka, va);
      if (t + BN < ikend) fetch(t + BN, kb, vb);
    };
    auto texp_own = [&](int t) -> int2 { return t + kh * BN < ikend ? texp_of(t + kh * BN) : int2{0, 0}; };
    if (ikt_first < ikend) {  // the entry issued the first step and this wave's exponent load
      x0 = x_first;
      wait_loads();
      x0 = uniform2(x0);
      E = x0.y == kEvAny ? 0 : x0.y;
    }
    for (int kt0 = ikt_first; kt0 < ikend; kt0 += 4 * BN) {
      __syncthreads();
      const bool more1 = kt0 + 2 * BN < ikend;
      if (more1) {
        fetch2(kt0 + 2 * BN, k_lds1, v_lds1, k_lds3, v_lds3);
        x1 = texp_own(kt0 + 2 * BN);
      }
      // One call per half (wave-uniform branch): with a select between the
      // stage pointers the compiler cannot tell the read stage from the one
      // the DMA above fills and waits for that DMA first.
      if (kh)
        compute(k_lds2, v_lds2, kt0 + BN, x0.x, x0.y);
      else
        compute(k_lds0, v_lds0, kt0, x0.x, x0.y);
      if (!more1) break;
      wait_loads();
      x1 = uniform2(x1);
      __syncthreads();
      const bool more2 = kt0 + 4 * BN < ikend;
      if (more2) {
        fetch2(kt0 + 4 * BN, k_lds0, v_lds0, k_lds2, v_lds2);
        x0 = texp_own(kt0 + 4 * BN);
      }
      if (kh)
        compute(k_lds3, v_lds3, kt0 + 3 * BN, x1.x, x1.y);
      else
        compute(k_lds1, v_lds1, kt0 + 2 * BN, x1.x, x1.y);
      if (!more2) break;
      wait_loads();
      x0 = uniform2(x0);
    }
    // The two key halves of each 32 queries: the kh = 1 wave hands its
    // partial (o, m, l per lane; E) to the kh = 0 wave through the free
    // stage buffers, which merges them as half 0's terms plus half 1's (the
    // same order every launch).  Both waves hold the same (dim, query) in
    // the same lane and register.
    typedef __attribute__((address_space(3))) float lfloat;
    static_assert(ND * 16 * 64 * 4 <= PrefillLds<D>::KBYTES && 130 * 4 <= PrefillLds<D>::VBYTES, "hand-off space");
    __syncthreads();  // every wave is done with the stages
    lfloat* const xo = (lfloat*)(wsb == 0 ? k_lds0 : k_lds1);
    lfloat* const xm = (lfloat*)(wsb == 0 ? v_lds0 : v_lds1);
    if (kh) {
#pragma unroll
      for (int dt = 0; dt < ND; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) xo[(dt * 16 + r) * 64 + lane] = o[dt][r];
      xm[lane] = m_ref;
      xm[64 + lane] = l_run;
      if (lane == 0) {
        xm[128] = __builtin_bit_cast(float, E);
        xm[129] = __builtin_bit_cast(float, acc);
      }
    }
    __syncthreads();
    if (kh) return;
    const float m1 = xm[lane], l1 = xm[64 + lane];
    const int E1 = __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, xm[128]));
    const int acc1 = __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, xm[129]));
    const float M = fmaxf(m_ref, m1);
    const float f0 = m_ref == -INFINITY ? 0.0f : exp2_fast(m_ref - M);
    const float f1 = m1 == -INFINITY ? 0.0f : exp2_fast(m1 - M);
    // The common unit: the larger of the two, or the other half's where one
    // half accumulated no tile (its E is only its first tile's, or none).
    const int Em = !acc1 ? E : (!acc ? E1 : (E > E1 ? E : E1));
    const float g0 = f0 * pow2_diff(E - Em), g1 = f1 * pow2_diff(E1 - Em);
#pragma unroll
    for (int dt = 0; dt < ND; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[dt][r] = o[dt][r] * g0 + xo[(dt * 16 + r) * 64 + lane] * g1;
    l_run = l_run * f0 + l1 * f1;
    m_ref = M;
    E = Em;
  }

  if constexpr (kBalanced<D>) {
    if (piece >= 0 && !prefill_merge_pieces<D, NW>(a, h, qb, piece, o, m_ref, l_run, E)) return;
  }

  prefill_write_out<D>(a, h, mq, hi, o, l_run, E);
}

// Entry: the workgroup's (head, query block), its queries in registers
// (f32) and its precision path, from the pre-pass statistics of the key
// tiles the work item reads:
//   XQ  q as two f16 pieces when the Cauchy-Schwarz bound on the item's
//       scores in log2 units, B = max |q| * max |k_t| * scale_log2, exceeds
//       32: f16 rounding moves each q element by at most 2^-11 of itself, so
//       a score by at most 2^-11 * B, which is 2^-6 at the threshold.
//   XP  P as two f16 pieces when the item's values have a crest factor
//       max |v| / rms(v) above 8: P's rounding error is weighted by
//       |v - out|, so outlier values carry it into the output.
// Keys of bf16 caches are exact in f16 (per-tile power-of-two scale), f16
// keys are the cache itself; P's rounding enters the output through V only.
template <int D, int NW, bool KSPLIT = false>
__device__ __forceinline__ void prefill_entry(const PrefillArgs& a) {
  constexpr int KS = D / 16;
  constexpr int BM = prefill_item_queries(NW, KSPLIT);
  constexpr int BN = prefill_block_n(D);
  constexpr int NT = 64 * NW;
  __shared__ float s_red[NW][5];
  __shared__ __attribute__((aligned(16))) char s_k0[PrefillLds<D>::KBYTES];
  __shared__ __attribute__((aligned(16))) char s_k1[PrefillLds<D>::KBYTES];
  __shared__ __attribute__((aligned(16))) char s_v0[PrefillLds<D>::VBYTES];
  __shared__ __attribute__((aligned(16))) char s_v1[PrefillLds<D>::VBYTES];
  // The key-split form's second tile per step (a 16-byte stand-in otherwise).
  __shared__ __attribute__((aligned(16))) char s_k2[KSPLIT ? PrefillLds<D>::KBYTES : 16];
  __shared__ __attribute__((aligned(16))) char s_k3[KSPLIT ? PrefillLds<D>::KBYTES : 16];
  __shared__ __attribute__((aligned(16))) char s_v2[KSPLIT ? PrefillLds<D>::VBYTES : 16];
  __shared__ __attribute__((aligned(16))) char s_v3[KSPLIT ? PrefillLds<D>::VBYTES : 16];
  PrefillLds<D> lds{(lchar*)s_k0, (lchar*)s_k1, (lchar*)s_v0, (lchar*)s_v1,
                    (lchar*)s_k2, (lchar*)s_k3, (lchar*)s_v2, (lchar*)s_v3};
  const int nblk = gridDim.y;
  int h, w;
  {
    // Workgroups are dispatched round-robin over the 8 XCDs in linear order.
    // When the heads split evenly, XCD x gets heads [x*hpx, (x+1)*hpx) --
    // with GQA these share KV heads, so each XCD's L2 holds fewer K/V tiles
    // -- and every XCD takes its longest (last) query blocks first.
    const int i = blockIdx.y * gridDim.x + blockIdx.x;
    int rank;  // position of the workgroup's query block in dispatch order
    if (a.n_heads % 8 == 0) {
      const int hpx = a.n_heads / 8, j = i / 8;
      h = (i % 8) * hpx + j % hpx;
      rank = j / hpx;
    } else {
      h = blockIdx.x;
      rank = blockIdx.y;
    }
    // Longest blocks first.  With kPrefillPairOrder (the whole grid is
    // resident at once, two workgroups per CU, nblk even) the second half
    // of the order runs the blocks in increasing length instead: rank r <
    // nblk/2 takes block nblk-1-r and rank r + nblk/2 block r, so when the
    // second round of workgroups fills the CUs in the first round's order,
    // every CU holds two blocks of nblk+1 blocks' keys in total.
    w = ((a.flags & kPrefillPairOrder) && rank >= nblk / 2) ? rank - nblk / 2 : nblk - 1 - rank;
  }
  // Work items.  Plain launches: block w, all its keys.  Balanced launches
  // (a.balance, nblk even): causal blocks b = p and c = nblk - 1 - p pair up
  // (their key counts sum to the same for every p) and the pair's keys are
  // cut in two equal halves at S: workgroup 2p takes block c's keys [0, S),
  // workgroup 2p + 1 the rest of block c and then all of block b.  Every
  // workgroup then has the same work, where the plain grid's longest block
  // has twice the average (a one-workgroup-per-CU grid waits for it).
  auto kend_of = [&](int q) -> long long {
    const int ml = ((q + 1) * BM < a.n_q ? (q + 1) * BM : a.n_q);
    return a.pos0 + ml;
  };
  int n_items = 1, qb0 = w, qb1 = 0, pc0 = -1;
  long long lo0 = 0, hi0 = 1LL << 62;
  if (kBalanced<D> && (a.flags & kPrefillBalance)) {
    const int p = w >> 1, c = nblk - 1 - p, b = p;
    const long long kc = kend_of(c), kb = kend_of(b);
    const long long S = (kb + kc) / 2 / BN * BN;
    if (S >= kc) {  // no split
      qb0 = (w & 1) ? b : c;
    } else if ((w & 1) == 0) {
      qb0 = c, pc0 = 0, hi0 = S;
    } else {
      qb0 = c, pc0 = 1, lo0 = S;
      qb1 = b, n_items = 2;
    }
  }
  const int kvh = (int)(((long long)h * a.n_kv) / a.n_heads);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hi = lane >> 5, lc = lane & 31;
  for (int it = 0; it < n_items; ++it) {
    const int qb = it == 0 ? qb0 : qb1;
    const int piece = it == 0 ? pc0 : -1;
    const long long k_lo = it == 0 ? lo0 : 0, k_hi = it == 0 ? hi0 : (1LL << 62);
    if (it > 0) __syncthreads();  // the previous item's LDS reads are done
    // The item's keys; the DMA of its first key tile into stage 0 goes out
    // before the q and statistics loads, so the three latencies overlap
    // (the body waits for the tile).
    long long kbeg, kend;
    item_keys<BM>(a, qb, k_lo, k_hi, kbeg, kend);
    int2 x_first = {0, 0};  // the first tile's (key, value) exponents
    {
      const long long kt_first = kbeg / BN * BN;
      if (kt_first < kend) {
        const TileSrc src = tile_src<D>(a, kvh);
        const TileDma<D, NW> dma(wave, lane, (int)src.krow_bytes, src.vrow_bytes);
        dma.issue_k(src.kbase, src.krow_bytes, kend, kt_first, lds.k0);
        dma.issue_v(src.vbase, src.vrow_bytes, kt_first, lds.v0);
        // Key-split: the first step's second tile too, and each wave's own
        // tile's exponents (none past the item's last key).
        if (KSPLIT && kt_first + BN < kend) {
          dma.issue_k(src.kbase, src.krow_bytes, kend, kt_first + BN, lds.k2);
          dma.issue_v(src.vbase, src.vrow_bytes, kt_first + BN, lds.v2);
        }
        const long long kx = kt_first + (KSPLIT ? (wave & 1) * BN : 0);
        if (a.texp && kx < kend)
          x_first = *reinterpret_cast<const int2*>(a.texp + ((long long)kvh * (a.vt_ld >> 6) + (kx >> 6)) * 2);
      }
    }
    const int mq = qb * BM + (KSPLIT ? wave >> 1 : wave) * 32 + lc;
    const int mr = mq < a.n_q ? mq : a.n_q - 1;  // padding lanes reuse the last query
    const float* qp = a.q + ((long long)mr * a.n_heads + h) * D + 8 * hi;
    // Q^T fragments (B operand): lane holds Q[mq][16ks + 8hi .. +8], read as
    // f32 and rounded to f16 after scaling by 2^-eq, eq from the largest |q|
    // of the wave's 32 (query, head) rows (wave-uniform); the score
    // multiplier takes 2^eq back.  A power-of-two scale is exact for every
    // value it keeps in f16's normal range.  The second piece lo = f16(x - hi)
    // makes 22 significant bits for the two-piece form.
    f16x8 qf[KS], ql[KS];
    int eq;
    float n2 = 0.0f;  // |q|^2 of the lane's half row
    f32x4 qv[KS][2];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      qv[ks][0] = *reinterpret_cast<const f32x4*>(qp + 16 * ks);
      qv[ks][1] = *reinterpret_cast<const f32x4*>(qp + 16 * ks + 4);
    }
    // The statistics of the item's key tiles (64-key pre-pass tiles; one
    // per thread, the rest, beyond 64 * NT keys, in a loop): largest
    // |k_t|^2, keys, largest |v|, sum of v^2.
    const float* ts = a.tstat + (long long)kvh * (a.vt_ld >> 6) * 8;
    const long long t_lo = kbeg >> 6, t_hi = (kend + 63) >> 6;
    f32x4 r0 = {0.0f, 0.0f, 0.0f, 0.0f}, r1 = {0.0f, 0.0f, 0.0f, 0.0f};
    if (t_lo + tid < t_hi) {
      r0 = *reinterpret_cast<const f32x4*>(ts + (t_lo + tid) * 8);
      r1 = *reinterpret_cast<const f32x4*>(ts + (t_lo + tid) * 8 + 4);
    }
    {
      float mx = 0.0f;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            mx = fmaxf(mx, fabsf(qv[ks][j][e]));
            n2 = fmaf(qv[ks][j][e], qv[ks][j][e], n2);
          }
      eq = __builtin_amdgcn_readfirstlane(scale_exp(wave_max(mx)));
      const float qscale = pow2f(-eq);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float x = qv[ks][j][e] * qscale;
            qf[ks][4 * j + e] = (_Float16)x;
            ql[ks][4 * j + e] = (_Float16)(x - (float)qf[ks][4 * j + e]);
          }
    }
    // |q|^2 of the lane's row (the lane pair hi = 0, 1 holds it), max over
    // the workgroup, with the tile statistics.
    float n2lo, n2hi;
    lane_halves(n2, n2lo, n2hi);
    const float wn2 = wave_max(n2lo + n2hi);
    float kn2 = r0[2], cnt = r0[3], vmx = r1[0], vss = r1[1];
    for (long long t = t_lo + tid + NT; t < t_hi; t += NT) {
      const f32x4 x0 = *reinterpret_cast<const f32x4*>(ts + t * 8);
      const f32x4 x1 = *reinterpret_cast<const f32x4*>(ts + t * 8 + 4);
      kn2 = fmaxf(kn2, x0[2]);
      cnt += x0[3];
      vmx = fmaxf(vmx, x1[0]);
      vss += x1[1];
    }
    kn2 = wave_max(kn2);
    vmx = wave_max(vmx);
    cnt = group_sum<64>(cnt);
    vss = group_sum<64>(vss);
    if (lane == 0) {
      s_red[wave][0] = wn2;
      s_red[wave][1] = kn2;
      s_red[wave][2] = vmx;
      s_red[wave][3] = vss;
      s_red[wave][4] = cnt;
    }
    __syncthreads();
    float qn2 = s_red[0][0];
    kn2 = s_red[0][1];
    vmx = s_red[0][2];
    vss = s_red[0][3];
    cnt = s_red[0][4];
#pragma unroll
    for (int ww = 1; ww < NW; ++ww) {
      qn2 = fmaxf(qn2, s_red[ww][0]);
      kn2 = fmaxf(kn2, s_red[ww][1]);
      vmx = fmaxf(vmx, s_red[ww][2]);
      vss += s_red[ww][3];
      cnt += s_red[ww][4];
    }
    const bool xq = sqrtf(qn2) * sqrtf(kn2) * a.scale_log2 > 32.0f;
    // crest^2 = max^2 * count / sum v^2 > 64, in f64 (no overflow for any f32).
    const bool xp = (double)vmx * vmx * ((double)cnt * D) > 64.0 * (double)vss;
    // Three compiled forms: both flags (also for xp alone, rare: values
    // with outliers), q alone, neither.  A fourth body inlined into the
    // kernel made the register allocator spill VGPRs in the d128 and d256
    // kernels.
    if (xp)
      prefill_body<D, NW, true, true, KSPLIT>(a, h, qb, kvh, qf, ql, eq, lds, k_lo, k_hi, piece, x_first);
    else if (xq)
      prefill_body<D, NW, true, false, KSPLIT>(a, h, qb, kvh, qf, ql, eq, lds, k_lo, k_hi, piece, x_first);
    else
      prefill_body<D, NW, false, false, KSPLIT>(a, h, qb, kvh, qf, ql, eq, lds, k_lo, k_hi, piece, x_first);
  }
}

}  // namespace vtb

// The attention kernels are the same for both cache dtypes (f16 operands);
// the pre-pass is per dtype.
#define VTB_PREFILL(D)                                                                     \
  extern "C" __global__ __launch_bounds__(256, vtb::prefill_waves_per_simd(D))             \
  void vtb_prefill_d##D(vtb::PrefillArgs a) {                                              \
    vtb::prefill_entry<D, 4>(a);                                                           \
  }
#define VTB_KVT(DTN, DTT, D)                                                               \
  extern "C" __global__ __launch_bounds__(256) void vtb_kvt_##DTN##_d##D(vtb::KvtArgs a) { \
    vtb::kvt_body<vtb::DTT, D>(a);                                                         \
  }

// Key-split small-prompt form (d <= 128): 64 queries per workgroup, two
// waves per 32 queries each taking every other key tile; one workgroup per
// CU (eight K / V^T stages, 140 KB of LDS at d128).
#define VTB_PREFILL_KS(D)                                                                  \
  extern "C" __global__ __launch_bounds__(256, 1) void vtb_prefill_ks_d##D(vtb::PrefillArgs a) { \
    vtb::prefill_entry<D, 4, true>(a);                                                     \
  }

VTB_PREFILL(64)
VTB_PREFILL(128)
VTB_PREFILL(256)
VTB_PREFILL_KS(64)
VTB_PREFILL_KS(128)
VTB_KVT(bf16, kv_bf16, 64)
VTB_KVT(bf16, kv_bf16, 128)
VTB_KVT(bf16, kv_bf16, 256)
VTB_KVT(f16, kv_f16, 64)
VTB_KVT(f16, kv_f16, 128)
VTB_KVT(f16, kv_f16, 256)
