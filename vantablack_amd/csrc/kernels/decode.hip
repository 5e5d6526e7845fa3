// Split-K decode attention over the layer-major KV cache (gfx950).
//
// Replaces vantablack's three Metal kernels attn_scores / softmax_rows /
// attn_weighted_sum (src/metal/bridge.m:490-603) and computes exactly what
// forward.cpuAttention does (src/runtime/forward.zig:187-228):
//   out[h] = sum_t softmax_t(q[h].K[t,kv_h] / sqrt(D)) V[t,kv_h],
//   kv_h = (h*n_kv)/n_heads, t over [window_start, pos].
//
// Work decomposition (one launch per layer):
//   grid  = (n_splits, n_kv, n_q); block = NW waves.
//   A workgroup owns one (query b, KV head, row split) and each of its waves
//   a contiguous run of the split's rows.  Every K/V row is read from HBM once
//   and used for all q heads of the GQA group, so GQA reuse costs no extra
//   HBM traffic.  Two forms of the row loop:
//   - scalar (f32 caches; GQA groups of 1 or 2): a K (or V) row of D
//     elements is spread over LPR = D*bytes/16 lanes, one 16-byte load per
//     lane; scores are reduced across the LPR lanes with DPP adds and
//     permlane swaps (no LDS);
//   - MFMA (f16/bf16 caches, GQA groups of 4..16; 4..8 at head_dim 256):
//     K and V are staged in LDS by DMA (two 16-key stages per wave); the G
//     dot products of a 16-key block are v_mfma_f32_16x16x32_{bf16,f16}
//     products of the keys with the queries as three pieces of the cache's
//     16-bit type (q*2^-e = p0 + p1 + p2 exactly, one power of two e per
//     query), so every product is exact and sums are f32; P.V is
//     v_mfma_f32_16x16x16_{bf16,f16} with P as 16-bit pieces and V read from
//     LDS with the transposing ds_read_b64_tr_b16 (details at the MFMA form
//     below).
//   Scalar form: loads are double-buffered in registers (the next tile's
//   loads are issued before this tile's math).  The softmax is online
//   (running max m, sum l, accumulator) per wave.
//   The waves combine into one (m, l, o) partial per workgroup through
//   per-wave LDS slots summed in a fixed order.  The last-arriving
//   workgroup of each (query, KV head) merges the partials: it loads every
//   partial's (m, l) into LDS and its share of the o columns in one batch of
//   16-byte loads, scales each by 2^(m - M) for the common max M, sums the
//   lanes that share a column by DPP, and writes out[h] = o/l.  It resets
//   the arrival counter to zero, so no memset is needed between launches.
//   Partials travel through agent-coherent stores/loads and a relaxed
//   counter; no device-wide fence (L2 writeback/invalidate) is executed.
//   With the XCD-local map (DecodeArgs::xcd_map) every split of a unit runs
//   on one XCD and the partials stay in that XCD's L2 (sc0 stores and
//   loads).
//   A single query with more splits than one workgroup merges flat instead
//   publishes its partials only, and a second launch (vtb_decode_merge)
//   merges every column in parallel.
//
// Numerics: scores and P.V are f32 on exactly-upcast K/V (MFMA form: exact
// products of the query pieces and the 16-bit keys, f32 sums; P enters P.V
// as 16-bit pieces, exact for groups of 4 and 16 (bf16) or 22 (f16)
// significant bits for groups of 8-16).  The
// 1/sqrt(D) scale is folded with log2(e) into q once, and exp is evaluated
// as exp2.
//
// Multi-query form (n_q > 1): query b sits at absolute position pos0 + b and
// attends [window_start(pos0+b), pos0+b] -- the row loop of
// prefill.attentionCausal (src/runtime/prefill.zig:237-287).  The f32-cache
// prefill path uses it; decode is n_q = 1.
#include "common.h"
#include "../tiles.h"

namespace vtb {

// RoPE of element i of one head x[0..D) (math.rope / math.ropeHalf,
// src/kernels/math.zig:85-133): pair partner i^1 (interleaved) or i +- D/2
// (half form), angle pos * inv_freq[pair] (the f32 product the reference
// forms), strict f32 products.
template <int D>
__device__ inline float rope_elem(const float* x, int i, const float* inv_freq, float pos_f, bool half) {
#pragma clang fp contract(off)
  const int j = half ? (i % (D / 2)) : (i >> 1);
  float sn, cs;
  rope_sincos(pos_f * inv_freq[j], &sn, &cs);
  const bool first = half ? (i < D / 2) : ((i & 1) == 0);
  const int i0 = half ? j : (i & ~1);
  const int i1 = half ? j + D / 2 : (i | 1);
  const float x0 = x[i0], x1 = x[i1];
  return first ? x0 * cs - x1 * sn : x0 * sn + x1 * cs;
}

// Cache policy of the MFMA form's K/V tile DMA (buffer intrinsic aux bits:
// 2 = non-temporal; K/V rows are streamed once per launch).
#ifndef VTB_DECODE_DMA_AUX
#define VTB_DECODE_DMA_AUX 2
#endif
constexpr int kDecodeDmaAux = VTB_DECODE_DMA_AUX;

// Compile-time integer argument (DPP control) for lambdas.
template <int N> struct ic { static constexpr int value = N; };

// The (query, KV head, row split) a workgroup owns.
struct DecodeUnit {
  int b, kvh, split, h_lo, gs, n_act;
  long long r0, r1;
};

// False when this workgroup has no rows (its query needs fewer splits) or
// its KV head no query heads.  With HG > 1 the workgroup owns KV heads
// [HG*y, HG*y + HG) of a uniform GQA map (n_heads == n_kv * G): query slots
// j = i*G + g are heads h_lo + j.
template <int HG = 1, int G = 1>
__device__ inline bool decode_unit(const DecodeArgs& a, DecodeUnit& u) {
  u.split = blockIdx.x;
  u.kvh = blockIdx.y;
  u.b = blockIdx.z;
  if (a.xcd_map > 0) {
    // XCD-local merge (one query; units a multiple of nx, checked by the
    // host): workgroups i = nx * k + x of one XCD x serve whole units.
    const int nx = a.xcd_map;
    const int i = blockIdx.x + gridDim.x * blockIdx.y;
    const int x = i % nx, k = i / nx;
    u.kvh = x * ((int)gridDim.y / nx) + k / (int)gridDim.x;
    u.split = k % (int)gridDim.x;
  }
  const long long qpos = a.pos0 + u.b;
  const long long wstart = (a.window <= 0 || qpos < a.window) ? 0 : qpos - a.window + 1;
  const long long L = qpos + 1 - wstart;
  u.r0 = wstart + (long long)u.split * a.rows_per_split;
  u.r1 = (u.r0 + a.rows_per_split < qpos + 1) ? u.r0 + a.rows_per_split : qpos + 1;
  if (u.r0 >= u.r1) return false;
  u.n_act = (int)((L + a.rows_per_split - 1) / a.rows_per_split);
  if constexpr (HG > 1) {
    u.h_lo = u.kvh * HG * G;
    u.gs = HG * G;
    return true;
  }
  // GQA group of this KV head: h with (h*n_kv)/n_heads == kvh.
  u.h_lo = (u.kvh * a.n_heads + a.n_kv - 1) / a.n_kv;
  const int h_hi = ((u.kvh + 1) * a.n_heads + a.n_kv - 1) / a.n_kv;
  u.gs = h_hi - u.h_lo;
  return u.gs > 0;
}

// Fused KV-slot append (forward.zig:267-270): the workgroup whose rows
// include the new row pos0 writes this KV head's K and V slice of it,
// rounded to the cache dtype, before any of its waves reads it.  Only this
// workgroup reads that slice, and the stores complete (vmcnt 0) before the
// barrier, so the later loads from the same CU see them.
template <typename KV, int D, int NT, int HG = 1>
__device__ __forceinline__ void decode_append(const DecodeArgs& a, const DecodeUnit& u) {
  if (a.k_new != nullptr && a.pos0 >= u.r0 && a.pos0 < u.r1) {
    for (int t = threadIdx.x; t < HG * D; t += NT) {
      const long long kvh = (long long)u.kvh * HG + t / D;
      const int i = t % D;
      const long long off = a.pos0 * (long long)a.n_kv * D + kvh * D;
      const float* kn = a.k_new + kvh * D;
      const float kval = a.rope_inv_freq ? rope_elem<D>(kn, i, a.rope_inv_freq, (float)a.rope_pos, a.rope_half != 0)
                                         : kn[i];
      store_kv<KV>((void*)a.k, off + i, kval);
      store_kv<KV>((void*)a.v, off + i, a.v_new[kvh * D + i]);
    }
    wait_stores();
    __syncthreads();
  }
}

// Split-merge thread layout.  When the result has at least as many float4
// columns as the workgroup has threads (WIDE), thread t takes columns
// t, t + NT, ... of every slot: each load instruction reads 1 KB of one
// slot.  Otherwise the columns form blocks of 16; a wave takes one block,
// its four 16-lane quarters reading four different slots (256 bytes of one
// slot each), and with more waves than blocks the extra waves take further
// slots of the same block (WPB waves per block).  The segmented form costs
// more instructions per loaded byte, which the one-wave-per-SIMD d256
// kernels feel (C5: 2.9 us per launch), so it is used only where the wide
// form would leave threads idle.
template <int G, int D, int NT>
struct MergeShape {
  static constexpr int NW = NT / 64;
  static constexpr int MC = G * D / 4;                    // float4 columns
  static constexpr bool WIDE = MC >= NT;
  static constexpr int NBLK = MC / 16;                    // 16-column blocks
  static constexpr int WPB = WIDE || NBLK >= NW ? 1 : NW / NBLK;  // waves per block
  static constexpr int CPT = WIDE ? MC / NT : (NBLK >= NW ? NBLK / NW : 1);  // columns (blocks) per thread
  static constexpr int MP = WIDE ? 1 : 4 * WPB;          // threads per column
};

// Merge `count` (<= 32) partials [first, first + count) of one (query, KV
// head) unit into out = O / L, or into a group partial (dst_o, dst_ml).
// src_o: the unit's [slot][G][D]; src_ml: the unit's [slot][G][2].
//   Every thread loads its column of slots p, p + MP, ... (MergeShape) in
//   one batch of 16-byte loads; each lane quad reads one 64-byte line.
//   (With the slots spread over adjacent lanes instead, a C3-sized merge of
//   64 KB took 2.1 against 0.9 us: each quad touched four lines.)
//   Alongside, 32 lanes per query g load the slots' (m, l), one slot each,
//   and reduce them by DPP / permlane: M = max m, weights f = 2^(m - M) and
//   L = sum l f go to LDS.  After one barrier every thread weights its
//   slots, the quarters of a wave add by permlane, and the WPB waves of a
//   block through LDS, in a fixed order.  Slots past `count` load at an
//   offset past the buffer's range: zeros, no memory access, no branch.
//   Every sum has a fixed order, so results are bit-reproducible.
template <int G, int D, int NT, int MAXS, bool XL>
__device__ __forceinline__ void decode_merge(const DecodeArgs& a, const DecodeUnit& u, const float* src_o,
                                             const float* src_ml, long long first, int count, bool to_out,
                                             float* dst_o, float* dst_ml, float* sh_w, float* sh_ml,
                                             f32x4* sh_red) {
  using S = MergeShape<G, D, NT>;
  constexpr int C4 = D / 4;
  constexpr int MC = G * C4;
  constexpr int MP = S::MP, CPT = S::CPT;
  constexpr int SPL = (MAXS + MP - 1) / MP;  // slots per thread
  static_assert(MAXS <= 32 && MC % 16 == 0, "merge shape");
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int p = S::WIDE ? 0 : S::WPB > 1 ? ((w / S::NBLK) << 2) | (lane >> 4) : lane >> 4;
  const int blk0 = S::WPB > 1 ? w % S::NBLK : w;
  // Column of pass c.
  auto column = [&](int c) { return S::WIDE ? tid + c * NT : (blk0 + c * S::NW) * 16 + (lane & 15); };
  // count is uniform; saying so keeps the buffer resources in SGPRs (the
  // compiler otherwise wrapped every load of the d256 merge in a
  // readfirstlane loop).
  count = __builtin_amdgcn_readfirstlane(count);
  const unsigned bytes_o = (unsigned)count * G * D * 4;
  const auto ro = buffer_rsrc(src_o + first * G * D, bytes_o);
  const auto rm = buffer_rsrc(src_ml + first * G * 2, (unsigned)count * G * 8);
  f32x4 ov[CPT][SPL];
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int col = column(c);
#pragma unroll
    for (int i = 0; i < SPL; ++i) {
      const int s = p + MP * i;
      ov[c][i] = part_load_f4<XL>(ro, s < count ? (s * MC + col) * 16 : (int)bytes_o);
    }
  }
  // (m, l) of slot s of query g in lane s of half-wave g (loop only when
  // 32*G exceeds the workgroup).
  for (int t0 = 0; t0 < 32 * G; t0 += NT) {
    const int t = t0 + tid;
    const int g = t >> 5, s = t & 31;
    float m, l;
    part_load8<XL>(rm, (s < count ? s * G + g : count * G) * 8, m, l);
    m = s < count ? m : -INFINITY;
    const float M = group_max<32>(m);
    const float Ms = M == -INFINITY ? 0.0f : M;
    const float f = m == -INFINITY ? 0.0f : exp2_fast(m - Ms);
    const float L = group_sum<32>(l * f);
    if (t < 32 * G) {
      sh_w[g * 32 + s] = f;
      if (s == 0) {
        sh_ml[2 * g] = M;
        sh_ml[2 * g + 1] = L;
      }
    }
  }
  __syncthreads();
  f32x4 O[CPT];
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int col = column(c);
    const int g = col / C4;
    float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < SPL; ++i) {
      const float f = sh_w[g * 32 + ((p + MP * i) & 31)];  // slots past count weigh 0 and loaded 0
      o[0] = fmaf(ov[c][i].x, f, o[0]);
      o[1] = fmaf(ov[c][i].y, f, o[1]);
      o[2] = fmaf(ov[c][i].z, f, o[2]);
      o[3] = fmaf(ov[c][i].w, f, o[3]);
    }
    if constexpr (!S::WIDE) {
#pragma unroll
      for (int k = 0; k < 4; ++k) o[k] = stride_sum<16>(o[k]);
    }
    O[c] = f32x4{o[0], o[1], o[2], o[3]};
  }
  if constexpr (S::WPB > 1) {
    if (lane < 16) sh_red[(w / S::NBLK) * MC + blk0 * 16 + lane] = O[0];
    __syncthreads();
    if (w >= S::NBLK) return;
    f32x4 r = sh_red[blk0 * 16 + lane];
#pragma unroll
    for (int q = 1; q < S::WPB; ++q) r += sh_red[q * MC + blk0 * 16 + lane];
    O[0] = r;
  }
  if (!S::WIDE && lane >= 16) return;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int col = column(c);
    const int g = col / C4, d4 = col % C4;
    if (g >= u.gs) continue;
    const float M = sh_ml[2 * g], L = sh_ml[2 * g + 1];
    if (to_out) {
      float* op = a.out + ((long long)u.b * a.n_heads + u.h_lo + g) * D + d4 * 4;
      op[0] = O[c].x / L;
      op[1] = O[c].y / L;
      op[2] = O[c].z / L;
      op[3] = O[c].w / L;
    } else {
      const auto rw = buffer_rsrc(dst_o, G * D * 4);
      part_store_f4<XL>(rw, col * 16, O[c]);
      if (d4 == 0) {
        part_store<XL>(&dst_ml[g * 2 + 0], M);
        part_store<XL>(&dst_ml[g * 2 + 1], L);
      }
    }
  }
}

// After the row loop: every wave has parked its (m, l, o) for the G slots in
// LDS (sm, sl, so; a wave without rows has m = -inf).  The workgroup combines
// them in wave order into its partial (or, with one split, the output) and
// the last-arriving workgroup of each (query, KV head) merges the partials.
//   Up to decode_merge_flat(G*D) active splits the merge is flat.  Beyond
//   that splits form groups of decode_merge_group; the last workgroup of a
//   group merges the group's partials into a group partial, and the last
//   group merger merges the group partials.
//   Partials of a unit ub: o at ws_o[ub][split][G][D], (m, l) at
//   ws_ml[ub][split][G][2]; group partials likewise with n_groups slots.
//   A workgroup's (m, l) values stay in one piece: with one query's slots
//   adjacent instead ([G][split][2]), eight workgroups wrote 8-byte pieces
//   of each 64-byte line and C5 took 1.3 us longer.
template <int G, int D, int NW, int SOS = G * D>
__device__ __forceinline__ void decode_finish(const DecodeArgs& a, const DecodeUnit& u, const float (*sm)[G],
                                              const float (*sl)[G], const float* so) {
  constexpr int NT = NW * 64;
  constexpr int C4 = D / 4;
  constexpr int MC = G * C4;
  constexpr int FLAT = decode_merge_flat(G * D);
  constexpr int GS = decode_merge_group;
  constexpr int WPB = MergeShape<G, D, NT>::WPB;
  __shared__ float sh_w[32 * G];
  __shared__ float sh_ml[2 * G];
  __shared__ f32x4 sh_red[WPB > 1 ? WPB * MC : 1];
  __shared__ int s_last;
  const bool single = (u.n_act == 1);
  const bool xl = kDecodeXclSlots(G * D) && a.xcd_map > 0;  // XCD-local hand-off (wave-uniform)
  const long long units = gridDim.y;  // (query, KV head or head group) units per query
  const long long ub = (long long)u.b * units + u.kvh;
  const long long part = ub * a.n_splits + u.split;
  const int n_groups = (a.n_splits + GS - 1) / GS;  // group slots per (query, KV head)
  float* ml_unit = a.ws_ml + ub * a.n_splits * G * 2;
  const auto rw = buffer_rsrc(a.ws_o + part * G * D, G * D * 4);
  for (int c = threadIdx.x; c < MC; c += NT) {
    const int g = c / C4, d4 = c % C4;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, sm[w][g]);
    float L = 0.0f;
    f32x4 O = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      if (sm[w][g] == -INFINITY) continue;
      const float f = exp2_fast(sm[w][g] - M);
      L = fmaf(sl[w][g], f, L);
      const f32x4 ow = *reinterpret_cast<const f32x4*>(&so[w * SOS + g * D + d4 * 4]);
      O.x = fmaf(ow.x, f, O.x);
      O.y = fmaf(ow.y, f, O.y);
      O.z = fmaf(ow.z, f, O.z);
      O.w = fmaf(ow.w, f, O.w);
    }
    if (g >= u.gs) continue;
    if (single) {
      float* op = a.out + ((long long)u.b * a.n_heads + u.h_lo + g) * D + d4 * 4;
      op[0] = O.x / L;
      op[1] = O.y / L;
      op[2] = O.z / L;
      op[3] = O.w / L;
    } else {
      // Agent-scope (sc1) stores are coherent across the XCDs' L2s, so the
      // partials need no cache-wide writeback (a __threadfence() here costs
      // a full L2 writeback + invalidate per workgroup on this chip).  With
      // the XCD-local map the unit's merger shares this workgroup's L2, and
      // the partials stay in it (sc0).
      float* mlp = &ml_unit[((long long)u.split * G + g) * 2];
      if (xl) {
        part_store_f4<true>(rw, (g * D + d4 * 4) * 4, O);
        if (d4 == 0) {
          part_store<true>(mlp, M);
          part_store<true>(mlp + 1, L);
        }
      } else {
        part_store_f4<false>(rw, (g * D + d4 * 4) * 4, O);
        if (d4 == 0) {
          part_store<false>(mlp, M);
          part_store<false>(mlp + 1, L);
        }
      }
    }
  }
  if (single || a.merge_mode == kDecodeMergeLaunch) return;

  const bool two_level = u.n_act > FLAT;
  const int n_grp = two_level ? (u.n_act + GS - 1) / GS : 1;
  const int grp = two_level ? u.split / GS : 0;
  const int members = two_level ? ((u.n_act - grp * GS) < GS ? u.n_act - grp * GS : GS) : u.n_act;
  unsigned* ctr0 = a.counters + ub * (n_groups + 1) * decode_counter_stride;

  // Arrival: every thread's coherent stores complete before the workgroup
  // counts itself in.
  auto arrive = [&](unsigned* ctr, int expect) -> bool {
    wait_stores();
    __syncthreads();
    if (threadIdx.x == 0) {
      const unsigned prev = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int last = (prev == (unsigned)(expect - 1));
      if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = last;
    }
    __syncthreads();
    return s_last != 0;
  };

  if (!arrive(ctr0 + (long long)grp * decode_counter_stride, members)) return;
  const float* o_unit = a.ws_o + ub * a.n_splits * G * D;
  auto merge_all = [&](auto xl_tag) {
    constexpr bool XL = decltype(xl_tag)::value != 0;
    if (!two_level) {
      // Up to 16 splits the merge issues loads for 16 slots only (slots past
      // the count still pass through the load pipeline).
      if (FLAT > GS && u.n_act <= GS)
        decode_merge<G, D, NT, GS, XL>(a, u, o_unit, ml_unit, 0, u.n_act, true, nullptr, nullptr, sh_w, sh_ml,
                                       sh_red);
      else
        decode_merge<G, D, NT, FLAT, XL>(a, u, o_unit, ml_unit, 0, u.n_act, true, nullptr, nullptr, sh_w, sh_ml,
                                         sh_red);
      return;
    }
    float* go_unit = a.wg_o + ub * n_groups * G * D;
    float* gml_unit = a.wg_ml + ub * n_groups * G * 2;
    decode_merge<G, D, NT, GS, XL>(a, u, o_unit, ml_unit, (long long)grp * GS, members, false,
                                   go_unit + (long long)grp * G * D, gml_unit + (long long)grp * G * 2, sh_w, sh_ml,
                                   sh_red);
    if (!arrive(ctr0 + (long long)n_groups * decode_counter_stride, n_grp)) return;
    decode_merge<G, D, NT, GS, XL>(a, u, go_unit, gml_unit, 0, n_grp, true, nullptr, nullptr, sh_w, sh_ml, sh_red);
  };
  if constexpr (kDecodeXclSlots(G * D)) {
    if (xl) {
      merge_all(ic<1>{});
      return;
    }
  }
  merge_all(ic<0>{});
}

// ----------------------------------------------------------------- scalar form
// HG > 1: the workgroup owns HG adjacent KV heads (a uniform GQA map) and
// one load instruction covers row t of all of them, HG*D contiguous
// elements: lane l serves head (l / LPR) % HG.  With one head per workgroup
// the heads at 256-byte offsets 256 mod 1024 streamed about 15% slower than
// the others (C2 shape: 21.8 against 19.0 us), and the launch waited for
// them; with two heads per workgroup every workgroup mixes address classes.
template <typename KV, int D, int G, int NIT, int NW, int HG>
__device__ __forceinline__ void decode_scalar_body(const DecodeArgs& a) {
  constexpr int EPL = Unpack<KV>::N;           // elements per lane per load
  constexpr int LPR = D / EPL;                 // lanes per head row
  constexpr int LPH = LPR * HG;                // lanes per load-instruction row
  constexpr int RPW = 64 / LPH;                // rows per load instruction
  constexpr int TR = RPW * NIT;                // rows per wave tile
  constexpr int NT = NW * 64;
  constexpr int GS = HG * G;                   // query slots of the workgroup
  static_assert(LPH >= 1 && LPH <= 64 && (64 % LPH) == 0, "bad row split");

  __shared__ float s_m[NW][GS];
  __shared__ float s_l[NW][GS];
  __shared__ __attribute__((aligned(16))) float s_o[NW][GS][D];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  DecodeUnit u;
  if (!decode_unit<HG, G>(a, u)) return;
  const int b = u.b, h_lo = u.h_lo, gs = u.gs;
  const long long r0 = u.r0, r1 = u.r1;
  decode_append<KV, D, NT, HG>(a, u);

  const int col = lane % LPR;
  const int hh = (lane / LPR) % HG;            // head of the group this lane serves
  const int rsub = lane / LPH;
  const long long kvh = (long long)u.kvh * HG + hh;
  const int qh0 = HG > 1 ? h_lo + hh * G : h_lo;  // first query head of the lane's KV head
  const long long row_stride = (long long)a.n_kv * D;  // elements
  const char* kbase = (const char*)a.k + (kvh * D + col * EPL) * KV::bytes;
  const char* vbase = (const char*)a.v + (kvh * D + col * EPL) * KV::bytes;

  // This wave's contiguous rows [w0, w1): an equal share, rounded to RPW.
  const long long per_wave = ((r1 - r0 + NW - 1) / NW + RPW - 1) / RPW * RPW;
  const long long w0 = r0 + (long long)wave * per_wave;
  const long long w1 = (w0 + per_wave < r1) ? w0 + per_wave : r1;

  auto issue = [&](long long t0, u32x4 (&kr)[NIT], u32x4 (&vr)[NIT]) {
#pragma unroll
    for (int i = 0; i < NIT; ++i) {
      long long row = t0 + i * RPW + rsub;
      long long rc = row < w1 ? row : w1 - 1;  // clamp: never read past the range
      kr[i] = load16(kbase + rc * row_stride * KV::bytes);
    }
#pragma unroll
    for (int i = 0; i < NIT; ++i) {
      long long row = t0 + i * RPW + rsub;
      long long rc = row < w1 ? row : w1 - 1;
      vr[i] = load16(vbase + rc * row_stride * KV::bytes);
    }
  };
  // Slots past the group (gs < G) reload head h_lo and are zeroed through the
  // scale: every load is valid, so none is predicated.  A predicated load per
  // element compiled to one dependent memory round trip each (~5 us of a
  // 17 us GQA launch).
  // Without RoPE the query loads go out before the first tile's loads (a
  // wave's loads return in order, so the q wait excludes the tile).
  u32x4 ka[NIT], va[NIT], kb[NIT], vb[NIT];
  long long t0 = w0;
  float qv[G][EPL];
  if (a.rope_inv_freq == nullptr) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float* qp = a.q + ((long long)b * a.n_heads + qh0 + (g < gs ? g : 0)) * D + col * EPL;
#pragma unroll
      for (int e = 0; e < EPL; ++e) qv[g][e] = qp[e];
    }
    __builtin_amdgcn_sched_barrier(0);
    issue(t0, ka, va);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float sc = g < gs ? a.scale_log2 : 0.0f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) qv[g][e] *= sc;
    }
  } else {
    // Fused RoPE of q (wave-uniform branch).  The lane's EPL elements hold
    // whole interleaved pairs; in the half form their partners are the
    // same positions in the other half, loaded alongside.  The angles
    // depend only on the element index, so the G heads share them.
#pragma clang fp contract(off)
    const bool half = a.rope_half != 0;
    const bool lower = col * EPL < D / 2;
    const float pos_f = (float)a.rope_pos;
    float cs[EPL], sn[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const int i = col * EPL + e;
      if (half || (e & 1) == 0) {
        rope_sincos(pos_f * a.rope_inv_freq[half ? (i % (D / 2)) : (i >> 1)], &sn[e], &cs[e]);
      } else {  // the second element of an interleaved pair shares its angle
        sn[e] = sn[e - 1];
        cs[e] = cs[e - 1];
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float* qp = a.q + ((long long)b * a.n_heads + qh0 + (g < gs ? g : 0)) * D + col * EPL;
      const float* pp = qp + (lower ? D / 2 : -(D / 2));
      const float sc = g < gs ? a.scale_log2 : 0.0f;
      float x[EPL], y[EPL];
#pragma unroll
      for (int e = 0; e < EPL; ++e) x[e] = qp[e];
      if (half) {  // wave-uniform: only the half form reads the partner block
#pragma unroll
        for (int e = 0; e < EPL; ++e) y[e] = pp[e];
      } else {
#pragma unroll
        for (int e = 0; e < EPL; ++e) y[e] = 0.0f;
      }
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        float r;
        if (half)
          r = lower ? x[e] * cs[e] - y[e] * sn[e] : y[e] * sn[e] + x[e] * cs[e];
        else
          r = (e & 1) == 0 ? x[e] * cs[e] - x[e + 1] * sn[e] : x[e - 1] * sn[e] + x[e] * cs[e];
        qv[g][e] = r * sc;
      }
    }
    issue(t0, ka, va);
  }

  float m[G], l[G], acc[G][EPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[g][e] = 0.0f;
  }

  auto compute = [&](long long t0, const u32x4 (&kr)[NIT], const u32x4 (&vr)[NIT]) {
    float s[G][NIT];
#pragma unroll
    for (int i = 0; i < NIT; ++i) {
      float kf[EPL];
      Unpack<KV>::run(kr[i], kf);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float d = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) d = fmaf(qv[g][e], kf[e], d);
        s[g][i] = d;
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mt = -INFINITY;
#pragma unroll
      for (int i = 0; i < NIT; ++i) {
        float v = group_sum<LPR>(s[g][i]);
        v = (t0 + i * RPW + rsub < w1) ? v : -INFINITY;
        s[g][i] = v;
        mt = fmaxf(mt, v);
      }
      mt = stride_max<LPH>(mt);
      const float mn = fmaxf(m[g], mt);  // finite: row t0 is always in range
      const float corr = exp2_fast(m[g] - mn);
      m[g] = mn;
      float ls = 0.0f;
#pragma unroll
      for (int i = 0; i < NIT; ++i) {
        s[g][i] = exp2_fast(s[g][i] - mn);
        ls += s[g][i];
      }
      l[g] = l[g] * corr + ls;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[g][e] *= corr;
    }
#pragma unroll
    for (int i = 0; i < NIT; ++i) {
      float vf[EPL];
      Unpack<KV>::run(vr[i], vf);
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[g][e] = fmaf(s[g][i], vf[e], acc[g][e]);
    }
  };

  // Every issue is unconditional (rows past w1 clamp to row w1 - 1, a line
  // already in flight): with no load under a branch the compiler's wait
  // counts stay exact, so each tile waits only for its own loads.
  if (t0 < w1) {
    for (;;) {
      issue(t0 + TR, kb, vb);
      __builtin_amdgcn_sched_barrier(0);
      compute(t0, ka, va);
      t0 += TR;
      if (t0 >= w1) break;
      issue(t0 + TR, ka, va);
      __builtin_amdgcn_sched_barrier(0);
      compute(t0, kb, vb);
      t0 += TR;
      if (t0 >= w1) break;
    }
  }

  // Combine the row groups of the wave (lanes sharing head and `col`).
#pragma unroll
  for (int g = 0; g < G; ++g) {
    l[g] = stride_sum<LPH>(l[g]);
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[g][e] = stride_sum<LPH>(acc[g][e]);
  }
  // Each wave parks (m, l, acc) in its own LDS slot; the workgroup combine
  // then sums the waves in a fixed order, so results are bit-reproducible.
  // A wave with no rows has m = -inf and contributes nothing.
  if (rsub == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int e = 0; e < EPL; ++e) s_o[wave][hh * G + g][col * EPL + e] = acc[g][e];
      if (col == 0) {
        s_m[wave][hh * G + g] = m[g];
        s_l[wave][hh * G + g] = l[g];
      }
    }
  }
  __syncthreads();
  decode_finish<GS, D, NW>(a, u, s_m, s_l, &s_o[0][0][0]);
}

// ------------------------------------------------------------------ MFMA form
// f16/bf16 caches with GQA groups of 4, 8 or 16: both products of a 16-key
// block run on the matrix cores, with K and V staged in LDS by DMA.
//
// Staging.  Each wave streams its own contiguous rows, 16 keys per block,
// through two LDS stages of its own (K rows, then V rows, 2*D bytes each).
// A block is filled by buffer_load_dwordx4 ... lds (16 bytes per lane, the
// lanes' LDS writes contiguous in lane order); lane slots pick their source
// chunk so that chunk c of row r lands in slot c ^ f(r) of the row
// (f = kswz / vswz), which spreads the later 16-byte K reads and 8-byte V^T
// reads over all LDS banks.  Rows past the wave's range lie outside the
// block's buffer descriptor and read as zero (their scores are masked).
// Both stages' blocks are in flight while a block is computed.
//
// Scores.  v_mfma_f32_16x16x32_{bf16,f16}: A = Q' (rows 4q + p of a row
// group of four queries, p = 0..2 the three exact 16-bit pieces of query q
// scaled by 2^-e, p = 3 zero), B = K^T from LDS (lane l: key l % 16, 8
// contiguous head elements), D/32 instructions per row group.  Lane l gets
// query l/16's three piece products against key l % 16 and adds them.
//
// P.V.  v_mfma_f32_16x16x16_{bf16,f16}: A = P' (rows: SL slots per query,
// QPR queries per row group; the first NPC slots hold the exact 16-bit
// pieces of P, the rest zero), B = V (16 keys x 16 head columns), read from
// the row-major V stage with ds_read_b64_tr_b16, which hands lane l of each
// 16-lane group g column l % 16 of keys 4g .. 4g + 3.  P crosses from the
// score layout (one key, one query per lane) to the A layout through a
// 512-byte LDS tile per wave.  O accumulates in f32, D/16 instructions per
// row group.  With SL = 2 (groups of 8 or 16) P enters as two pieces, 16
// significant bits for bf16 (relative error <= 2^-17 per weight) and 22 for
// f16; with SL = 4 (groups of 4) as three, exact.  For f16 P is scaled by
// 2^7 first (P <= 2^8 stays inside f16's range; the scale leaves at the end).
//
// Softmax.  Online, with a lazy reference: a query's running max m is only
// raised when a block's max exceeds it by more than 8 (log2 units), so
// P <= 2^8 and most blocks skip the O rescale.  l sums the f32 P before
// rounding.  The rescale factors cross to the P.V layout through LDS.
template <typename KV> struct DecMfma;
template <> struct DecMfma<kv_bf16> {
  __device__ static inline f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
  __device__ static inline f32x4 mma16(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c,
                                                     0, 0, 0);
  }
  // x = piece + rest: piece the nearest bf16, rest exact in f32.
  __device__ static inline uint16_t piece(float x, float& rest) {
    const uint16_t h = f32_to_bf16_rne(x);
    rest = x - __builtin_bit_cast(float, (uint32_t)h << 16);
    return h;
  }
  // P enters unscaled: bf16 has f32's exponent range.
  static constexpr float kPScale = 1.0f;
};
template <> struct DecMfma<kv_f16> {
  __device__ static inline f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  }
  __device__ static inline f32x4 mma16(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0, 0,
                                                 0);
  }
  __device__ static inline uint16_t piece(float x, float& rest) {
    const _Float16 h = (_Float16)x;  // v_cvt_f16_f32: round to nearest even
    rest = x - (float)h;
    return __builtin_bit_cast(uint16_t, h);
  }
  // P <= 2^8 (lazy reference); times 2^7 stays below f16's largest finite
  // value, and weights down to 2^-21 stay normal.
  static constexpr float kPScale = 128.0f;
};

// Slot of chunk c of staged row r: c ^ kswz(r) for K, c ^ vswz(r) for V
// (C = D/8 chunks per row).  K is read 16 rows x one chunk per 16 lanes,
// V^T 4 rows x two chunks per 16 lanes; the XOR spreads both over the banks.
template <int D>
__device__ constexpr int kswz(int r) { return r % (D / 8); }
template <int D>
__device__ constexpr int vswz(int r) { return (2 * r) % (D / 8); }

typedef __attribute__((address_space(3))) char dchar;

template <typename KV, int D, int G, int NW>
__device__ __forceinline__ void decode_mfma_body(const DecodeArgs& a) {
  static_assert(G % 4 == 0, "MFMA decode takes GQA groups of 4, 8, 16");
  constexpr int NG = G / 4;            // score row groups (four queries each)
  constexpr int KM = D / 32;           // score MFMAs per 16-key block and row group
  constexpr int C = D / 8;             // 16-byte chunks per K or V row
  constexpr int RB = 2 * D;            // bytes per staged row
  constexpr int VOFF = 16 * RB;        // the V rows follow the K rows in a stage
  constexpr int SB = 2 * 16 * RB;      // bytes per wave per stage
  constexpr int NI = 16 * C / 64;      // DMA instructions per 16-row K (or V) block
  constexpr int QPR = G >= 8 ? 8 : 4;  // queries per P.V row group
  constexpr int SL = 16 / QPR;         // P' rows per query
  constexpr int NPC = SL < 3 ? SL : 3; // P pieces per query
  constexpr int NPG = G / QPR;         // P.V row groups
  constexpr int ND = D / 16;           // P.V MFMAs per row group (16-column blocks)
  constexpr int NT = NW * 64;
  constexpr int QLD = D + 8;           // Q' row stride in LDS (16-byte pad)
  constexpr bool QREG = NG * KM <= 8;  // Q' operands held in registers (else read per block)
  static_assert(NI * 64 == 16 * C && NI >= 1, "DMA block");
  static_assert((long long)G * D * 4 <= SB, "a wave's partial must fit its stage");

  __shared__ __attribute__((aligned(16))) char s_stg0[NW * SB];
  constexpr int NSTG = decode_mfma_stages(D);
  __shared__ __attribute__((aligned(16))) char s_stg1[NSTG > 1 ? NW * SB : 16];
  __shared__ float s_m[NW][G];
  __shared__ float s_l[NW][G];
  __shared__ __attribute__((aligned(16))) uint16_t s_q[4 * G][QLD];
  __shared__ float s_qe[G];
  __shared__ __attribute__((aligned(16))) uint16_t s_p[NW][NPG][16 * 16];
  __shared__ float s_cr[NW][G];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  DecodeUnit u;
  if (!decode_unit(a, u)) return;
  const int b = u.b, kvh = u.kvh, h_lo = u.h_lo, gs = u.gs;
  const long long r0 = u.r0, r1 = u.r1;
  decode_append<KV, D, NT>(a, u);

  const long long rs = (long long)a.n_kv * D * 2;  // row stride, bytes
  const char* kbase = (const char*)a.k + (long long)kvh * D * 2;
  const char* vbase = (const char*)a.v + (long long)kvh * D * 2;
  const int kcol = lane & 15, grp = lane >> 4;

  // This wave's contiguous rows [w0, w1): an equal share, rounded to 16.
  const long long per_wave = ((r1 - r0 + NW - 1) / NW + 15) / 16 * 16;
  const long long w0 = r0 + (long long)wave * per_wave;
  const long long w1 = (w0 + per_wave < r1) ? w0 + per_wave : r1;
  const int n_blk = w0 < w1 ? (int)((w1 - w0 + 15) / 16) : 0;

  // DMA source offsets of this lane inside a block (the same for every
  // block): slot s = 64 i + lane is chunk (s % C) ^ f(row) of row s / C.
  int koff[NI], voff[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int s = 64 * i + lane, r = s / C, cs = s % C;
    koff[i] = (int)(r * rs) + 16 * (cs ^ kswz<D>(r));
    voff[i] = (int)(r * rs) + 16 * (cs ^ vswz<D>(r));
  }
  dchar* const stg0 = (dchar*)s_stg0 + wave * SB;
  dchar* const stg1 = (dchar*)s_stg1 + (NSTG > 1 ? wave * SB : 0);
  // Block j (rows w0 + 16 j ...) of K and V into a stage.
  auto issue = [&](int j, dchar* st) {
    const long long t0 = w0 + 16LL * j;
    const long long nr = w1 - t0 < 16 ? w1 - t0 : 16;
    const auto rk = buffer_rsrc(kbase + t0 * rs, (unsigned)(nr * rs));
    const auto rv = buffer_rsrc(vbase + t0 * rs, (unsigned)(nr * rs));
#pragma unroll
    for (int i = 0; i < NI; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (__attribute__((address_space(3))) void*)(st + 1024 * i), 16,
                                               koff[i], 0, 0, kDecodeDmaAux);
#pragma unroll
    for (int i = 0; i < NI; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (__attribute__((address_space(3))) void*)(st + VOFF + 1024 * i),
                                               16, voff[i], 0, 0, kDecodeDmaAux);
  };

  // Stage Q' in LDS: wave w takes queries w, w + NW, ...; lane l holds
  // elements E*l .. +E-1.  Each query is scaled by the power of two 2^-e that
  // brings its largest |x| into [2^14, 2^15) (exact), then split into three
  // pieces of the cache's 16-bit type.  Slots past the group (gs < G) are
  // zero.  The query loads are issued before the first blocks' DMA: a wave's
  // loads return in order, so the staging waits only for them.
  constexpr int E = D / 64;
  constexpr int QPW = (G + NW - 1) / NW;  // queries staged per wave
  const bool rope = a.rope_inv_freq != nullptr;
  const bool rhalf = a.rope_half != 0;
  float qx0[QPW][E], qx1[QPW][E], qfr[QPW][E];
  // Every query load is unconditional (no branch between a load and its
  // wait): without RoPE the pair loads read the element itself and the
  // frequency load reads q.
#pragma unroll
  for (int j = 0; j < QPW; ++j) {
    const int g = wave + j * NW;
    const float* qp = a.q + ((long long)b * a.n_heads + h_lo + (g < gs ? g : 0)) * D;
    const float* fr = rope ? a.rope_inv_freq : qp;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int i = lane * E + e;
      const int jf = rhalf ? (i % (D / 2)) : (i >> 1);
      qx0[j][e] = qp[!rope ? i : rhalf ? jf : (i & ~1)];
      qx1[j][e] = qp[!rope ? i : rhalf ? jf + D / 2 : (i | 1)];
      qfr[j][e] = fr[jf];
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  if (n_blk > 0) issue(0, stg0);
  if (NSTG > 1 && n_blk > 1) issue(1, stg1);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < QPW; ++j) {
#pragma clang fp contract(off)
    const int g = wave + j * NW;
    float x[E];
    float mx = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int i = lane * E + e;
      float xv = qx0[j][e];
      if (rope) {  // rope_elem's arithmetic on the loaded pair
        float sn, cs;
        rope_sincos((float)a.rope_pos * qfr[j][e], &sn, &cs);
        const bool firstel = rhalf ? (i < D / 2) : ((i & 1) == 0);
        xv = firstel ? qx0[j][e] * cs - qx1[j][e] * sn : qx0[j][e] * sn + qx1[j][e] * cs;
      }
      x[e] = g < gs ? xv * a.scale_log2 : 0.0f;
      mx = fmaxf(mx, fabsf(x[e]));
    }
    const int ex = scale_exp(group_max<64>(mx));
    const float down = pow2f(-ex);
    if (g < G) {  // wave-uniform
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int i = lane * E + e;
        float r1v, r2v, r3v;
        s_q[4 * g + 0][i] = DecMfma<KV>::piece(x[e] * down, r1v);
        s_q[4 * g + 1][i] = DecMfma<KV>::piece(r1v, r2v);
        s_q[4 * g + 2][i] = DecMfma<KV>::piece(r2v, r3v);
        s_q[4 * g + 3][i] = 0;
      }
      if (lane == 0) s_qe[g] = pow2f(ex);
    }
  }
  // The P' tile's zero slots (rows NPC .. SL-1 of every query) stay zero.
  if constexpr (NPC < SL) {
    for (int i = lane; i < NPG * 16 * 16; i += 64) {
      const int row = (i >> 4) & 15;
      if (row % SL >= NPC) s_p[wave][i >> 8][i & 255] = 0;
    }
  }
  __syncthreads();
  auto qfrag = [&](int gi, int km) -> u32x4 {
    return *reinterpret_cast<const u32x4*>(&s_q[16 * gi + kcol][32 * km + 8 * grp]);
  };
  u32x4 qa[QREG ? NG : 1][QREG ? KM : 1];
  if constexpr (QREG) {
#pragma unroll
    for (int gi = 0; gi < NG; ++gi)
#pragma unroll
      for (int km = 0; km < KM; ++km) qa[gi][km] = qfrag(gi, km);
  }
  float qup[NG];
#pragma unroll
  for (int gi = 0; gi < NG; ++gi) qup[gi] = s_qe[4 * gi + grp];

  // Online softmax state.  Score layout: lanes of group grp in row group gi
  // hold query 4 gi + grp: its reference max m and their keys' share of its
  // sum.  P.V layout: lane l holds rows 4 grp .. +3 of every 16-column O
  // tile of each P.V row group.
  float m[NG], lsum[NG];
#pragma unroll
  for (int gi = 0; gi < NG; ++gi) {
    m[gi] = -INFINITY;
    lsum[gi] = 0.0f;
  }
  f32x4 o[NPG][ND];
#pragma unroll
  for (int pg = 0; pg < NPG; ++pg)
#pragma unroll
    for (int nd = 0; nd < ND; ++nd) o[pg][nd] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  uint16_t* const pt = &s_p[wave][0][0];
  float* const crw = &s_cr[wave][0];
  // V^T operand read of lane l = 16 g + 4 j + c: row 4 g + j, columns
  // n0 + 4 c .. + 3 (chunk n0/8 + c/2, half c % 2).
  const int vrow = 4 * grp + ((lane >> 2) & 3), vc = lane & 3;

  auto compute = [&](const dchar* st, int j) {
    const long long t0 = w0 + 16LL * j;
    // Scores of the 16 keys for every row group.
    u32x4 kb[KM];
#pragma unroll
    for (int km = 0; km < KM; ++km) {
      const int ch = grp + 4 * km;
      kb[km] = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
          st + kcol * RB + 16 * (ch ^ kswz<D>(kcol)));
    }
    float s[NG];
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
      f32x4 c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int km = 0; km < KM; ++km) c = DecMfma<KV>::mma(QREG ? qa[QREG ? gi : 0][QREG ? km : 0] : qfrag(gi, km),
                                                           kb[km], c);
      const float v = ((c.x + c.y) + c.z) * qup[gi];
      s[gi] = (t0 + kcol < w1) ? v : -INFINITY;
    }
    // Block max per query; raise the references that grew by more than 8.
    float mt[NG];
    bool grow = false;
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
      mt[gi] = group_max<16>(s[gi]);  // finite: key t0 is always in range
      grow = grow || mt[gi] > m[gi] + 8.0f;
    }
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {
#pragma unroll
      for (int gi = 0; gi < NG; ++gi) {
        const bool gg = mt[gi] > m[gi] + 8.0f;
        const float corr = gg ? exp2_fast(m[gi] - mt[gi]) : 1.0f;  // m = -inf: 0
        m[gi] = gg ? mt[gi] : m[gi];
        lsum[gi] *= corr;
        if (kcol == 0) crw[4 * gi + grp] = corr;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int pg = 0; pg < NPG; ++pg) {
        // Rows 4 grp + r of row group pg hold query pg*QPR + (4 grp + r) / SL.
        float cr[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) cr[r] = crw[pg * QPR + (4 * grp + r) / SL];
#pragma unroll
        for (int nd = 0; nd < ND; ++nd)
#pragma unroll
          for (int r = 0; r < 4; ++r) o[pg][nd][r] *= cr[r];
      }
    }
    // P of this lane's (query, key), its pieces into the P' tile at row
    // (q % QPR) * SL + piece, column = key.
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
      const float p = exp2_fast(s[gi] - m[gi]);
      lsum[gi] += p;
      const int q = 4 * gi + grp;
      uint16_t* prow = pt + (q / QPR) * 256 + ((q % QPR) * SL) * 16 + kcol;
      float rest = p * DecMfma<KV>::kPScale;
#pragma unroll
      for (int pp = 0; pp < NPC; ++pp) {
        float nxt;
        prow[16 * pp] = DecMfma<KV>::piece(rest, nxt);
        rest = nxt;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // O += P' V: A = P' rows (lane: row l % 16, keys 4 grp .. +3), B = V^T.
#pragma unroll
    for (int pg = 0; pg < NPG; ++pg) {
      const u32x2 pa = *reinterpret_cast<const u32x2*>(pt + pg * 256 + kcol * 16 + 4 * grp);
#pragma unroll
      for (int nd = 0; nd < ND; ++nd) {
        const int ch = 2 * nd + (vc >> 1);
        const dchar* vp = st + VOFF + vrow * RB + 16 * (ch ^ vswz<D>(vrow)) + 8 * (vc & 1);
        const s16x4 vt = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4*)(vp));
        o[pg][nd] = DecMfma<KV>::mma16(pa, __builtin_bit_cast(u32x2, vt), o[pg][nd]);
      }
    }
    // The next block's P' writes and DMA into this stage come after these
    // reads in the wave's program order; LDS operations of a wave complete
    // in order, and the DMA is issued after the wait below.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };

  // Two stages per wave (NSTG = 2): block j in stage j % 2, block j + 2
  // issued into it once block j has been computed.  vmcnt counts this wave's
  // DMA instructions (2 NI per block), so "block j has landed" is vmcnt <=
  // 2 NI while block j + 1 is in flight, else 0.  One stage (NSTG = 1): block
  // j + 1 is issued into the stage once block j has been computed.
  if constexpr (NSTG == 1) {
    for (int j = 0; j < n_blk; ++j) {
      wait_vmcnt<0>();
      compute(stg0, j);
      if (j + 1 < n_blk) {
        wait_lds();
        issue(j + 1, stg0);
      }
    }
  } else {
    for (int j = 0; j < n_blk; j += 2) {
      if (j + 1 < n_blk) wait_vmcnt<2 * NI>(); else wait_vmcnt<0>();
      compute(stg0, j);
      if (j + 2 < n_blk) {
        wait_lds();
        issue(j + 2, stg0);
      }
      if (j + 1 >= n_blk) break;
      if (j + 2 < n_blk) wait_vmcnt<2 * NI>(); else wait_vmcnt<0>();
      compute(stg1, j + 1);
      if (j + 3 < n_blk) {
        wait_lds();
        issue(j + 3, stg1);
      }
    }
  }

  // The wave's partial: l over the 16 lanes of each query's group; O over
  // each query's SL rows (the pieces), unscaled.  A wave without rows has
  // m = -inf and contributes nothing.
#pragma unroll
  for (int gi = 0; gi < NG; ++gi) lsum[gi] = group_sum<16>(lsum[gi]);
  if (kcol == 0) {
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
      s_m[wave][4 * gi + grp] = m[gi];
      s_l[wave][4 * gi + grp] = lsum[gi];
    }
  }
  // s_o[wave][G][D] takes the place of the wave's own first stage, whose
  // DMA has landed and whose reads are done.
  float* const so = (float*)(s_stg0 + wave * SB);
  constexpr float kUnscale = 1.0f / DecMfma<KV>::kPScale;
#pragma unroll
  for (int pg = 0; pg < NPG; ++pg)
#pragma unroll
    for (int nd = 0; nd < ND; ++nd) {
      const int col = 16 * nd + kcol;
      if constexpr (SL == 4) {
        so[(pg * QPR + grp) * D + col] = ((o[pg][nd][0] + o[pg][nd][1]) + o[pg][nd][2]) * kUnscale;
      } else {
        so[(pg * QPR + 2 * grp) * D + col] = (o[pg][nd][0] + o[pg][nd][1]) * kUnscale;
        so[(pg * QPR + 2 * grp + 1) * D + col] = (o[pg][nd][2] + o[pg][nd][3]) * kUnscale;
      }
    }
  __syncthreads();
  decode_finish<G, D, NW, SB / 4>(a, u, s_m, s_l, reinterpret_cast<const float*>(s_stg0));
}

template <typename KV, int D, int G, int HG = 1>
__device__ __forceinline__ void decode_body(const DecodeArgs& a) {
  if constexpr (decode_uses_mfma(KV::bytes, D, G))
    decode_mfma_body<KV, D, G, decode_waves(KV::bytes, D, G)>(a);
  else
    decode_scalar_body<KV, D, G, decode_nit(G), decode_waves(KV::bytes, D, G), HG>(a);
}

// The split merge as a launch of its own, after a decode launch whose
// workgroups only published their partials (kDecodeMergeLaunch: used when
// the in-kernel merge would take two levels, C5: 256 partials of 8 KiB,
// 21.4 -> 17.3 us per layer in a stamped probe; at one level a second
// launch costs what it saves).  Wave w of workgroup i merges float4 column
// 4 i + w of the concatenated unit results: lane l loads (m, l) and the
// column of partials l, l + 64, l + 128, l + 192 (past n_splits: zeros
// through the buffer range check), then M = max m, weights 2^(m - M),
// L = sum l 2^(m - M) and the weighted column sum reduce over the wave in
// a fixed order, and lane 0 writes O / L.
__device__ __forceinline__ void decode_merge_launch(const DecodeMergeArgs& a) {
  const int lane = threadIdx.x & 63;
  const int D = a.head_dim, C4 = D / 4, MC = a.slots * C4;
  const long long colg = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (colg >= (long long)a.n_units * MC) return;  // wave-uniform
  const int ub = (int)(colg / MC), col = (int)(colg % MC);
  const int g = col / C4, d4 = col % C4;
  const int b = ub / a.units, kvg = ub % a.units;
  int h_lo, gs;
  if (a.hg > 1) {
    h_lo = kvg * a.slots;
    gs = a.slots;
  } else {
    h_lo = (kvg * a.n_heads + a.n_kv - 1) / a.n_kv;
    gs = ((kvg + 1) * a.n_heads + a.n_kv - 1) / a.n_kv - h_lo;
  }
  if (g >= gs) return;  // wave-uniform: slots past a partial GQA group
  const int n = a.n_splits;
  const unsigned bytes_o = (unsigned)n * MC * 16, bytes_m = (unsigned)n * a.slots * 8;
  const auto ro = buffer_rsrc(a.ws_o + (long long)ub * n * a.slots * D, bytes_o);
  const auto rm = buffer_rsrc(a.ws_ml + (long long)ub * n * a.slots * 2, bytes_m);
  f32x4 ov[4];
  float mv[4], lv[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int s = lane + 64 * k;
    ov[k] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                          ro, s < n ? (s * MC + col) * 16 : (int)bytes_o, 0, 0));
    // Whole-vector bit-cast (a bit_cast of one ext-vector element reads
    // element 0 with this compiler).
    const f32x2 ml = __builtin_bit_cast(
        f32x2, __builtin_amdgcn_raw_buffer_load_b64(rm, s < n ? (s * a.slots + g) * 8 : (int)bytes_m, 0, 0));
    mv[k] = s < n ? ml.x : -INFINITY;
    lv[k] = ml.y;
  }
  float M = fmaxf(fmaxf(mv[0], mv[1]), fmaxf(mv[2], mv[3]));
  M = group_max<64>(M);
  const float Ms = M == -INFINITY ? 0.0f : M;
  float L = 0.0f;
  float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float f = mv[k] == -INFINITY ? 0.0f : exp2_fast(mv[k] - Ms);
    L = fmaf(lv[k], f, L);
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = fmaf(ov[k][e], f, o[e]);
  }
  L = group_sum<64>(L);
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = group_sum<64>(o[e]);
  if (lane == 0) {
    float* op = a.out + ((long long)b * a.n_heads + h_lo + g) * D + d4 * 4;
    op[0] = o[0] / L;
    op[1] = o[1] / L;
    op[2] = o[2] / L;
    op[3] = o[3] / L;
  }
}

}  // namespace vtb

extern "C" __global__ __launch_bounds__(256) void vtb_decode_merge(vtb::DecodeMergeArgs a) {
  vtb::decode_merge_launch(a);
}

// The XCD (XCC_ID bits 3:0) each workgroup runs on, for the host's check of
// the round-robin dealing of workgroups over XCDs that the XCD-local split
// merge relies on.
extern "C" __global__ __launch_bounds__(64) void vtb_xcc_probe(int* out) {
  int v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  if (threadIdx.x == 0) out[blockIdx.x] = v & 0xf;
}

// Split-K workspace of the no-allocation decode entry
// (vtb_hip_segment_attn_decode_append_noalloc): a fixed device array of this
// code object, zero at load, its address taken once by the host with
// hipModuleGetGlobal (the module-API counterpart of hipGetSymbolAddress; the
// kernels are loaded with hipModuleLoadData, so the name is exported with C
// linkage -- a definition in an extern "C" block -- rather than made static,
// and marked used so the linker keeps it).  Each context loads its own copy
// of the code object and so holds its own array.  The kernels reach it only through
// the pointers the host passes in DecodeArgs.
extern "C" {
__device__ __attribute__((aligned(256), used)) unsigned char vtb_decode_scratch[vtb::decode_scratch_bytes];
}

// Kernel entry points, one per (KV dtype, head_dim, max GQA group).  Looked
// up by name with hipModuleGetFunction: vtb_decode_<kv>_d<D>_g<G>.
#define VTB_DECODE(KVN, KVT, D, G)                                                         \
  extern "C" __global__ __launch_bounds__(vtb::decode_waves(vtb::KVT::bytes, D, G) * 64) void \
      vtb_decode_##KVN##_d##D##_g##G(vtb::DecodeArgs a) {                                 \
    vtb::decode_body<vtb::KVT, D, G>(a);                                                  \
  }

#define VTB_DECODE_G(KVN, KVT, D) \
  VTB_DECODE(KVN, KVT, D, 1)      \
  VTB_DECODE(KVN, KVT, D, 2)      \
  VTB_DECODE(KVN, KVT, D, 4)      \
  VTB_DECODE(KVN, KVT, D, 8)      \
  VTB_DECODE(KVN, KVT, D, 16)

#define VTB_DECODE_D(KVN, KVT) \
  VTB_DECODE_G(KVN, KVT, 64)   \
  VTB_DECODE_G(KVN, KVT, 128)  \
  VTB_DECODE_G(KVN, KVT, 256)

VTB_DECODE_D(f32, kv_f32)
VTB_DECODE_D(f16, kv_f16)
VTB_DECODE_D(bf16, kv_bf16)

// Head-group entry points (uniform GQA maps with groups of 1 or 2 and
// n_kv a multiple of the group): vtb_decodeh_<kv>_d<D>_g<G>, HG =
// decode_head_group(kv bytes, D) KV heads per workgroup.
#define VTB_DECODEH(KVN, KVT, D, G)                                                        \
  extern "C" __global__ __launch_bounds__(vtb::decode_waves(vtb::KVT::bytes, D, G) * 64) void \
      vtb_decodeh_##KVN##_d##D##_g##G(vtb::DecodeArgs a) {                                \
    vtb::decode_body<vtb::KVT, D, G, vtb::decode_head_group(vtb::KVT::bytes, D)>(a);      \
  }
#define VTB_DECODEH_D(KVN, KVT) \
  VTB_DECODEH(KVN, KVT, 64, 1)  \
  VTB_DECODEH(KVN, KVT, 64, 2)  \
  VTB_DECODEH(KVN, KVT, 128, 1) \
  VTB_DECODEH(KVN, KVT, 128, 2) \
  VTB_DECODEH(KVN, KVT, 256, 1) \
  VTB_DECODEH(KVN, KVT, 256, 2)
VTB_DECODEH_D(f32, kv_f32)
VTB_DECODEH_D(f16, kv_f16)
VTB_DECODEH_D(bf16, kv_bf16)
