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
//   HBM traffic.
//   Inside a wave, a K (or V) row of D elements is spread over LPR = D*bytes/16
//   lanes, one 16-byte load per lane; RPW = 64/LPR rows are read per load
//   instruction, NIT instructions per tile.  Tiles are double-buffered in
//   registers: the next tile's loads are issued before this tile's math.
//   Scores are reduced across the LPR lanes with DPP adds and the rows of a
//   load instruction combined with DPP / permlane swaps (no LDS); the softmax
//   is online (running max m, sum l, accumulator acc) per wave, in registers.
//   The waves combine into one (m, l, o) partial per workgroup through
//   per-wave LDS slots summed in a fixed order.  The last-arriving
//   workgroup of each (query, KV head) merges the partials (log-sum-exp):
//   the lanes of each float4 column of the result share the partials, load
//   theirs in one batch of 16-byte buffer loads and combine by a DPP
//   butterfly, then write out[h] = o/l.  It resets the arrival counter to
//   zero, so no memset is needed between launches.
//   Partials travel through agent-coherent stores/loads and a relaxed
//   counter; no device-wide fence (L2 writeback/invalidate) is executed.
//
// Numerics: all arithmetic is f32 on exactly-upcast K/V.  The 1/sqrt(D)
// scale is folded with log2(e) into q once, and exp is evaluated as exp2.
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

// Compile-time integer argument (merge batch size, DPP control) for lambdas.
template <int N> struct merge_batch { static constexpr int value = N; };

template <typename KV, int D, int G, int NIT, int NW>
__device__ __forceinline__ void decode_body(const DecodeArgs& a) {
  constexpr int EPL = Unpack<KV>::N;           // elements per lane per load
  constexpr int LPR = D / EPL;                 // lanes per row
  constexpr int RPW = 64 / LPR;                // rows per load instruction
  constexpr int TR = RPW * NIT;                // rows per wave tile
  constexpr int NT = NW * 64;                  // threads per workgroup
  static_assert(LPR >= 1 && LPR <= 64 && (64 % LPR) == 0, "bad row split");

  __shared__ float s_m[NW][G];
  __shared__ float s_l[NW][G];
  __shared__ float s_o[NW][G][D];
  __shared__ int s_last;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int split = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;

  const long long qpos = a.pos0 + b;
  const long long wstart = (a.window <= 0 || qpos < a.window) ? 0 : qpos - a.window + 1;
  const long long L = qpos + 1 - wstart;
  const long long r0 = wstart + (long long)split * a.rows_per_split;
  const long long r1 = (r0 + a.rows_per_split < qpos + 1) ? r0 + a.rows_per_split : qpos + 1;
  if (r0 >= r1) return;  // this query needs fewer splits; not counted below
  const int n_act = (int)((L + a.rows_per_split - 1) / a.rows_per_split);

  // GQA group of this KV head: h with (h*n_kv)/n_heads == kvh.
  const int h_lo = (kvh * a.n_heads + a.n_kv - 1) / a.n_kv;
  const int h_hi = ((kvh + 1) * a.n_heads + a.n_kv - 1) / a.n_kv;
  const int gs = h_hi - h_lo;
  if (gs <= 0) return;


  // Fused KV-slot append (forward.zig:267-270): the workgroup whose rows
  // include the new row pos0 writes this KV head's K and V slice of it,
  // rounded to the cache dtype, before any of its waves reads it.  Only this
  // workgroup reads that slice, and the stores complete (vmcnt 0) before the
  // barrier, so the later loads from the same CU see them.
  if (a.k_new != nullptr && a.pos0 >= r0 && a.pos0 < r1) {
    const long long off = a.pos0 * (long long)a.n_kv * D + (long long)kvh * D;
    const float* kn = a.k_new + (long long)kvh * D;
    for (int i = threadIdx.x; i < D; i += NT) {
      const float kval = a.rope_inv_freq ? rope_elem<D>(kn, i, a.rope_inv_freq, (float)a.rope_pos, a.rope_half != 0)
                                         : kn[i];
      store_kv<KV>((void*)a.k, off + i, kval);
      store_kv<KV>((void*)a.v, off + i, a.v_new[(long long)kvh * D + i]);
    }
    wait_stores();
    __syncthreads();
  }

  const int col = lane % LPR;
  const int rsub = lane / LPR;
  const long long row_stride = (long long)a.n_kv * D;  // elements
  const char* kbase = (const char*)a.k + ((long long)kvh * D + col * EPL) * KV::bytes;
  const char* vbase = (const char*)a.v + ((long long)kvh * D + col * EPL) * KV::bytes;

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
  float qv[G][EPL];
  if (a.rope_inv_freq == nullptr) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float* qp = a.q + ((long long)b * a.n_heads + h_lo + (g < gs ? g : 0)) * D + col * EPL;
      const float sc = g < gs ? a.scale_log2 : 0.0f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) qv[g][e] = qp[e] * sc;
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
      const float* qp = a.q + ((long long)b * a.n_heads + h_lo + (g < gs ? g : 0)) * D + col * EPL;
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
      mt = stride_max<LPR>(mt);
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

  u32x4 ka[NIT], va[NIT], kb[NIT], vb[NIT];
  long long t0 = w0;
  if (t0 < w1) issue(t0, ka, va);
  while (t0 < w1) {
    if (t0 + TR < w1) issue(t0 + TR, kb, vb);
    __builtin_amdgcn_sched_barrier(0);
    compute(t0, ka, va);
    t0 += TR;
    if (t0 >= w1) break;
    if (t0 + TR < w1) issue(t0 + TR, ka, va);
    __builtin_amdgcn_sched_barrier(0);
    compute(t0, kb, vb);
    t0 += TR;
  }

  // Combine the row groups of the wave (lanes sharing `col`).
#pragma unroll
  for (int g = 0; g < G; ++g) {
    l[g] = stride_sum<LPR>(l[g]);
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[g][e] = stride_sum<LPR>(acc[g][e]);
  }
  // Each wave parks (m, l, acc) in its own LDS slot; the workgroup combine
  // then sums the waves in a fixed order, so results are bit-reproducible.
  // A wave with no rows has m = -inf and contributes nothing.
  if (rsub == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int e = 0; e < EPL; ++e) s_o[wave][g][col * EPL + e] = acc[g][e];
      if (col == 0) {
        s_m[wave][g] = m[g];
        s_l[wave][g] = l[g];
      }
    }
  }
  __syncthreads();

  const bool single = (n_act == 1);
  const long long part = ((long long)b * a.n_kv + kvh) * a.n_splits + split;
  for (int idx = threadIdx.x; idx < G * D; idx += NT) {
    const int g = idx / D, d = idx % D;
    if (g >= gs) continue;
    float Mg = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) Mg = fmaxf(Mg, s_m[w][g]);
    float Lg = 0.0f, Og = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      if (s_m[w][g] == -INFINITY) continue;
      const float f = exp2_fast(s_m[w][g] - Mg);
      Lg += s_l[w][g] * f;
      Og += s_o[w][g][d] * f;
    }
    if (single) {
      a.out[((long long)b * a.n_heads + h_lo + g) * D + d] = Og / Lg;
    } else {
      // Agent-scope atomic stores are coherent across the XCDs' L2s, so the
      // partials need no cache-wide writeback (a __threadfence() here costs
      // a full L2 writeback + invalidate per workgroup on this chip).
      store_coherent(&a.ws_o[(part * G + g) * D + d], Og);
      if (d == 0) {
        store_coherent(&a.ws_ml[(part * G + g) * 2 + 0], Mg);
        store_coherent(&a.ws_ml[(part * G + g) * 2 + 1], Lg);
      }
    }
  }
  if (single) return;

  // Merge.  Up to decode_merge_flat active splits, the last workgroup to
  // arrive merges them all (batches of 8 independent loads, as many rounds
  // as batches).  Beyond that the merge has two levels: splits form groups
  // of decode_merge_group; the last workgroup of a group merges the group's
  // partials in one batch into a group partial, and the last group merger
  // merges the group partials.  A flat merge of a long MQA cache (C5: 256
  // splits of one KV head) was ~100 us of dependent load rounds through one
  // workgroup; the extra level costs ~1 us, so short split lists stay flat.
  constexpr int GS = decode_merge_group;
  const bool two_level = n_act > decode_merge_flat;
  const int n_groups = (a.n_splits + GS - 1) / GS;  // group slots per (query, KV head)
  const int n_grp = two_level ? (n_act + GS - 1) / GS : 1;
  const int grp = two_level ? split / GS : 0;
  const int members = two_level ? ((n_act - grp * GS) < GS ? n_act - grp * GS : GS) : n_act;
  unsigned* ctr0 = a.counters + ((long long)b * a.n_kv + kvh) * (n_groups + 1) * decode_counter_stride;

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
  // Merge `count` partials src[first .. first+count) of this (query, KV
  // head) -- [slot][G][D] values, [slot][G][2] (m, l) -- into out = O / L,
  // or into slot dst of the group partials.  A partial is MC float4 columns;
  // MP adjacent lanes share a column and lane p takes slots p, p + MP, ...:
  // MB slots per lane per batch, all loads of a batch in flight together,
  // then a log-sum-exp butterfly over the MP lanes (DPP, within a row).
  // Slots past `count`, and lanes without a live column, load at an offset
  // past the buffer's range: zeros, no memory access, no branch.
  constexpr int MC = G * D / 4;
  constexpr int MP = NT >= 16 * MC ? 16 : (NT >= MC ? NT / MC : 1);
  constexpr int MCP = NT / MP;  // columns per pass
  auto merge = [&](auto batch, const float* src_o, const float* src_ml, long long first, int count, bool to_out,
                   long long dst) {
    constexpr int MB = decltype(batch)::value;
    const int p = threadIdx.x % MP;
    const auto ro = buffer_rsrc(src_o + first * G * D, (unsigned)count * G * D * 4);
    const auto rm = buffer_rsrc(src_ml + first * G * 2, (unsigned)count * G * 8);
    for (int c0 = 0; c0 < MC; c0 += MCP) {
      const int c = c0 + (int)threadIdx.x / MP;
      const int g = c / (D / 4), d4 = c % (D / 4);
      const bool live = c < MC && g < gs;
      float M = -INFINITY, L = 0.0f, O[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int f0 = 0; f0 < count; f0 += MP * MB) {
        float ov[MB][4], mv[MB], lv[MB];
#pragma unroll
        for (int i = 0; i < MB; ++i) {
          const int sl = f0 + p + MP * i;
          const int se = (live && sl < count) ? sl : count;
          buffer_load16_coherent(ro, ((se * G + g) * D + d4 * 4) * 4, ov[i][0], ov[i][1], ov[i][2], ov[i][3]);
          buffer_load8_coherent(rm, (se * G + g) * 8, mv[i], lv[i]);
        }
        float Mb = M;
#pragma unroll
        for (int i = 0; i < MB; ++i) {
          const bool ok = live && f0 + p + MP * i < count;
          mv[i] = ok ? mv[i] : -INFINITY;
          Mb = fmaxf(Mb, mv[i]);
        }
        // Branch-free (a branch here lets the compiler split the loads and
        // sink the parts used under it, a second round trip): with nothing
        // attended yet Mb stays -inf and every factor is 0.
        const float Ms = Mb == -INFINITY ? 0.0f : Mb;
        const float cm = M == -INFINITY ? 0.0f : exp2_fast(M - Ms);
        L *= cm;
#pragma unroll
        for (int k = 0; k < 4; ++k) O[k] *= cm;
#pragma unroll
        for (int i = 0; i < MB; ++i) {
          const float f = mv[i] == -INFINITY ? 0.0f : exp2_fast(mv[i] - Ms);
          L = fmaf(lv[i], f, L);
#pragma unroll
          for (int k = 0; k < 4; ++k) O[k] = fmaf(ov[i][k], f, O[k]);
        }
        M = Mb;
      }
      // Butterfly over the MP lanes of the column (every lane active).
      auto fold = [&](auto ctrl) {
        constexpr int CTRL = decltype(ctrl)::value;
        const float Mo = dpp<CTRL>(M), Lo = dpp<CTRL>(L);
        float Oo[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) Oo[k] = dpp<CTRL>(O[k]);
        const float Mn = fmaxf(M, Mo);
        const float fa = M == -INFINITY ? 0.0f : exp2_fast(M - Mn);
        const float fb = Mo == -INFINITY ? 0.0f : exp2_fast(Mo - Mn);
        L = L * fa + Lo * fb;
#pragma unroll
        for (int k = 0; k < 4; ++k) O[k] = O[k] * fa + Oo[k] * fb;
        M = Mn;
      };
      if constexpr (MP >= 2) fold(merge_batch<DPP_XOR1>{});
      if constexpr (MP >= 4) fold(merge_batch<DPP_XOR2>{});
      if constexpr (MP >= 8) fold(merge_batch<DPP_HALF_MIRROR>{});
      if constexpr (MP >= 16) fold(merge_batch<DPP_MIRROR>{});
      if (live && p == 0) {
        if (to_out) {
          float* op = a.out + ((long long)b * a.n_heads + h_lo + g) * D + d4 * 4;
#pragma unroll
          for (int k = 0; k < 4; ++k) op[k] = O[k] / L;
        } else {
          float* op = a.wg_o + (dst * G + g) * D + d4 * 4;
#pragma unroll
          for (int k = 0; k < 4; ++k) store_coherent(op + k, O[k]);
          store_coherent(&a.wg_ml[(dst * G + g) * 2 + 0], M);
          store_coherent(&a.wg_ml[(dst * G + g) * 2 + 1], L);
        }
      }
    }
  };

  if (!arrive(ctr0 + (long long)grp * decode_counter_stride, members)) return;
  const long long part0 = ((long long)b * a.n_kv + kvh) * a.n_splits;
  if (!two_level) {
    // One slot per lane when the splits fit the column's lanes (C2's 8
    // splits over 8 lanes); a batch of up to 16 slots per lane otherwise.
    constexpr int MBF = (decode_merge_flat + MP - 1) / MP < 16 ? (decode_merge_flat + MP - 1) / MP : 16;
    if (MBF > 1 && n_act <= MP)
      merge(merge_batch<1>{}, a.ws_o, a.ws_ml, part0, n_act, true, 0);
    else
      merge(merge_batch<MBF>{}, a.ws_o, a.ws_ml, part0, n_act, true, 0);
    return;
  }
  const long long gpart0 = ((long long)b * a.n_kv + kvh) * n_groups;
  constexpr int MBG = (GS + MP - 1) / MP;
  merge(merge_batch<MBG>{}, a.ws_o, a.ws_ml, part0 + (long long)grp * GS, members, false, gpart0 + grp);
  if (!arrive(ctr0 + (long long)n_groups * decode_counter_stride, n_grp)) return;
  merge(merge_batch<MBG>{}, a.wg_o, a.wg_ml, gpart0, n_grp, true, 0);
}

}  // namespace vtb

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
#define VTB_DECODE(KVN, KVT, D, G)                                                     \
  extern "C" __global__ __launch_bounds__(vtb::decode_waves(G) * 64) void             \
      vtb_decode_##KVN##_d##D##_g##G(vtb::DecodeArgs a) {                             \
    vtb::decode_body<vtb::KVT, D, G, vtb::decode_nit(G), vtb::decode_waves(G)>(a);    \
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
