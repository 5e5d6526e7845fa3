// Tile constants shared by the gfx950 kernels and the host launcher, so the
// host's split planning always matches what each compiled kernel assumes.
#pragma once

namespace vtb {

// Decode, scalar form (f32 caches, and GQA groups of 1 or 2): 16-byte loads
// per lane per wave tile (NIT), by GQA group width.  Tiles are
// double-buffered, so a wave keeps 2 x 2 x NIT loads in flight; NIT shrinks
// as the group widens to keep the q/acc registers resident.
#ifndef VTB_DECODE_NIT1
#define VTB_DECODE_NIT1 4
#endif
#ifndef VTB_DECODE_WAVES1
#define VTB_DECODE_WAVES1 4
#endif
#ifndef VTB_DECODE_NIT4
#define VTB_DECODE_NIT4 4
#endif
#ifndef VTB_DECODE_NIT8
#define VTB_DECODE_NIT8 2
#endif
constexpr int decode_nit(int g) {
  return g == 1 ? VTB_DECODE_NIT1 : g <= 4 ? VTB_DECODE_NIT4 : (g == 8 ? VTB_DECODE_NIT8 : 1);
}

// Decode, MFMA form: f16/bf16 caches with GQA groups of 4 or more compute
// the G query-key dot products of each 16-key block on
// v_mfma_f32_16x16x32_{bf16,f16} (queries as three exact pieces) and P.V on
// v_mfma_f32_16x16x16_{bf16,f16}, with K and V staged in LDS by DMA (two
// 16-key stages per wave).  Not for groups of 9-16 at head_dim 256: that
// body needs more than the 512 registers a wave can hold (the compiler
// spilled 600 of them to scratch), so those shapes take the scalar form.
constexpr bool decode_uses_mfma(int kv_bytes, int head_dim, int g) {
  return kv_bytes == 2 && g >= 4 && !(g >= 16 && head_dim >= 256);
}

// Waves per decode workgroup.  Scalar form: for g = 1 one wave per SIMD
// streams best: 16-wave workgroups keep 4x the loads in flight per CU and
// measured ~1.6 us slower per C2 launch at 8K context (deeper DRAM queues,
// 4x the waves to dispatch), with the same bytes moved.
#ifndef VTB_DECODE_WAVES4
#define VTB_DECODE_WAVES4 8
#endif
#ifndef VTB_DECODE_WAVES8
#define VTB_DECODE_WAVES8 8
#endif
// MFMA form: the K/V stages of every wave (64 * head_dim bytes each) fill
// about 128 KiB of LDS: 8 waves (two per SIMD) of two stages for head_dim
// <= 128, of one stage for 256 (decode_mfma_stages); groups of 16 halve the
// waves to leave room for their query pieces.
#ifndef VTB_DECODE_MFMA_WAVES
#define VTB_DECODE_MFMA_WAVES 8
#endif
#ifndef VTB_DECODE_MFMA_WAVES_D256
#define VTB_DECODE_MFMA_WAVES_D256 8
#endif
constexpr int decode_mfma_waves(int head_dim, int g) {
  return (head_dim >= 256 ? VTB_DECODE_MFMA_WAVES_D256 : VTB_DECODE_MFMA_WAVES) / (g >= 16 ? 2 : 1);
}
// LDS stages per wave of the MFMA form (2: block j+1's DMA in flight while
// block j is computed; 1: one block at a time, the SIMD's other wave
// overlapping).  head_dim 256: eight waves of one stage (two waves per SIMD,
// 150 KB of LDS) instead of four of two: C5 18.2-18.4 -> 16.8 us per layer
// (four waves of one stage: 17.5-17.7).
#ifndef VTB_DECODE_MFMA_STAGES_D256
#define VTB_DECODE_MFMA_STAGES_D256 1
#endif
constexpr int decode_mfma_stages(int head_dim) { return head_dim >= 256 ? VTB_DECODE_MFMA_STAGES_D256 : 2; }
constexpr int decode_waves(int kv_bytes, int head_dim, int g) {
  return decode_uses_mfma(kv_bytes, head_dim, g) ? decode_mfma_waves(head_dim, g)
         : g == 1                      ? VTB_DECODE_WAVES1
         : g <= 4                      ? VTB_DECODE_WAVES4
                                       : (g == 8 ? VTB_DECODE_WAVES8 : 4);
}

// Scalar form, uniform GQA maps with groups of 1 or 2: KV heads per
// workgroup (2 when two heads' rows fit one 64-lane load instruction).  At
// the C2 shape two heads per workgroup measured 26.0 us per launch against
// 26.2-26.4 for four (whose 32-way merge reads 4x the partials) and 27.1
// for one.
constexpr int decode_head_group(int kv_bytes, int head_dim) {
  return 64 / (head_dim * kv_bytes / 16) >= 2 ? 2 : 1;
}

// Split-K arrival counters sit one per 128 bytes, so the atomics of
// different (query, KV head) pairs never share a cache line.
constexpr int decode_counter_stride = 32;

// Split merge: up to decode_merge_flat(G * head_dim) active splits are
// merged by the last workgroup alone; beyond that, groups of
// decode_merge_group splits are merged by each group's last workgroup, then
// the group partials by the last group merger.  The flat limit keeps the
// last workgroup's reads near 64 KiB.
constexpr int decode_merge_flat(int partial_floats) { return partial_floats <= 512 ? 32 : 16; }
constexpr int decode_merge_group = 16;
// Kernels built with the XCD-local split merge (DecodeArgs::xcd_map): partials
// of up to 1024 floats.  The d256 kernels with groups of 8 or more (one wave
// per SIMD) needed stack for the second merge form.
constexpr bool kDecodeXclSlots(int partial_floats) { return partial_floats <= 1024; }
// Splits per (query, KV head) are capped so the group partials fit one
// merge: decode_merge_group groups of decode_merge_group splits.
constexpr int decode_max_splits = decode_merge_group * decode_merge_group;

// The decode code object's file-scope scratch (vtb_decode_scratch), used by
// the no-allocation decode entry: arrival counters in the first
// decode_scratch_counter_bytes, the split and group partials after them.
constexpr unsigned long long decode_scratch_bytes = 8ull << 20;
constexpr unsigned long long decode_scratch_counter_bytes = 256ull << 10;

// Rows per split are a multiple of this: the rows one wave load instruction
// covers (scalar form) or one 16-key MFMA block.
constexpr int decode_split_quantum(int head_dim, int kv_bytes, int g, int hg = 1) {
  return decode_uses_mfma(kv_bytes, head_dim, g) ? 16 : 64 / (head_dim * kv_bytes / 16 * hg);
}

// Prefill (MFMA): 4 waves x 32 queries per workgroup; keys per LDS tile by
// head_dim (the K and V^T tiles stay near 36 KiB of LDS).
constexpr int prefill_block_m(int) { return 128; }
// Queries per work item: 32 per wave, or in the key-split small-prompt form
// (two waves per 32 queries, each taking every other key tile) 64.
constexpr int prefill_item_queries(int nw, bool key_split) { return key_split ? 64 : 32 * nw; }
constexpr int prefill_block_n(int head_dim) { return head_dim <= 128 ? 64 : 32; }
// Minimum resident waves per SIMD the prefill kernel is compiled for: two
// waves let one wave's softmax and LDS waits hide behind the other's MFMAs
// (d <= 128 fits 256 registers without spilling; d256 needs more).
constexpr int prefill_waves_per_simd(int head_dim) { return head_dim <= 128 ? 2 : 1; }

}  // namespace vtb
