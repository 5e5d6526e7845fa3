// Tile constants shared by the gfx950 kernels and the host launcher, so the
// host's split planning always matches what each compiled kernel assumes.
#pragma once

namespace vtb {

// Decode: 16-byte loads per lane per wave tile (NIT), by GQA group width.
// Tiles are double-buffered, so a wave keeps 2 x 2 x NIT loads in flight;
// NIT shrinks as the group widens to keep the q/acc registers resident.
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

// Waves per decode workgroup.  For g = 1 one wave per SIMD streams best:
// 16-wave workgroups keep 4x the loads in flight per CU and measured ~1.6 us
// slower per C2 launch at 8K context (deeper DRAM queues, 4x the waves to
// dispatch), with the same bytes moved.
#ifndef VTB_DECODE_WAVES4
#define VTB_DECODE_WAVES4 8
#endif
#ifndef VTB_DECODE_WAVES8
#define VTB_DECODE_WAVES8 8
#endif
constexpr int decode_waves(int g) {
  return g == 1 ? VTB_DECODE_WAVES1 : g <= 4 ? VTB_DECODE_WAVES4 : (g == 8 ? VTB_DECODE_WAVES8 : 4);
}

// Split-K arrival counters sit one per 128 bytes, so the atomics of
// different (query, KV head) pairs never share a cache line.
constexpr int decode_counter_stride = 32;

// Split merge: up to decode_merge_flat active splits are merged by the
// last workgroup alone; beyond that, groups of decode_merge_group splits are
// merged by each group's last workgroup in one batch of loads, then the
// group partials by the last group merger.
constexpr int decode_merge_flat = 32;
constexpr int decode_merge_group = 16;

// The decode code object's file-scope scratch (vtb_decode_scratch), used by
// the no-allocation decode entry: arrival counters in the first
// decode_scratch_counter_bytes, the split and group partials after them.
constexpr unsigned long long decode_scratch_bytes = 8ull << 20;
constexpr unsigned long long decode_scratch_counter_bytes = 256ull << 10;

// Rows read by one wave load instruction (the split granularity).
constexpr int decode_rows_per_load(int head_dim, int kv_bytes) {
  return 64 / (head_dim * kv_bytes / 16);
}

// Prefill (MFMA): 4 waves x 32 queries per workgroup; keys per LDS tile by
// head_dim (the K and V^T tiles stay near 36 KiB of LDS).
constexpr int prefill_block_m(int) { return 128; }
// Queries per workgroup of the wide (8-wave, d <= 128) prefill kernels.
constexpr int prefill_block_m_wide = 256;
constexpr int prefill_block_n(int head_dim) { return head_dim <= 128 ? 64 : 32; }
// Minimum resident waves per SIMD the prefill kernel is compiled for: two
// waves let one wave's softmax and LDS waits hide behind the other's MFMAs
// (d <= 128 fits 256 registers without spilling; d256 needs more).
constexpr int prefill_waves_per_simd(int head_dim) { return head_dim <= 128 ? 2 : 1; }

}  // namespace vtb
