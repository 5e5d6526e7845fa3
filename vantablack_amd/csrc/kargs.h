// Kernel argument blocks, the single definition shared by the gfx950 kernels
// (hipcc --genco) and the host launcher (g++).  Each kernel takes one of
// these structs by value; hipModuleLaunchKernel copies the host's bytes into
// the kernel argument segment, so both compilers must lay the struct out
// identically.  Only fixed-size scalar and pointer members are used, and the
// static_asserts below pin every struct's size and the offsets of its wide
// members: a member added or reordered in a way the two targets would lay out
// differently fails to compile on whichever side disagrees.
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace vtb {

// Decode attention (vtb_decode_*), also the f32-cache prefill.
struct DecodeArgs {
  const float* q;       // [n_q][n_heads][D] f32
  const void* k;        // layer base: row t at k + t*n_kv*D elements
  const void* v;
  float* out;           // [n_q][n_heads][D] f32
  float* ws_o;          // [n_q][units][n_splits][G][D]
  float* ws_ml;         // [n_q][units][n_splits][G][2]
  float* wg_o;          // [n_q][units][n_groups][G][D] group partials
  float* wg_ml;         // [n_q][units][n_groups][G][2]
  unsigned* counters;   // [n_q][n_kv][n_groups + 1] x decode_counter_stride, zero between launches
  int n_heads;
  int n_kv;
  int n_splits;
  int rows_per_split;   // multiple of NW * RPW
  long long pos0;       // absolute position of query 0
  long long window;     // sliding window in rows; <= 0 disables it
  float scale_log2;     // (1/sqrt(D)) * log2(e)
  int merge_mode;       // kDecodeMergeInKernel or kDecodeMergeLaunch
  const float* k_new;   // optional (decode only): f32 K/V row appended at
  const float* v_new;   //   row pos0 before attention; null when not fused
  const float* rope_inv_freq;  // optional: [D/2] 1/base^(2j/D); RoPE of q and
  long long rope_pos;          //   k_new at absolute position rope_pos is
  int rope_half;               //   fused when set (half form if rope_half)
  // XCD-local split merge (one query, in-kernel merge): the number of XCDs
  // nx the launch's workgroups are dealt over round-robin, 0 when off.
  // Workgroup i then serves unit (i % nx) * (units / nx) + (i / nx) /
  // n_splits, split (i / nx) % n_splits, so every split of a unit runs on
  // one XCD and its partials travel through that XCD's L2 (sc0 stores and
  // loads) instead of through to memory (sc1).
  int xcd_map;
};
static_assert(sizeof(DecodeArgs) == 152, "DecodeArgs layout");
static_assert(offsetof(DecodeArgs, n_heads) == 72 && offsetof(DecodeArgs, pos0) == 88 &&
                  offsetof(DecodeArgs, scale_log2) == 104 && offsetof(DecodeArgs, k_new) == 112 &&
                  offsetof(DecodeArgs, rope_pos) == 136 && offsetof(DecodeArgs, rope_half) == 144,
              "DecodeArgs layout");
// DecodeArgs::merge_mode.  kDecodeMergeInKernel: the last-arriving
// workgroup of each unit merges the split partials (in groups past
// decode_merge_flat).  kDecodeMergeLaunch: the workgroups only publish their
// partials and a vtb_decode_merge launch after the kernel merges them.
constexpr int kDecodeMergeInKernel = 0;
constexpr int kDecodeMergeLaunch = 1;

// Split merge as a launch of its own (vtb_decode_merge): one wave per
// float4 column of one unit's result, its lanes over the split partials
// (4 per lane: n_splits <= 256).  Units and their query heads as in the
// decode launch: unit u = (query b, KV head group kvg) with u = b * units +
// kvg; hg KV heads of uniform GQA groups of g per unit when hg > 1, else
// the group of KV head kvg under the (h * n_kv) / n_heads map.
struct DecodeMergeArgs {
  const float* ws_o;    // [n_units][n_splits][slots][D]
  const float* ws_ml;   // [n_units][n_splits][slots][2]
  float* out;           // [n_q][n_heads][D]
  int n_splits;
  int slots;            // query slots per unit (hg * g, or the kernel's G)
  int head_dim;
  int units;            // units per query
  int n_units;          // units * n_q
  int n_heads;
  int n_kv;
  int hg;
};
static_assert(sizeof(DecodeMergeArgs) == 56, "DecodeMergeArgs layout");

// Causal prefill attention (vtb_prefill_d*).  Every MFMA operand is f16:
// the f32 queries are converted in registers with a power-of-two scale per
// wave (32 queries of one head); keys come from the conversion pass (or
// straight from an f16 cache) with a power-of-two exponent per 64-key tile,
// V^T likewise.  A workgroup reads the conversion pass's statistics of the
// key tiles it attends and takes q as two f16 pieces when the
// Cauchy-Schwarz bound on its scores, max |q| * max |k_t| * scale_log2,
// exceeds 32, and P as two pieces when its values' crest factor (max / rms)
// exceeds 8.
struct PrefillArgs {
  const float* q;            // [n_q][n_heads][D] f32 (prefill.zig's s.q)
  const void* k;             // f16 keys: key t of KV head h at k + h*k_head_stride + t*k_row_stride elements
  const void* vt;            // f16 V^T from the pre-pass: [n_kv][D][vt_ld]
  float* out;                // [n_q][n_heads][D] f32
  const int* texp;           // [n_kv][vt_ld / 64][2]: a tile's keys / values were scaled by 2^-ek / 2^-ev; null: 0
  const float* tstat;        // [n_kv][vt_ld / 64][8]: the conversion pass's tile statistics
  long long k_row_stride;    // elements between consecutive keys of one head
  long long k_head_stride;   // elements between KV heads
  long long pos0;            // absolute position of query 0
  long long window;          // sliding window in rows; <= 0 disables it
  int n_q;
  int n_heads;
  int n_kv;
  int vt_ld;                 // keys per V^T row (multiple of 64, >= pos0 + n_q)
  float scale_log2;          // (1/sqrt(D)) * log2(e)
  int flags;                 // kPrefillBalance
  float* part_o;             // balance: split-block partials [n_heads][nblk / 2][2][threads][D / 2] f32
  float* part_ml;            // [n_heads][nblk / 2][2][threads][4]: (m, l, E, 0), O in units of 2^E
  unsigned* part_ctr;        // [n_heads][nblk / 2] x 32 arrival counters, zero between launches
};
// PrefillArgs::flags.  kPrefillBalance: paired key ranges (prefill_entry;
// d256, nblk even).  kPrefillPairOrder: the grid fits two workgroups per
// CU at once, so the second half of the dispatch order takes the query
// blocks complementary to the first half's (prefill_entry).
constexpr int kPrefillBalance = 1;
constexpr int kPrefillPairOrder = 2;
static_assert(sizeof(PrefillArgs) == 128 && offsetof(PrefillArgs, flags) == 100 &&
                  offsetof(PrefillArgs, part_o) == 104 && offsetof(PrefillArgs, part_ctr) == 120,
              "PrefillArgs layout");
static_assert(offsetof(PrefillArgs, texp) == 32 && offsetof(PrefillArgs, tstat) == 40 &&
                  offsetof(PrefillArgs, k_row_stride) == 48 && offsetof(PrefillArgs, pos0) == 64 &&
                  offsetof(PrefillArgs, n_q) == 80 && offsetof(PrefillArgs, vt_ld) == 92 &&
                  offsetof(PrefillArgs, scale_log2) == 96,
              "PrefillArgs layout");

// Prefill conversion pass (vtb_kvt_*): one workgroup per (64-key tile, KV
// head), for the tiles [tile_lo, n_tiles) some query attends.  V^T as f16
// (keys permuted inside each 16-key group) and, for bf16 caches, the keys as
// f16.  A bf16 key tile is scaled by the power of two 2^-ek that brings its
// largest magnitude into [2^14, 2^15), a bf16 value tile by 2^-ev with ev
// that exponent rounded up to a multiple of 4 (largest magnitude in
// [2^11, 2^15): tiles of one head then share ev unless their ranges differ by
// 16x, and the attention rescales O only when ev changes); (ek, ev) go to
// texp.  Each tile's statistics go to tstat: largest |k|, sum of k^2,
// largest key-row |k_t|^2, valid keys, largest |v|, sum of v^2.
struct KvtArgs {
  const void* k;         // layer base: row t at k + t*n_kv*D elements
  const void* v;
  void* k16;             // bf16 caches: f16 keys [n_kv][vt_ld][D]; null for f16 caches
  void* vt;              // f16 [n_kv][D][vt_ld]
  float* tstat;          // [n_kv][n_tiles][8]
  int* texp;             // bf16 caches: [n_kv][n_tiles][2] = (ek, ev); null for f16 caches
  int n_rows;            // rows of K/V to convert; keys >= n_rows are zero
  int n_kv;
  int vt_ld;             // n_tiles * 64
  int tile_lo;           // first tile converted (blockIdx.x + tile_lo is the tile)
};
static_assert(sizeof(KvtArgs) == 64 && offsetof(KvtArgs, n_rows) == 48, "KvtArgs layout");

// KV-slot append (vtb_kv_append_*).
struct AppendArgs {
  void* dst;           // already offset to the first destination element
  const float* src;
  long long n;
  int vec;             // 1 when dst/src allow 16-byte (f32) / 8-byte (16-bit) stores
  int pad;
};
static_assert(sizeof(AppendArgs) == 32 && offsetof(AppendArgs, n) == 16, "AppendArgs layout");

// Fill (vtb_fill_u32): dst[i] = value for i < n.  Clears counters with a
// kernel rather than hipMemsetAsync, which some callers cannot capture.
struct FillArgs {
  uint32_t* dst;
  long long n;
  uint32_t value;
  int pad;
};
static_assert(sizeof(FillArgs) == 24 && offsetof(FillArgs, value) == 16, "FillArgs layout");

// Plain f32 copy (vtb_copy_f32).
struct CopyArgs {
  float* dst;
  const float* src;
  long long n;
};
static_assert(sizeof(CopyArgs) == 24, "CopyArgs layout");

// Quantised GEMV (vtb_gemv_*).
struct GemvArgs {
  const uint8_t* w;    // m rows of row_bytes
  const float* x;      // [k], 16-byte aligned
  float* out;          // [m]
  unsigned w_bytes;    // m * row_bytes rounded up to a multiple of 4
  int m;
  int k;
  int row_bytes;
  // Up to two more row blocks of the same format sharing x (the Q/K/V or
  // gate/up projections of one layer): workgroups [wg1, wg2) compute block 1
  // and [wg2, grid) block 2, each with its own weights, output and rows.
  int nblk;            // 1, 2 or 3
  int wg1, wg2;
  const uint8_t* w1;
  float* out1;
  unsigned w_bytes1;
  int m1;
  const uint8_t* w2;
  float* out2;
  unsigned w_bytes2;
  int m2;
  // Gated pair (the FFN's gate and up with its activation, nblk 1): a
  // workgroup takes rows [R/2 wg, +R/2) of both W_gate (w) and W_up (w1) and
  // writes act(gate) * up to out; 1 = silu (swiglu), 2 = gelu_approx.
  int gated;
  int pad;
};
static_assert(sizeof(GemvArgs) == 112, "GemvArgs layout");
static_assert(offsetof(GemvArgs, w1) == 56 && offsetof(GemvArgs, w2) == 80 && offsetof(GemvArgs, gated) == 104,
              "GemvArgs layout");

// Batched-matmul activation pre-pass (vtb_xsplit).
struct XSplitArgs {
  const float* x;      // [B][k]
  uint16_t* planes;    // [2][Bp][k] f16 bits: h1, h2 of x * 2^e
  float* sums;         // [Bp][k / 16]: sum of each 16-column group of x * 2^e
  float* inv_scale;    // [Bp]: 2^-e of each token
  int B;
  int Bp;              // B rounded up to the token tile; rows >= B are zero
  int k;
  int pad;
};
static_assert(sizeof(XSplitArgs) == 48 && offsetof(XSplitArgs, B) == 32, "XSplitArgs layout");

// Batched quantised matmul (vtb_qgemm_*).
struct QGemmArgs {
  const uint8_t* w;          // m rows of row_bytes
  const uint16_t* planes;    // [2][Bp][k] f16 bits from vtb_xsplit
  const float* sums;         // [Bp][k / 16] (of x * 2^e)
  const float* inv_scale;    // [Bp]: 2^-e
  float* out;                // [B][m]
  unsigned w_bytes;          // m * row_bytes rounded up to a multiple of 4
  int m;
  int k;
  int B;
  int Bp;
  int row_bytes;
  int n_rb;                  // row blocks of 128
  int n_tb;                  // token blocks of 128
};
static_assert(sizeof(QGemmArgs) == 72 && offsetof(QGemmArgs, w_bytes) == 40, "QGemmArgs layout");

// Row-wise rmsnorm (vtb_rmsnorm_f32); one workgroup per row (gridDim.x rows).
struct RmsNormArgs {
  float* out;
  const float* in;
  const float* w;
  int n;
  int n4;              // float4 chunks per row (n / 4 when every row of the three arrays is 16-byte aligned, else 0)
  float eps;
  int pad;
};
static_assert(sizeof(RmsNormArgs) == 40 && offsetof(RmsNormArgs, n) == 24, "RmsNormArgs layout");

// RoPE of rows x heads in place (vtb_rope_rows_f32).
struct RopeRowsArgs {
  float* x;                // [rows][heads][head_dim] f32
  const float* inv_freq;   // [head_dim / 2]
  long long pos0;          // position of row 0
  int rows;
  int heads;
  int head_dim;
  int half;                // ropeHalf pairing (i, i + d/2) instead of (2i, 2i+1)
};
static_assert(sizeof(RopeRowsArgs) == 40 && offsetof(RopeRowsArgs, pos0) == 16, "RopeRowsArgs layout");

// Residual add + rmsnorm (vtb_add_rmsnorm_f32).
struct AddNormArgs {
  float* x;            // residual stream, updated in place
  const float* b;      // addend
  float* out;          // normalised output (may be x)
  const float* w;
  int n;
  int n4;              // float4 chunks when all four arrays are 16-byte aligned, else 0
  float eps;
  int pad;
};
static_assert(sizeof(AddNormArgs) == 48 && offsetof(AddNormArgs, n) == 32, "AddNormArgs layout");

// Elementwise ops (vtb_swiglu_f32, vtb_gelu_approx_f32, vtb_residual_add_f32).
struct EltArgs {
  float* a;            // gate (activations) or the residual target
  const float* b;      // up, or the residual addend
  int n;
  int n4;              // as RmsNormArgs::n4
};
static_assert(sizeof(EltArgs) == 24 && offsetof(EltArgs, n) == 16, "EltArgs layout");

}  // namespace vtb
