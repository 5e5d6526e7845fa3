// Host shim of the gfx950 KV-cache attention path: the C ABI in
// include/vtb_hip.h.  Built with g++ against the HIP runtime only; the
// kernels are gfx950 code objects (hipcc --genco) embedded in this library
// and loaded with hipModuleLoadData, launched with hipModuleLaunchKernel.
//
// Mirrors the conventions of vantablack's Metal bridge (src/metal/bridge.m):
// opaque handles, NULL on failed construction, int return codes, segments
// that enqueue asynchronously and a wait_idle drain.
#include "vtb_hip.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "kargs.h"
#include "tiles.h"

using vtb::AddNormArgs;
using vtb::AppendArgs;
using vtb::CopyArgs;
using vtb::DecodeArgs;
using vtb::DecodeMergeArgs;
using vtb::EltArgs;
using vtb::FillArgs;
using vtb::GemvArgs;
using vtb::PrefillArgs;
using vtb::QGemmArgs;
using vtb::RmsNormArgs;
using vtb::RopeRowsArgs;
using vtb::KvtArgs;
using vtb::XSplitArgs;

extern "C" {
// Code objects embedded by blobs.S (.incbin of the hipcc --genco outputs).
extern const unsigned char vtb_blob_decode[];
extern const unsigned char vtb_blob_prefill[];
extern const unsigned char vtb_blob_kvcopy[];
extern const unsigned char vtb_blob_gemv[];
extern const unsigned char vtb_blob_qgemm[];
extern const unsigned char vtb_blob_layer[];
}

namespace {

constexpr int kNumKv = 3;     // f32, f16, bf16
constexpr int kNumD = 3;      // 64, 128, 256
constexpr int kNumG = 5;      // 1, 2, 4, 8, 16
const int kGs[kNumG] = {1, 2, 4, 8, 16};
const char* kKvNames[kNumKv] = {"f32", "f16", "bf16"};
const int kKvBytes[kNumKv] = {4, 2, 2};

int d_index(size_t d) { return d == 64 ? 0 : d == 128 ? 1 : d == 256 ? 2 : -1; }






}  // namespace

// Quantised GEMV formats (GGUF blocks, src/kernels/simd.zig) and rows per wave.
constexpr int kNumQuant = 4;
const char* const kQuantNames[kNumQuant] = {"q8_0", "q4_k", "q5_k", "q6_k"};
constexpr size_t kQuantBlockBytes[kNumQuant] = {34, 144, 176, 210};
constexpr size_t kQuantBlockElems[kNumQuant] = {32, 256, 256, 256};
constexpr int kNumGemvR = 3;
constexpr int kGemvRs[kNumGemvR] = {1, 2, 4};



struct VtbHipCtx {
  int device = 0;
  int cu_count = 0;
  hipStream_t stream = nullptr;
  hipModule_t mod_decode = nullptr, mod_prefill = nullptr, mod_kvcopy = nullptr, mod_gemv = nullptr,
              mod_qgemm = nullptr;
  hipFunction_t f_decode[kNumKv][kNumD][kNumG] = {};
  hipFunction_t f_decodeh[kNumKv][kNumD][2] = {};  // vtb_decodeh_<kv>_d<D>_g<1|2>: head-group form
  hipFunction_t f_decode_merge = nullptr;            // vtb_decode_merge: the split merge as its own launch
  // XCDs the workgroups of a launch are dealt over round-robin (workgroup i
  // on XCD (i + r) mod xcd_map, r varying per launch), from vtb_xcc_probe at
  // init; 0 when the dealing did not check out (no XCD-local merge).
  int xcd_map = 0;
  hipFunction_t f_prefill[kNumD] = {};
  hipFunction_t f_prefill_ks[kNumD] = {};  // key-split small-prompt form (d <= 128)
  hipFunction_t f_kvt[kNumKv][kNumD] = {};  // pre-pass per cache dtype (f16, bf16)
  hipFunction_t f_append[kNumKv] = {};
  hipFunction_t f_copy = nullptr;
  hipFunction_t f_fill = nullptr;
  hipFunction_t f_gemv[kNumQuant][kNumGemvR] = {};  // vtb_gemv_<kind>_r<1|2|4>
  hipFunction_t f_xsplit = nullptr;
  hipModule_t mod_layer = nullptr;  // rmsnorm, swiglu, gelu_approx, residual_add
  hipFunction_t f_rmsnorm = nullptr, f_swiglu = nullptr, f_gelu = nullptr, f_resadd = nullptr, f_addnorm = nullptr;
  hipFunction_t f_rope_rows = nullptr;
  hipFunction_t f_qgemm[kNumQuant] = {};  // vtb_qgemm_<kind>
  // Split-K workspace and arrival counters (counters are zero between launches).
  void* ws = nullptr;
  size_t ws_bytes = 0;
  unsigned* counters = nullptr;
  size_t n_counters = 0;
  // The decode code object's fixed scratch (vtb_decode_scratch): device
  // address from hipModuleGetGlobal at init, counters cleared there once.
  // Used only by the no-allocation decode entry; null if unavailable.
  unsigned char* dscratch = nullptr;
  // Prefill scratch written by the vtb_kvt_* pre-pass: f16 V^T, f16 keys
  // (bf16 caches), the per-tile statistics and exponents.
  void* pf = nullptr;
  size_t pf_bytes = 0;
  // Batched-matmul activation scratch: three bf16 planes [3][Bp][k] and the
  // 16-column sums [Bp][k/16], written by vtb_xsplit.
  void* qg = nullptr;
  size_t qg_bytes = 0;
  // RoPE inverse-frequency tables 1/base^(2j/d) on the device, one per
  // (base, head_dim) seen; the host copy stays alive for the async upload.
  struct RopeTable {
    float base;
    size_t head_dim;
    std::vector<float> host;
    float* dev;
  };
  std::vector<RopeTable> rope_tables;
  std::string err;
};

struct VtbHipBuf {
  VtbHipCtx* ctx;
  void* ptr;
  size_t bytes;
  bool owned;
};

struct VtbHipSeg {
  VtbHipCtx* ctx;
  int rc;
};

struct VtbHipKvCache {
  VtbHipCtx* ctx;
  size_t n_layers, n_kv_heads, head_dim, max_seq;
  int dtype;
  size_t pos;
  VtbHipBuf* k;
  VtbHipBuf* v;
};

namespace {

int set_err(VtbHipCtx* ctx, int rc, const char* what, hipError_t e = hipSuccess) {
  // The error is handled here: clear HIP's last-error slot so it does not
  // surface later in an unrelated caller (e.g. torch's next allocation).
  if (e != hipSuccess) (void)hipGetLastError();
  if (ctx) {
    char buf[512];
    if (e != hipSuccess)
      snprintf(buf, sizeof buf, "%s: %s", what, hipGetErrorString(e));
    else
      snprintf(buf, sizeof buf, "%s", what);
    ctx->err = buf;
  }
  return rc;
}

#define HIP_TRY(ctx, call, what)                                  \
  do {                                                            \
    hipError_t e_ = (call);                                       \
    if (e_ != hipSuccess) return set_err((ctx), VTB_HIP_EDEVICE, (what), e_); \
  } while (0)

int kv_bytes(int dtype) { return (dtype >= 0 && dtype < kNumKv) ? kKvBytes[dtype] : 0; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int launch(VtbHipCtx* ctx, hipFunction_t f, unsigned gx, unsigned gy, unsigned gz, unsigned bx,
           void* args, unsigned lds_bytes = 0) {
  void* params[] = {args};
  HIP_TRY(ctx, hipModuleLaunchKernel(f, gx, gy, gz, bx, 1, 1, lds_bytes, ctx->stream, params, nullptr),
          "hipModuleLaunchKernel");
  return VTB_HIP_OK;
}

// Grow the split-K workspace / counter array.  Growth waits for in-flight
// work first, so a buffer is never freed under a running kernel.
int ensure_workspace(VtbHipCtx* ctx, size_t ws_bytes, size_t n_counters) {
  if (ws_bytes > ctx->ws_bytes) {
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    if (ctx->ws) HIP_TRY(ctx, hipFree(ctx->ws), "hipFree");
    ctx->ws = nullptr;
    ctx->ws_bytes = 0;
    size_t sz = std::max(ws_bytes, (size_t)1 << 20);
    HIP_TRY(ctx, hipMalloc(&ctx->ws, sz), "hipMalloc(workspace)");
    ctx->ws_bytes = sz;
  }
  if (n_counters > ctx->n_counters) {
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    if (ctx->counters) HIP_TRY(ctx, hipFree(ctx->counters), "hipFree");
    ctx->counters = nullptr;
    ctx->n_counters = 0;
    size_t n = std::max(n_counters, (size_t)4096);
    HIP_TRY(ctx, hipMalloc((void**)&ctx->counters, n * sizeof(unsigned)), "hipMalloc(counters)");
    FillArgs fa;
    memset(&fa, 0, sizeof fa);
    fa.dst = ctx->counters;
    fa.n = (long long)n;
    const int rc = launch(ctx, ctx->f_fill, (unsigned)((n + 255) / 256), 1, 1, 256, &fa);
    if (rc) return rc;
    ctx->n_counters = n;
  }
  return VTB_HIP_OK;
}

int env_int(const char* name, int dflt) {
  const char* s = getenv(name);
  if (!s || !*s) return dflt;
  int v = atoi(s);
  return v > 0 ? v : dflt;
}
// An on/off switch: "0" turns it off, any other value on.
bool env_flag(const char* name, bool dflt) {
  const char* s = getenv(name);
  if (!s || !*s) return dflt;
  return atoi(s) != 0;
}

// Split-K decode / f32 prefill launcher.  Queries b in [0, n_q) sit at
// pos0 + b and attend [window_start, pos0 + b] of the layer rows at k/v.
// With k_new/v_new (decode, n_q == 1) the kernel first writes that f32 row,
// rounded to the cache dtype, into row pos0 (the fused KV-slot append).
// The device table inv_freq[j] = 1/base^(2j/d), j < d/2, exactly as
// math.rope / math.ropeHalf compute it (src/kernels/math.zig:94-96, :123-125:
// an f32 exponent, f32 pow, f32 reciprocal), built once per (base, d) with
// the host libm and uploaded on the context stream.  The kernel then forms
// each angle as the same f32 product pos * inv_freq[j].
const float* rope_table(VtbHipCtx* ctx, float base, size_t head_dim) {
  for (const auto& t : ctx->rope_tables)
    if (t.base == base && t.head_dim == head_dim) return t.dev;
  VtbHipCtx::RopeTable t{base, head_dim, std::vector<float>(head_dim / 2), nullptr};
  for (size_t j = 0; j < head_dim / 2; ++j)
    t.host[j] = 1.0f / powf(base, (float)(2 * j) / (float)head_dim);
  if (hipMalloc((void**)&t.dev, t.host.size() * sizeof(float)) != hipSuccess) {
    set_err(ctx, VTB_HIP_EDEVICE, "hipMalloc (rope table)");
    return nullptr;
  }
  if (hipMemcpyAsync(t.dev, t.host.data(), t.host.size() * sizeof(float), hipMemcpyHostToDevice, ctx->stream) !=
      hipSuccess) {
    (void)hipFree(t.dev);
    set_err(ctx, VTB_HIP_EDEVICE, "hipMemcpyAsync (rope table)");
    return nullptr;
  }
  ctx->rope_tables.push_back(std::move(t));
  return ctx->rope_tables.back().dev;
}

// RoPE fused into a decode launch: q and k_new are rotated at rope_pos.
struct RopeArgs {
  const float* inv_freq = nullptr;  // null: no RoPE
  long long pos = 0;
  int half = 0;
};

// The split plan of a decode launch: one workgroup per CU (the workgroup's
// waves fill the CU, and few splits keep the final merge short), rows per
// split a multiple of the rows one wave load instruction covers; split
// partials, then group partials (two-level merge), each (o[G][D],
// m/l[G][2]); one arrival counter per group plus one for the groups.
struct DecodePlan {
  long long rps, n_splits;
  size_t n_part, n_gpart, ws_need, ctr_need;
};
void decode_sizes(size_t n_q, size_t n_kv, size_t head_dim, int G, long long n_splits, DecodePlan* p) {
  const size_t n_groups = ((size_t)n_splits + vtb::decode_merge_group - 1) / vtb::decode_merge_group;
  p->n_splits = n_splits;
  p->n_part = n_q * n_kv * (size_t)n_splits * G;
  p->n_gpart = n_q * n_kv * n_groups * G;
  p->ws_need = n_splits > 1 ? (p->n_part + p->n_gpart) * (head_dim + 2) * sizeof(float) : 0;
  p->ctr_need = n_q * n_kv * (n_groups + 1) * vtb::decode_counter_stride;
}
long long decode_target_splits(VtbHipCtx* ctx, size_t n_q, size_t n_kv) {
  const long long target = env_int("VTB_DECODE_TARGET_WGS", std::max(ctx->cu_count, 1));
  const long long units = (long long)(n_kv * n_q);
  return std::min((long long)vtb::decode_max_splits, std::max(1LL, (target + units - 1) / units));
}
// units: (query, KV head group) units per query; G: the kernel's group
// width; HG: KV heads per workgroup (the partial has HG*G query slots).
int plan_decode(VtbHipCtx* ctx, size_t n_q, size_t units, size_t head_dim, long long Lmax, int dtype, int G,
                int HG, DecodePlan* p) {
  const long long quantum = vtb::decode_split_quantum((int)head_dim, kKvBytes[dtype], G, HG);
  const long long want = decode_target_splits(ctx, n_q, units);
  long long rps = (Lmax + want - 1) / want;
  rps = std::max(quantum, (rps + quantum - 1) / quantum * quantum);
  // Short ranges: a single query whose plan has more splits than the
  // kernel's flat merge takes (decode_merge_flat; more would need the merge
  // launch) gets that many splits instead, when each then holds at most
  // kDecodeShortSplitRows rows: the second launch costs more than the
  // longer splits.  C1 (512 rows, 4 KV heads, f32 d64): 64 splits of 8 rows
  // and the merge launch 9.2 us, 32 splits of 16 rows 7.95 us.
  constexpr long long kDecodeShortSplitRows = 32;
  const long long flat = vtb::decode_merge_flat(G * HG * (int)head_dim);
  if (n_q == 1 && (Lmax + rps - 1) / rps > flat) {
    const long long r = ((Lmax + flat - 1) / flat + quantum - 1) / quantum * quantum;
    if (r <= kDecodeShortSplitRows) rps = r;
  }
  const long long n_splits = (Lmax + rps - 1) / rps;
  if (n_splits > 65535) return set_err(ctx, VTB_HIP_EUNSUPPORTED, "too many splits");
  p->rps = rps;
  decode_sizes(n_q, units, head_dim, G * HG, n_splits, p);
  return VTB_HIP_OK;
}

// Largest workspace plan_decode asks for over every range length up to
// Lmax_hi: rows per split are at least ceil(L / want) and at least one
// load quantum, so a launch has at most min(want, ceil(Lmax_hi / quantum))
// splits, and the sizes grow with the split count.
void decode_bound(VtbHipCtx* ctx, size_t n_q, size_t units, size_t head_dim, long long Lmax_hi, int dtype, int G,
                  int HG, DecodePlan* p) {
  const long long quantum = vtb::decode_split_quantum((int)head_dim, kKvBytes[dtype], G, HG);
  const long long n_splits = std::min(decode_target_splits(ctx, n_q, units), (Lmax_hi + quantum - 1) / quantum);
  p->rps = 0;
  decode_sizes(n_q, units, head_dim, G * HG, std::max(1LL, n_splits), p);
}

// KV heads per decode workgroup: the head-group form (decode_head_group
// heads, one row of all of them per load instruction) for uniform GQA maps
// with groups of 1 or 2 on the scalar path whose KV-head count it divides;
// VTB_DECODE_HG=1 forces one head per workgroup.
int decode_heads_per_wg(size_t n_heads, size_t n_kv, size_t head_dim, int dtype, int G) {
  if (vtb::decode_uses_mfma(kKvBytes[dtype], (int)head_dim, G) || G > 2 || n_heads != n_kv * (size_t)G) return 1;
  const int hg = vtb::decode_head_group(kKvBytes[dtype], (int)head_dim);
  if (hg <= 1 || n_kv % (size_t)hg != 0) return 1;
  const char* e = getenv("VTB_DECODE_HG");
  if (e && atoi(e) == 1) return 1;
  return hg;
}

// GQA group width the decode kernels are instantiated for (1, 2, 4, 8, 16),
// or -1 above 16.
int decode_group_index(size_t n_heads, size_t n_kv) {
  const size_t gmax = (n_heads + n_kv - 1) / n_kv;
  int gi = 0;
  while (gi < kNumG && (size_t)kGs[gi] < gmax) ++gi;
  return gi == kNumG ? -1 : gi;
}

// A caller-provided split-K workspace (the no-allocation entry's fixed
// scratch): partials of ws_bytes and n_counters arrival counters that are
// zero on entry.  Null: the context's workspace, grown on demand.
struct DecodeWorkspace {
  float* ws;
  size_t ws_bytes;
  unsigned* counters;
  size_t n_counters;
};

int launch_decode(VtbHipCtx* ctx, float* out, const float* q, const void* k, const void* v,
                  size_t n_q, size_t n_heads, size_t n_kv, size_t head_dim, long long pos0,
                  long long window, float inv_sqrt_hd, int dtype, const float* k_new = nullptr,
                  const float* v_new = nullptr, RopeArgs rope = RopeArgs(),
                  const DecodeWorkspace* fixed = nullptr) {
  const int di = d_index(head_dim);
  if (di < 0) return set_err(ctx, VTB_HIP_EUNSUPPORTED, "head_dim must be 64, 128 or 256");
  if (dtype < 0 || dtype >= kNumKv) return set_err(ctx, VTB_HIP_EINVAL, "bad kv dtype");
  if (n_heads == 0 || n_kv == 0 || n_q == 0 || pos0 < 0)
    return set_err(ctx, VTB_HIP_EINVAL, "empty shape");
  if (!aligned16(k) || !aligned16(v)) return set_err(ctx, VTB_HIP_EINVAL, "K/V not 16-byte aligned");
  const int gi = decode_group_index(n_heads, n_kv);
  if (gi < 0) return set_err(ctx, VTB_HIP_EUNSUPPORTED, "GQA group wider than 16");
  const int G = kGs[gi];
  if (n_q > 65535 || n_kv > 65535) return set_err(ctx, VTB_HIP_EUNSUPPORTED, "grid too large");

  // Longest attended range over the queries.
  long long Lmax = 0;
  for (long long b : {0LL, (long long)n_q - 1}) {
    long long qp = pos0 + b;
    long long ws = (window <= 0 || qp < window) ? 0 : qp - window + 1;
    Lmax = std::max(Lmax, qp + 1 - ws);
  }
  // The MFMA form's tile DMA addresses 16 rows of one KV head with 32-bit
  // offsets.
  if (vtb::decode_uses_mfma(kKvBytes[dtype], (int)head_dim, G) && (long long)(n_kv * head_dim) * 2 * 16 >= (1LL << 31))
    return set_err(ctx, VTB_HIP_EUNSUPPORTED, "KV row too wide");
  const int HG = decode_heads_per_wg(n_heads, n_kv, head_dim, dtype, G);
  DecodePlan pl;
  int rc0 = plan_decode(ctx, n_q, n_kv / HG, head_dim, Lmax, dtype, G, HG, &pl);
  if (rc0) return rc0;
  const long long rps = pl.rps, n_splits = pl.n_splits;
  const size_t n_part = pl.n_part, n_gpart = pl.n_gpart, ws_need = pl.ws_need, ctr_need = pl.ctr_need;
  float* ws = nullptr;
  unsigned* counters = nullptr;
  if (fixed) {
    if (ws_need > fixed->ws_bytes || ctr_need > fixed->n_counters)
      return set_err(ctx, VTB_HIP_EUNSUPPORTED,
                     "attn_decode_append_noalloc: the split-K workspace this shape needs exceeds the fixed "
                     "scratch (8 MiB: 256 KiB of counters, the rest partials)");
    ws = fixed->ws;
    counters = fixed->counters;
  } else {
    int rc = ensure_workspace(ctx, ws_need, ctr_need);
    if (rc) return rc;
    ws = (float*)ctx->ws;
    counters = ctx->counters;
  }

  DecodeArgs a;
  memset(&a, 0, sizeof a);
  a.q = q;
  a.k = k;
  a.v = v;
  a.out = out;
  a.ws_o = ws;
  a.ws_ml = a.ws_o + n_part * head_dim;
  a.wg_o = a.ws_ml + n_part * 2;
  a.wg_ml = a.wg_o + n_gpart * head_dim;
  a.counters = counters;
  a.n_heads = (int)n_heads;
  a.n_kv = (int)n_kv;
  a.n_splits = (int)n_splits;
  a.rows_per_split = (int)rps;
  a.pos0 = pos0;
  a.window = window;
  a.scale_log2 = inv_sqrt_hd * 1.4426950408889634f;
  if (k_new && (n_q != 1 || !v_new)) return set_err(ctx, VTB_HIP_EINVAL, "fused append needs one query");
  a.k_new = k_new;
  a.v_new = v_new;
  if (rope.inv_freq && (n_q != 1 || !k_new)) return set_err(ctx, VTB_HIP_EINVAL, "fused RoPE needs the fused append");
  a.rope_inv_freq = rope.inv_freq;
  a.rope_pos = rope.pos;
  a.rope_half = rope.half;
  // A single query's merge that would take two levels in the kernel (more
  // splits than decode_merge_flat) runs as a launch of its own after it;
  // VTB_DECODE_MERGE_LAUNCH=0 keeps it in the kernel.  (With several queries
  // the early ones have fewer active splits: in the kernel.)
  const bool merge_launch = n_q == 1 && n_splits > vtb::decode_merge_flat(G * HG * (int)head_dim) &&
                            env_flag("VTB_DECODE_MERGE_LAUNCH", true);
  a.merge_mode = merge_launch ? vtb::kDecodeMergeLaunch : vtb::kDecodeMergeInKernel;
  // XCD-local merge: one query on the MFMA form with an in-kernel (flat)
  // merge whose units split evenly over the XCDs; each unit's (m, l)
  // partials then fill whole 128-byte lines ((n_splits * slots) % 16 == 0),
  // so no line is written by two XCDs.  (C3: 9.9 -> 9.6 us per launch; the
  // scalar head-group form at the C2 shape measured the same either way,
  // 25.1 against 25.2 us, and keeps its units spread over the XCDs.)
  const long long units = (long long)(n_kv / HG);
  if (ctx->xcd_map > 0 && n_q == 1 && n_splits > 1 && !merge_launch && units % ctx->xcd_map == 0 &&
      (n_splits * G * HG) % 16 == 0 && vtb::kDecodeXclSlots(G * HG * (int)head_dim) &&
      vtb::decode_uses_mfma(kKvBytes[dtype], (int)head_dim, G))
    a.xcd_map = ctx->xcd_map;
  hipFunction_t f = HG > 1 ? ctx->f_decodeh[dtype][di][G - 1] : ctx->f_decode[dtype][di][gi];
  int rc = launch(ctx, f, (unsigned)n_splits, (unsigned)(n_kv / HG), (unsigned)n_q,
                  64 * vtb::decode_waves(kKvBytes[dtype], (int)head_dim, G), &a);
  if (rc || !merge_launch) return rc;
  DecodeMergeArgs m;
  memset(&m, 0, sizeof m);
  m.ws_o = a.ws_o;
  m.ws_ml = a.ws_ml;
  m.out = out;
  m.n_splits = (int)n_splits;
  m.slots = G * HG;
  m.head_dim = (int)head_dim;
  m.units = (int)(n_kv / HG);
  m.n_units = (int)(n_q * (n_kv / HG));
  m.n_heads = (int)n_heads;
  m.n_kv = (int)n_kv;
  m.hg = HG;
  const long long cols = (long long)m.n_units * m.slots * (long long)(head_dim / 4);
  return launch(ctx, ctx->f_decode_merge, (unsigned)((cols + 3) / 4), 1, 1, 256, &m);
}

// Prefill scratch layout for keys [0, vt_ld) of n_kv heads: f16 V^T
// [n_kv][D][vt_ld], the tile statistics [n_kv][vt_ld / 64][8] f32, then
// (bf16 caches) f16 keys [n_kv][vt_ld][D] and the tile exponents
// [n_kv][vt_ld / 64][2] int, then (balanced launches) the split-block
// partials; sections 256-byte aligned.
struct PrefillScratch {
  size_t vt = 0, tstat = 0, k16 = 0, texp = 0, bal_o = 0, bal_ml = 0, bytes = 0;
};
// Balanced launches (4-wave kernel): split-block partials for n_heads heads
// of nblk query blocks, threads per workgroup nt: o (head_dim / 2 floats per
// thread and piece) and (m, l, E, 0).
size_t prefill_balance_floats(size_t n_heads, size_t nblk, size_t head_dim, size_t nt) {
  return n_heads * nblk * nt * (head_dim / 2);
}
size_t prefill_balance_ml_floats(size_t n_heads, size_t nblk, size_t nt) { return n_heads * nblk * nt * 4; }
PrefillScratch prefill_scratch(size_t n_kv, size_t head_dim, long long vt_ld, int dtype, size_t bal_floats = 0,
                               size_t bal_ml_floats = 0) {
  auto up = [](size_t x) { return (x + 255) / 256 * 256; };
  PrefillScratch p;
  const size_t plane = n_kv * head_dim * (size_t)vt_ld * 2;
  const size_t n_tiles = (size_t)(vt_ld / 64);
  p.vt = 0;
  p.tstat = up(plane);
  p.bytes = p.tstat + up(n_kv * n_tiles * 8 * sizeof(float));
  if (dtype == VTB_HIP_BF16) {
    p.k16 = p.bytes;
    p.texp = p.k16 + up(plane);
    p.bytes = p.texp + up(n_kv * n_tiles * 2 * sizeof(int));
  }
  if (bal_floats) {
    p.bal_o = p.bytes;
    p.bal_ml = p.bal_o + up(bal_floats * sizeof(float));
    p.bytes = p.bal_ml + up(bal_ml_floats * sizeof(float));
  }
  return p;
}

// Grow a context scratch buffer.  Growth waits for in-flight work first, so
// a buffer is never freed under a running kernel.
int ensure_scratch(VtbHipCtx* ctx, void** buf, size_t* have, size_t need, const char* what) {
  if (need <= *have) return VTB_HIP_OK;
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  if (*buf) HIP_TRY(ctx, hipFree(*buf), "hipFree");
  *buf = nullptr;
  *have = 0;
  HIP_TRY(ctx, hipMalloc(buf, need), what);
  *have = need;
  return VTB_HIP_OK;
}

// MFMA prefill: q is f32 (prefill.zig's s.q); k/v the layer base of an f16
// or bf16 cache.  One pre-pass (V^T, tile statistics and, for bf16, the
// scaled f16 keys and tile exponents) over the 64-key tiles from the window
// start of the first query to pos0 + n_q, then the attention.
int launch_prefill_mfma(VtbHipCtx* ctx, float* out, const float* q, const void* k, const void* v,
                        size_t n_q, size_t n_heads, size_t n_kv, size_t head_dim, long long pos0,
                        long long window, float inv_sqrt_hd, int dtype) {
  const int di = d_index(head_dim);
  if (di < 0) return set_err(ctx, VTB_HIP_EUNSUPPORTED, "head_dim must be 64, 128 or 256");
  if (dtype != VTB_HIP_F16 && dtype != VTB_HIP_BF16)
    return set_err(ctx, VTB_HIP_EINVAL, "MFMA prefill needs an f16 or bf16 cache");
  if (!ctx->f_prefill[di] || !ctx->f_kvt[dtype][di])
    return set_err(ctx, VTB_HIP_EUNSUPPORTED, "prefill kernel not built for this shape");
  if (!aligned16(k) || !aligned16(v) || !aligned16(q))
    return set_err(ctx, VTB_HIP_EINVAL, "q/K/V not 16-byte aligned");
  // Key-split small prompts (d <= 128): when the plain grid of 128-query
  // workgroups would fill at most half the CUs, a workgroup takes 64
  // queries and two waves share each 32, taking alternate key tiles, so the
  // longest causal block runs half its tiles per wave and twice as many CUs
  // work.  C4 (32/8 heads, d128) at 512 tokens: 26.4 -> 23.9 us per call;
  // at 1024 tokens (a plain grid of one workgroup per CU) it measured 42.8
  // against 38.9 us, hence the half.  VTB_PREFILL_KS=0 turns it off, =2
  // forces it.
  const int ks_mode = env_flag("VTB_PREFILL_KS", true) ? env_int("VTB_PREFILL_KS", 1) : 0;
  const size_t bm_plain = (size_t)vtb::prefill_block_m((int)head_dim);
  const bool ks = ctx->f_prefill_ks[di] && ks_mode != 0 &&
                  (ks_mode == 2 || 2LL * (long long)(n_heads * ((n_q + bm_plain - 1) / bm_plain)) <= ctx->cu_count);
  const size_t bm = ks ? (size_t)vtb::prefill_item_queries(4, true) : bm_plain;
  const size_t nblk = (n_q + bm - 1) / bm;
  if (nblk > 65535 || n_heads > 0x7fffffff) return set_err(ctx, VTB_HIP_EUNSUPPORTED, "grid too large");
  // Balanced pairs of query blocks (prefill_entry; the d256 kernel, whose
  // one-wave-per-SIMD workgroups fill the CUs once at the shapes it takes):
  // an even block count and causal ranges not cut by a window.  C5 (4096
  // tokens, 8/1 heads): 140 against 214 us per call.  VTB_PREFILL_BALANCE=0
  // turns it off.
  const bool balance = !ks && env_flag("VTB_PREFILL_BALANCE", true) && head_dim >= 256 && nblk >= 2 &&
                       nblk % 2 == 0 && (window <= 0 || window >= pos0 + (long long)n_q);
  const size_t nt = 256;
  // Pre-pass over keys [0, pos0 + n_q), padded to whole 64-key tiles, from
  // the tile of the first query's window start on (no query reads earlier
  // keys).
  const long long n_rows = pos0 + (long long)n_q;
  const long long key_lo = window > 0 && pos0 >= window ? pos0 - window + 1 : 0;
  const long long bn = vtb::prefill_block_n((int)head_dim);
  const long long vt_ld = (n_rows + 63) / 64 * 64;  // multiple of the pre-pass tile and of bn
  // The kernels compare positions in 32-bit arithmetic, and their tile DMA
  // uses 32-bit offsets within a head's V^T and within a K tile.
  if (vt_ld % bn != 0 || vt_ld >= (1LL << 30) || (long long)head_dim * vt_ld * 2 >= (1LL << 31) ||
      (long long)(n_kv * head_dim) * 2 * bn >= (1LL << 31))
    return set_err(ctx, VTB_HIP_EUNSUPPORTED, "prompt too long");
  const PrefillScratch ps =
      prefill_scratch(n_kv, head_dim, vt_ld, dtype, balance ? prefill_balance_floats(n_heads, nblk, head_dim, nt) : 0,
                      balance ? prefill_balance_ml_floats(n_heads, nblk, nt) : 0);
  int rc = ensure_scratch(ctx, &ctx->pf, &ctx->pf_bytes, ps.bytes, "hipMalloc(prefill scratch)");
  if (rc) return rc;
  if (balance) {
    rc = ensure_workspace(ctx, 0, n_heads * (nblk / 2) * vtb::decode_counter_stride);
    if (rc) return rc;
  }
  char* base = (char*)ctx->pf;
  const bool bf = dtype == VTB_HIP_BF16;
  KvtArgs ka;
  memset(&ka, 0, sizeof ka);
  ka.k = k;
  ka.v = v;
  ka.vt = base + ps.vt;
  ka.tstat = (float*)(base + ps.tstat);
  if (bf) {
    ka.k16 = base + ps.k16;
    ka.texp = (int*)(base + ps.texp);
  }
  ka.n_rows = (int)n_rows;
  ka.n_kv = (int)n_kv;
  ka.vt_ld = (int)vt_ld;
  ka.tile_lo = (int)(key_lo / 64);
  rc = launch(ctx, ctx->f_kvt[dtype][di], (unsigned)(vt_ld / 64 - ka.tile_lo), (unsigned)n_kv, 1, 256, &ka);
  if (rc) return rc;

  PrefillArgs a;
  memset(&a, 0, sizeof a);
  a.q = q;
  if (bf) {  // the pre-pass's f16 keys, [n_kv][vt_ld][D]
    a.k = ka.k16;
    a.k_row_stride = (long long)head_dim;
    a.k_head_stride = vt_ld * (long long)head_dim;
  } else {   // the f16 cache itself, [row][n_kv][D]
    a.k = k;
    a.k_row_stride = (long long)(n_kv * head_dim);
    a.k_head_stride = (long long)head_dim;
  }
  a.vt = ka.vt;
  a.texp = ka.texp;
  a.tstat = ka.tstat;
  a.vt_ld = (int)vt_ld;
  a.out = out;
  a.n_q = (int)n_q;
  a.n_heads = (int)n_heads;
  a.n_kv = (int)n_kv;
  a.pos0 = pos0;
  a.window = window;
  a.scale_log2 = inv_sqrt_hd * 1.4426950408889634f;
  // One round of workgroups, two per CU (d <= 128: 72 KB of LDS each): the
  // pair order evens each CU's causal load.  VTB_PREFILL_PAIR_ORDER=0 turns
  // it off.
  if (!balance && !ks && head_dim <= 128 && nblk % 2 == 0 && (long long)(n_heads * nblk) > (long long)ctx->cu_count &&
      (long long)(n_heads * nblk) <= 2LL * ctx->cu_count && (window <= 0 || window >= pos0 + (long long)n_q) &&
      env_flag("VTB_PREFILL_PAIR_ORDER", true))
    a.flags |= vtb::kPrefillPairOrder;
  if (balance) {
    a.flags |= vtb::kPrefillBalance;
    a.part_o = (float*)(base + ps.bal_o);
    a.part_ml = (float*)(base + ps.bal_ml);
    a.part_ctr = ctx->counters;
  }
  // x = head (fastest), y = query block: the longest (causal) blocks of every
  // head are dispatched first.
  return launch(ctx, ks ? ctx->f_prefill_ks[di] : ctx->f_prefill[di], (unsigned)n_heads, (unsigned)nblk, 1,
                (unsigned)nt, &a);
}

// Quantised GEMV launcher: out[m] = W[m, k] . x.  One workgroup per R rows
// with one wave per 2048 columns (k <= 32768; R = 4 only up to 16384).  R is
// 4 where it still gives two workgroups per CU, except for Q6_K with k above
// 8192 (R = 4: 15.3 us, R = 2: 14.4 us for 4096 x 11008), else 2, else 1;
// VTB_GEMV_R overrides.
// Up to three row blocks of one format sharing x go in one launch
// (launch_gemv_blocks); R is chosen on the total rows.
int launch_gemv_blocks(VtbHipCtx* ctx, int qk, int nblk, float* const outs[], const void* const ws[],
                       const size_t ms[], const float* x, size_t k) {
  if (qk < 0 || qk >= kNumQuant) return set_err(ctx, VTB_HIP_EINVAL, "bad quant kind");
  if (nblk < 1 || nblk > 3) return set_err(ctx, VTB_HIP_EINVAL, "matmul: 1 to 3 row blocks");
  if (k == 0 || k % kQuantBlockElems[qk] != 0)
    return set_err(ctx, VTB_HIP_EINVAL, "matmul: k must be a positive multiple of the block size");
  if (k > 16 * 2048) return set_err(ctx, VTB_HIP_EUNSUPPORTED, "matmul: k above 32768");
  const size_t row_bytes = k / kQuantBlockElems[qk] * kQuantBlockBytes[qk];
  size_t m = 0;
  for (int b = 0; b < nblk; ++b) {
    if (ms[b] == 0) return set_err(ctx, VTB_HIP_EINVAL, "matmul: empty row block");
    // Offsets stay below 2^31 with room for one block past the end, where
    // the kernel points the loads of rows past m.
    if (ms[b] > 0x7fff0000 / row_bytes) return set_err(ctx, VTB_HIP_EUNSUPPORTED, "matmul: weights beyond 2 GiB");
    if ((uintptr_t)ws[b] % 4 != 0) return set_err(ctx, VTB_HIP_EINVAL, "matmul: weights not 4-byte aligned");
    m += ms[b];
  }
  if (!aligned16(x)) return set_err(ctx, VTB_HIP_EINVAL, "matmul: activations not 16-byte aligned");
  int ri = 0;
  const long long forced = env_int("VTB_GEMV_R", 0);
  for (int i = kNumGemvR - 1; i >= 0; --i) {
    const long long wgs = ((long long)m + kGemvRs[i] - 1) / kGemvRs[i];
    if (kGemvRs[i] == 4 && k > 8 * 2048) continue;  // the R = 4 kernels take at most 8 waves
    if (!forced && kGemvRs[i] == 4 && qk == 3 && k > 4 * 2048) continue;
    if (forced ? forced == kGemvRs[i] : wgs >= 2LL * std::max(ctx->cu_count, 1)) {
      ri = i;
      break;
    }
  }
  const size_t R = (size_t)kGemvRs[ri];
  // The range is rounded up to whole dwords: a raw buffer load returns zero
  // for a dword only partly in range, and the last field of a 34- or
  // 210-byte block can end two bytes into one.  With the base 4-byte
  // aligned that dword lies in the page holding the tensor's last bytes.
  auto wbytes = [&](size_t rows) { return (unsigned)((rows * row_bytes + 3) & ~(size_t)3); };
  GemvArgs a;
  memset(&a, 0, sizeof a);
  a.w = (const uint8_t*)ws[0];
  a.x = x;
  a.out = outs[0];
  a.w_bytes = wbytes(ms[0]);
  a.m = (int)ms[0];
  a.k = (int)k;
  a.row_bytes = (int)row_bytes;
  a.nblk = nblk;
  size_t grid = (ms[0] + R - 1) / R;
  if (nblk > 1) {
    a.wg1 = (int)grid;
    a.w1 = (const uint8_t*)ws[1], a.out1 = outs[1], a.w_bytes1 = wbytes(ms[1]), a.m1 = (int)ms[1];
    grid += (ms[1] + R - 1) / R;
  }
  if (nblk > 2) {
    a.wg2 = (int)grid;
    a.w2 = (const uint8_t*)ws[2], a.out2 = outs[2], a.w_bytes2 = wbytes(ms[2]), a.m2 = (int)ms[2];
    grid += (ms[2] + R - 1) / R;
  }
  const unsigned waves = (unsigned)((k + 2047) / 2048);
  // Per wave the kernel stages its 2048 activations as 8 rows of (64 + 4)
  // float4 in dynamic LDS.
  const unsigned lds = waves * 8u * (64u + 4u) * 16u;
  return launch(ctx, ctx->f_gemv[qk][ri], (unsigned)grid, 1, 1, 64 * waves, &a, lds);
}

// Gated pair: out[i] = act(W_gate[i,:] . x) * (W_up[i,:] . x), the FFN's
// gate/up GEMVs and its activation in one launch (act 1 = silu, 2 =
// gelu_approx).  R/2 rows of each matrix per workgroup, R = 4 or 2.
int launch_gemv_gated(VtbHipCtx* ctx, int qk, int act, float* out, const void* w_gate, const void* w_up,
                      const float* x, size_t m, size_t k) {
  if (qk < 0 || qk >= kNumQuant) return set_err(ctx, VTB_HIP_EINVAL, "bad quant kind");
  if (act != 1 && act != 2) return set_err(ctx, VTB_HIP_EINVAL, "matmul_gated: bad activation");
  if (m == 0 || k == 0 || k % kQuantBlockElems[qk] != 0)
    return set_err(ctx, VTB_HIP_EINVAL, "matmul_gated: k must be a positive multiple of the block size");
  if (k > 16 * 2048) return set_err(ctx, VTB_HIP_EUNSUPPORTED, "matmul_gated: k above 32768");
  const size_t row_bytes = k / kQuantBlockElems[qk] * kQuantBlockBytes[qk];
  if (m > 0x7fff0000 / row_bytes) return set_err(ctx, VTB_HIP_EUNSUPPORTED, "matmul_gated: weights beyond 2 GiB");
  if ((uintptr_t)w_gate % 4 != 0 || (uintptr_t)w_up % 4 != 0)
    return set_err(ctx, VTB_HIP_EINVAL, "matmul_gated: weights not 4-byte aligned");
  if (!aligned16(x)) return set_err(ctx, VTB_HIP_EINVAL, "matmul_gated: activations not 16-byte aligned");
  // R = 4 (two rows of each matrix) while that keeps two workgroups per CU
  // and k fits its 8 waves, else R = 2.
  int ri = -1;
  for (int i = 0; i < kNumGemvR; ++i) {
    if (kGemvRs[i] == 2) ri = i;
    if (kGemvRs[i] == 4 && k <= 8 * 2048 && (long long)((m + 1) / 2) >= 2LL * std::max(ctx->cu_count, 1)) {
      ri = i;
      break;
    }
  }
  if (ri < 0) return set_err(ctx, VTB_HIP_EUNSUPPORTED, "matmul_gated: no 2- or 4-row kernel");
  const size_t RH = (size_t)kGemvRs[ri] / 2;
  GemvArgs a;
  memset(&a, 0, sizeof a);
  a.w = (const uint8_t*)w_gate;
  a.x = x;
  a.out = out;
  a.w_bytes = (unsigned)((m * row_bytes + 3) & ~(size_t)3);
  a.m = (int)m;
  a.k = (int)k;
  a.row_bytes = (int)row_bytes;
  a.nblk = 1;
  a.w1 = (const uint8_t*)w_up;
  a.w_bytes1 = a.w_bytes;
  a.m1 = (int)m;
  a.gated = act;
  const unsigned waves = (unsigned)((k + 2047) / 2048);
  const unsigned lds = waves * 8u * (64u + 4u) * 16u;
  return launch(ctx, ctx->f_gemv[qk][ri], (unsigned)((m + RH - 1) / RH), 1, 1, 64 * waves, &a, lds);
}

int launch_gemv(VtbHipCtx* ctx, int qk, float* out, const void* w, const float* x, size_t m, size_t k) {
  float* const outs[1] = {out};
  const void* const ws[1] = {w};
  const size_t ms[1] = {m};
  return launch_gemv_blocks(ctx, qk, 1, outs, ws, ms, x, k);
}

// Batched-matmul scratch for B tokens of width k: two bf16 planes
// [2][Bp][k], the 16-column sums [Bp][k/16] and the inverse scales [Bp],
// Bp = B rounded up to 128.
size_t qgemm_scratch_bytes(size_t B, size_t k) {
  const size_t Bp = (B + 127) / 128 * 128;
  return 2 * Bp * k * 2 + Bp * (k / 16) * 4 + Bp * 4;
}

// Batched quantised matmul launcher: out[B][m] = acts[B][k] . W^T.  The
// pre-pass scales each token by a power of two and splits it into two f16
// planes, 16-column sums and the token's inverse scale in the
// context's scratch (grown on demand, after the stream drains); the GEMM
// then runs one workgroup per 128 tokens x 128 rows.
// Up to three weight matrices of one format over the same activations share
// one pre-pass (the Q/K/V or gate/up projections of a prefill layer).
int launch_qgemm_blocks(VtbHipCtx* ctx, int qk, int nblk, float* const outs[], const void* const ws[],
                        const size_t ms[], const float* acts, size_t k, size_t B) {
  if (qk < 0 || qk >= kNumQuant) return set_err(ctx, VTB_HIP_EINVAL, "bad quant kind");
  if (nblk < 1 || nblk > 3) return set_err(ctx, VTB_HIP_EINVAL, "matmul_batched: 1 to 3 weight blocks");
  if (k == 0 || B == 0 || k % kQuantBlockElems[qk] != 0 || k % 32 != 0)
    return set_err(ctx, VTB_HIP_EINVAL, "matmul_batched: k must be a positive multiple of the block size");
  // prefill.zig MAX_K: the reference returns DimTooLarge above it.
  if (k > 32768) return set_err(ctx, VTB_HIP_EUNSUPPORTED, "matmul_batched: k above 32768");
  const size_t row_bytes = k / kQuantBlockElems[qk] * kQuantBlockBytes[qk];
  for (int b = 0; b < nblk; ++b) {
    const size_t m = ms[b];
    if (m == 0) return set_err(ctx, VTB_HIP_EINVAL, "matmul_batched: empty weight block");
    if (m > 0x7fff0000 / row_bytes) return set_err(ctx, VTB_HIP_EUNSUPPORTED, "matmul_batched: weights beyond 2 GiB");
    if (B > (1u << 24) || m > (1u << 24)) return set_err(ctx, VTB_HIP_EUNSUPPORTED, "matmul_batched: too many tokens or rows");
    if ((uintptr_t)ws[b] % 4 != 0) return set_err(ctx, VTB_HIP_EINVAL, "matmul_batched: weights not 4-byte aligned");
  }
  if (!aligned16(acts)) return set_err(ctx, VTB_HIP_EINVAL, "matmul_batched: activations not 16-byte aligned");
  const size_t Bp = (B + 127) / 128 * 128;
  const size_t planes_bytes = 2 * Bp * k * 2, sums_bytes = Bp * (k / 16) * 4;
  int rc0 = ensure_scratch(ctx, &ctx->qg, &ctx->qg_bytes, qgemm_scratch_bytes(B, k),
                           "hipMalloc(batched matmul scratch)");
  if (rc0) return rc0;
  uint16_t* planes = (uint16_t*)ctx->qg;
  float* sums = (float*)((char*)ctx->qg + planes_bytes);
  float* inv_scale = (float*)((char*)ctx->qg + planes_bytes + sums_bytes);
  XSplitArgs xa;
  memset(&xa, 0, sizeof xa);
  xa.x = acts;
  xa.planes = planes;
  xa.sums = sums;
  xa.inv_scale = inv_scale;
  xa.B = (int)B;
  xa.Bp = (int)Bp;
  xa.k = (int)k;
  int rc = launch(ctx, ctx->f_xsplit, (unsigned)Bp, 1, 1, 256, &xa);
  if (rc) return rc;
  for (int b = 0; b < nblk; ++b) {
    QGemmArgs a;
    memset(&a, 0, sizeof a);
    a.w = (const uint8_t*)ws[b];
    a.planes = planes;
    a.sums = sums;
    a.inv_scale = inv_scale;
    a.out = outs[b];
    // Rounded up to whole dwords: the last 2-byte-aligned field can end two
    // bytes into one (see launch_gemv).
    a.w_bytes = (unsigned)((ms[b] * row_bytes + 3) & ~(size_t)3);
    a.m = (int)ms[b];
    a.k = (int)k;
    a.B = (int)B;
    a.Bp = (int)Bp;
    a.row_bytes = (int)row_bytes;
    a.n_rb = (int)((ms[b] + 127) / 128);
    a.n_tb = (int)(Bp / 128);
    rc = launch(ctx, ctx->f_qgemm[qk], (unsigned)(a.n_rb * a.n_tb), 1, 1, 256, &a);
    if (rc) return rc;
  }
  return VTB_HIP_OK;
}

int launch_qgemm(VtbHipCtx* ctx, int qk, float* out, const void* w, const float* acts, size_t m, size_t k,
                 size_t B) {
  float* const outs[1] = {out};
  const void* const ws[1] = {w};
  const size_t ms[1] = {m};
  return launch_qgemm_blocks(ctx, qk, 1, outs, ws, ms, acts, k, B);
}

int launch_append(VtbHipCtx* ctx, void* dst, const float* src, size_t n, int dtype) {
  if (n == 0) return VTB_HIP_OK;
  if (dtype < 0 || dtype >= kNumKv) return set_err(ctx, VTB_HIP_EINVAL, "bad kv dtype");
  AppendArgs a;
  memset(&a, 0, sizeof a);
  a.dst = dst;
  a.src = src;
  a.n = (long long)n;
  const uintptr_t dmask = kKvBytes[dtype] == 4 ? 15u : 7u;
  a.vec = ((reinterpret_cast<uintptr_t>(dst) & dmask) == 0 && aligned16(src)) ? 1 : 0;
  const size_t threads = (n + 3) / 4;
  const size_t blocks = (threads + 255) / 256;
  if (blocks > 0x7fffffff) return set_err(ctx, VTB_HIP_EINVAL, "append too large");
  return launch(ctx, ctx->f_append[dtype], (unsigned)blocks, 1, 1, 256, &a);
}

long long window_arg(size_t sliding_window) {
  if (sliding_window == VTB_HIP_NO_WINDOW || sliding_window > (size_t)(1LL << 62)) return 0;
  return (long long)sliding_window;
}

bool buf_ok(const VtbHipBuf* b, size_t off, size_t bytes) {
  return b && b->ptr && off <= b->bytes && bytes <= b->bytes - off;
}

char* bptr(VtbHipBuf* b, size_t off = 0) { return static_cast<char*>(b->ptr) + off; }

}  // namespace

// ============================================================== lifecycle

// Number of XCDs the workgroups of one launch are dealt over, read from the
// per-workgroup XCC ids of a launch (xcc[i] of workgroup i): nx when every
// workgroup i runs on the XCD of workgroup i mod nx and workgroups
// 0 .. nx-1 run on nx different XCDs, else 0.  The XCD-local split merge
// (DecodeArgs::xcd_map) relies on exactly this dealing.
extern "C" int vtb_hip_xcd_deal(const int* xcc, int n) {
  if (!xcc || n <= 0) return 0;
  int nx = 0;
  bool seen[16] = {};
  for (int i = 0; i < n; ++i) {
    if (xcc[i] < 0 || xcc[i] >= 16) return 0;
    if (!seen[xcc[i]]) {
      seen[xcc[i]] = true;
      ++nx;
    }
  }
  if (n < 2 * nx) return 0;  // too few workgroups to see the pattern repeat
  for (int i = nx; i < n; ++i)
    if (xcc[i] != xcc[i % nx]) return 0;
  return nx;
}

// Runs vtb_xcc_probe twice over 4096 workgroups and checks the dealing of
// both launches (vtb_hip_xcd_deal; the starting XCD may differ between
// launches).  0 on any failure or when VTB_DECODE_XCD_LOCAL=0.
int probe_xcd_map(VtbHipCtx* ctx) {
  if (!env_flag("VTB_DECODE_XCD_LOCAL", true)) return 0;
  hipFunction_t f = nullptr;
  if (hipModuleGetFunction(&f, ctx->mod_decode, "vtb_xcc_probe") != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  constexpr int kN = 4096;
  int* d = nullptr;
  if (hipMalloc((void**)&d, kN * sizeof(int)) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  std::vector<int> h(kN);
  int nx = -1;
  for (int rep = 0; rep < 2; ++rep) {
    struct {
      int* out;
    } pa{d};
    int r = -1;
    if (launch(ctx, f, kN, 1, 1, 64, &pa) == VTB_HIP_OK &&
        hipMemcpyAsync(h.data(), d, kN * sizeof(int), hipMemcpyDeviceToHost, ctx->stream) == hipSuccess &&
        hipStreamSynchronize(ctx->stream) == hipSuccess)
      r = vtb_hip_xcd_deal(h.data(), kN);
    if (r <= 0 || (nx > 0 && r != nx)) {
      nx = 0;
      break;
    }
    nx = r;
  }
  (void)hipFree(d);
  (void)hipGetLastError();
  ctx->err.clear();
  return nx > 0 ? nx : 0;
}

extern "C" VtbHipCtx* vtb_hip_init(void) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return nullptr;
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) return nullptr;
  VtbHipCtx* ctx = new VtbHipCtx();
  ctx->err.reserve(512);  // error texts (< 512 bytes) then never allocate
  ctx->device = dev;
  ctx->cu_count = prop.multiProcessorCount;
  bool ok = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) == hipSuccess;
  ok = ok && hipModuleLoadData(&ctx->mod_decode, vtb_blob_decode) == hipSuccess;
  ok = ok && hipModuleLoadData(&ctx->mod_prefill, vtb_blob_prefill) == hipSuccess;
  ok = ok && hipModuleLoadData(&ctx->mod_kvcopy, vtb_blob_kvcopy) == hipSuccess;
  ok = ok && hipModuleLoadData(&ctx->mod_gemv, vtb_blob_gemv) == hipSuccess;
  ok = ok && hipModuleLoadData(&ctx->mod_qgemm, vtb_blob_qgemm) == hipSuccess;
  ok = ok && hipModuleLoadData(&ctx->mod_layer, vtb_blob_layer) == hipSuccess;
  char name[96];
  for (int kv = 0; ok && kv < kNumKv; ++kv) {
    for (int di = 0; ok && di < kNumD; ++di) {
      const int D = 64 << di;
      for (int gi = 0; ok && gi < kNumG; ++gi) {
        snprintf(name, sizeof name, "vtb_decode_%s_d%d_g%d", kKvNames[kv], D, kGs[gi]);
        ok = hipModuleGetFunction(&ctx->f_decode[kv][di][gi], ctx->mod_decode, name) == hipSuccess;
      }
      for (int g = 1; ok && g <= 2; ++g) {
        snprintf(name, sizeof name, "vtb_decodeh_%s_d%d_g%d", kKvNames[kv], D, g);
        ok = hipModuleGetFunction(&ctx->f_decodeh[kv][di][g - 1], ctx->mod_decode, name) == hipSuccess;
      }
      if (kv != VTB_HIP_F32) {
        snprintf(name, sizeof name, "vtb_kvt_%s_d%d", kKvNames[kv], D);
        if (hipModuleGetFunction(&ctx->f_kvt[kv][di], ctx->mod_prefill, name) != hipSuccess)
          ctx->f_kvt[kv][di] = nullptr;  // shape not built: reported at launch
      }
      if (kv == 0) {
        snprintf(name, sizeof name, "vtb_prefill_d%d", D);
        if (hipModuleGetFunction(&ctx->f_prefill[di], ctx->mod_prefill, name) != hipSuccess)
          ctx->f_prefill[di] = nullptr;
        snprintf(name, sizeof name, "vtb_prefill_ks_d%d", D);
        if (D > 128 || hipModuleGetFunction(&ctx->f_prefill_ks[di], ctx->mod_prefill, name) != hipSuccess)
          ctx->f_prefill_ks[di] = nullptr;
      }
    }
    if (ok) {
      snprintf(name, sizeof name, "vtb_kv_append_%s", kKvNames[kv]);
      ok = hipModuleGetFunction(&ctx->f_append[kv], ctx->mod_kvcopy, name) == hipSuccess;
    }
  }
  ok = ok && hipModuleGetFunction(&ctx->f_decode_merge, ctx->mod_decode, "vtb_decode_merge") == hipSuccess;
  ok = ok && hipModuleGetFunction(&ctx->f_copy, ctx->mod_kvcopy, "vtb_copy_f32") == hipSuccess;
  ok = ok && hipModuleGetFunction(&ctx->f_fill, ctx->mod_kvcopy, "vtb_fill_u32") == hipSuccess;
  for (int qk = 0; ok && qk < kNumQuant; ++qk)
    for (int ri = 0; ok && ri < kNumGemvR; ++ri) {
      snprintf(name, sizeof name, "vtb_gemv_%s_r%d", kQuantNames[qk], kGemvRs[ri]);
      ok = hipModuleGetFunction(&ctx->f_gemv[qk][ri], ctx->mod_gemv, name) == hipSuccess;
    }
  ok = ok && hipModuleGetFunction(&ctx->f_xsplit, ctx->mod_qgemm, "vtb_xsplit") == hipSuccess;
  ok = ok && hipModuleGetFunction(&ctx->f_rmsnorm, ctx->mod_layer, "vtb_rmsnorm_f32") == hipSuccess;
  ok = ok && hipModuleGetFunction(&ctx->f_swiglu, ctx->mod_layer, "vtb_swiglu_f32") == hipSuccess;
  ok = ok && hipModuleGetFunction(&ctx->f_gelu, ctx->mod_layer, "vtb_gelu_approx_f32") == hipSuccess;
  ok = ok && hipModuleGetFunction(&ctx->f_resadd, ctx->mod_layer, "vtb_residual_add_f32") == hipSuccess;
  ok = ok && hipModuleGetFunction(&ctx->f_addnorm, ctx->mod_layer, "vtb_add_rmsnorm_f32") == hipSuccess;
  ok = ok && hipModuleGetFunction(&ctx->f_rope_rows, ctx->mod_layer, "vtb_rope_rows_f32") == hipSuccess;
  for (int qk = 0; ok && qk < kNumQuant; ++qk) {
    snprintf(name, sizeof name, "vtb_qgemm_%s", kQuantNames[qk]);
    ok = hipModuleGetFunction(&ctx->f_qgemm[qk], ctx->mod_qgemm, name) == hipSuccess;
  }
  (void)hipGetLastError();  // absent optional kernels are not an error for the caller
  if (!ok) {
    vtb_hip_destroy(ctx);
    return nullptr;
  }
  // The no-allocation decode entry's scratch: this device's copy of the
  // code object's array, its counter region cleared once (it is zero at
  // load; every launch leaves its counters at zero again).
  {
    hipDeviceptr_t p = nullptr;
    size_t sz = 0;
    if (hipModuleGetFunction(&ctx->f_fill, ctx->mod_kvcopy, "vtb_fill_u32") == hipSuccess &&
        hipModuleGetGlobal(&p, &sz, ctx->mod_decode, "vtb_decode_scratch") == hipSuccess &&
        sz == vtb::decode_scratch_bytes && p != nullptr) {
      FillArgs fa;
      memset(&fa, 0, sizeof fa);
      fa.dst = (uint32_t*)p;
      fa.n = (long long)(vtb::decode_scratch_counter_bytes / sizeof(uint32_t));
      if (launch(ctx, ctx->f_fill, (unsigned)((fa.n + 255) / 256), 1, 1, 256, &fa) == VTB_HIP_OK &&
          hipStreamSynchronize(ctx->stream) == hipSuccess)
        ctx->dscratch = (unsigned char*)p;
    }
    (void)hipGetLastError();
    ctx->err.clear();
  }
  ctx->xcd_map = probe_xcd_map(ctx);
  return ctx;
}

extern "C" void vtb_hip_destroy(VtbHipCtx* ctx) {
  if (!ctx) return;
  if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
  if (ctx->ws) (void)hipFree(ctx->ws);
  if (ctx->counters) (void)hipFree(ctx->counters);
  if (ctx->pf) (void)hipFree(ctx->pf);
  if (ctx->qg) (void)hipFree(ctx->qg);
  for (auto& t : ctx->rope_tables) (void)hipFree(t.dev);
  if (ctx->mod_decode) (void)hipModuleUnload(ctx->mod_decode);
  if (ctx->mod_prefill) (void)hipModuleUnload(ctx->mod_prefill);
  if (ctx->mod_kvcopy) (void)hipModuleUnload(ctx->mod_kvcopy);
  if (ctx->mod_gemv) (void)hipModuleUnload(ctx->mod_gemv);
  if (ctx->mod_qgemm) (void)hipModuleUnload(ctx->mod_qgemm);
  if (ctx->mod_layer) (void)hipModuleUnload(ctx->mod_layer);
  if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
  delete ctx;
}

extern "C" void* vtb_hip_stream(VtbHipCtx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

extern "C" const char* vtb_hip_last_error(VtbHipCtx* ctx) { return ctx ? ctx->err.c_str() : ""; }

extern "C" int vtb_hip_cu_count(VtbHipCtx* ctx) { return ctx ? ctx->cu_count : 0; }

extern "C" int vtb_hip_xcd_map(VtbHipCtx* ctx) { return ctx ? ctx->xcd_map : 0; }

// ============================================================== buffers

extern "C" VtbHipBuf* vtb_hip_alloc(VtbHipCtx* ctx, size_t bytes) {
  if (!ctx || bytes == 0) return nullptr;
  void* p = nullptr;
  const hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess) {
    set_err(ctx, VTB_HIP_EDEVICE, "hipMalloc failed", e);
    return nullptr;
  }
  return new VtbHipBuf{ctx, p, bytes, true};
}

extern "C" VtbHipBuf* vtb_hip_wrap(VtbHipCtx* ctx, void* device_ptr, size_t bytes) {
  if (!ctx || !device_ptr || bytes == 0) return nullptr;
  return new VtbHipBuf{ctx, device_ptr, bytes, false};
}

extern "C" void vtb_hip_release(VtbHipBuf* buf) {
  if (!buf) return;
  // hipFree waits for the device itself, so release never touches buf->ctx
  // and stays safe after the context is destroyed.
  if (buf->owned && buf->ptr) (void)hipFree(buf->ptr);
  delete buf;
}

extern "C" void* vtb_hip_buf_device_ptr(VtbHipBuf* buf) { return buf ? buf->ptr : nullptr; }

extern "C" size_t vtb_hip_buf_size(VtbHipBuf* buf) { return buf ? buf->bytes : 0; }

extern "C" int vtb_hip_upload(VtbHipCtx* ctx, VtbHipBuf* dst, size_t dst_offset, const void* src,
                              size_t bytes) {
  if (!ctx || !src || !buf_ok(dst, dst_offset, bytes)) return set_err(ctx, VTB_HIP_EINVAL, "upload: bad range");
  if (bytes == 0) return VTB_HIP_OK;
  HIP_TRY(ctx, hipMemcpyAsync(bptr(dst, dst_offset), src, bytes, hipMemcpyHostToDevice, ctx->stream),
          "hipMemcpyAsync(H2D)");
  // The source is caller memory that may be reused at once: complete the copy.
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  return VTB_HIP_OK;
}

extern "C" int vtb_hip_download(VtbHipCtx* ctx, void* dst, VtbHipBuf* src, size_t src_offset,
                                size_t bytes) {
  if (!ctx || !dst || !buf_ok(src, src_offset, bytes)) return set_err(ctx, VTB_HIP_EINVAL, "download: bad range");
  if (bytes == 0) return VTB_HIP_OK;
  HIP_TRY(ctx, hipMemcpyAsync(dst, bptr(src, src_offset), bytes, hipMemcpyDeviceToHost, ctx->stream),
          "hipMemcpyAsync(D2H)");
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  return VTB_HIP_OK;
}

// ============================================================== segments

extern "C" VtbHipSeg* vtb_hip_segment_begin(VtbHipCtx* ctx) {
  if (!ctx) return nullptr;
  return new VtbHipSeg{ctx, VTB_HIP_OK};
}

extern "C" int vtb_hip_segment_commit(VtbHipSeg* seg) {
  if (!seg) return VTB_HIP_EINVAL;
  int rc = seg->rc;
  delete seg;
  return rc;
}

extern "C" int vtb_hip_wait_idle(VtbHipCtx* ctx) {
  if (!ctx) return VTB_HIP_EINVAL;
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  return VTB_HIP_OK;
}

static void seg_note(VtbHipSeg* seg, int rc) {
  if (seg && seg->rc == VTB_HIP_OK) seg->rc = rc;
}

extern "C" void vtb_hip_segment_copy(VtbHipSeg* seg, VtbHipBuf* dst_buf, size_t dst_offset_bytes,
                                     VtbHipBuf* src_buf, size_t src_offset_bytes, size_t n_floats) {
  if (!seg) return;
  VtbHipCtx* ctx = seg->ctx;
  if (n_floats == 0) return;
  if ((dst_offset_bytes | src_offset_bytes) & 3u || n_floats > ((size_t)1 << 40) ||
      !buf_ok(dst_buf, dst_offset_bytes, n_floats * 4) || !buf_ok(src_buf, src_offset_bytes, n_floats * 4))
    return seg_note(seg, set_err(ctx, VTB_HIP_EINVAL, "copy: bad range"));
  CopyArgs a{(float*)bptr(dst_buf, dst_offset_bytes), (const float*)bptr(src_buf, src_offset_bytes),
             (long long)n_floats};
  seg_note(seg, launch(ctx, ctx->f_copy, (unsigned)((n_floats + 255) / 256), 1, 1, 256, &a));
}


extern "C" void vtb_hip_segment_rmsnorm_rows(VtbHipSeg* seg, VtbHipBuf* out_buf, VtbHipBuf* in_buf,
                                             VtbHipBuf* weight_buf, size_t weight_offset, size_t n, size_t rows,
                                             float eps) {
  if (!seg) return;
  VtbHipCtx* ctx = seg->ctx;
  if (n == 0 || rows == 0) return;
  if (n > 0x7fffffff / 4 || rows > 0x7fffffff || weight_offset % 4 || !buf_ok(out_buf, 0, rows * n * 4) ||
      !buf_ok(in_buf, 0, rows * n * 4) || !buf_ok(weight_buf, weight_offset, n * 4))
    return seg_note(seg, set_err(ctx, VTB_HIP_EINVAL, "rmsnorm: bad range"));
  RmsNormArgs a;
  memset(&a, 0, sizeof a);
  a.out = (float*)bptr(out_buf, 0);
  a.in = (const float*)bptr(in_buf, 0);
  a.w = (const float*)bptr(weight_buf, weight_offset);
  a.n = (int)n;
  a.n4 = (aligned16(a.out) && aligned16(a.in) && aligned16(a.w) && (rows == 1 || n % 4 == 0)) ? (int)(n / 4) : 0;
  a.eps = eps;
  seg_note(seg, launch(ctx, ctx->f_rmsnorm, (unsigned)rows, 1, 1, 1024, &a));
}

extern "C" void vtb_hip_segment_rmsnorm(VtbHipSeg* seg, VtbHipBuf* out_buf, VtbHipBuf* in_buf, VtbHipBuf* weight_buf,
                                        size_t weight_offset, size_t n, float eps) {
  vtb_hip_segment_rmsnorm_rows(seg, out_buf, in_buf, weight_buf, weight_offset, n, 1, eps);
}


extern "C" void vtb_hip_segment_rope_rows(VtbHipSeg* seg, VtbHipBuf* x_buf, size_t rows, size_t n_heads,
                                          size_t head_dim, size_t pos0, float base, int half) {
  if (!seg) return;
  VtbHipCtx* ctx = seg->ctx;
  if (rows == 0 || n_heads == 0) return;
  if (head_dim == 0 || head_dim % 2 || head_dim > 4096 || rows > 0x7fffffff || n_heads > 65535 ||
      pos0 > ((size_t)1 << 40) || !buf_ok(x_buf, 0, rows * n_heads * head_dim * 4))
    return seg_note(seg, set_err(ctx, VTB_HIP_EINVAL, "rope_rows: bad shape"));
  const float* inv = rope_table(ctx, base, head_dim);
  if (!inv) return seg_note(seg, VTB_HIP_EDEVICE);  // rope_table recorded the cause
  RopeRowsArgs a{(float*)bptr(x_buf, 0), inv, (long long)pos0, (int)rows, (int)n_heads, (int)head_dim, half ? 1 : 0};
  const size_t pairs = rows * n_heads * (head_dim / 2);
  seg_note(seg, launch(ctx, ctx->f_rope_rows, (unsigned)((pairs + 255) / 256), 1, 1, 256, &a));
}


extern "C" void vtb_hip_segment_residual_add_rmsnorm(VtbHipSeg* seg, VtbHipBuf* x_buf, VtbHipBuf* b_buf,
                                                     VtbHipBuf* out_buf, VtbHipBuf* weight_buf,
                                                     size_t weight_offset, size_t n, float eps) {
  if (!seg) return;
  VtbHipCtx* ctx = seg->ctx;
  if (n == 0) return;
  if (n > 0x7fffffff / 4 || weight_offset % 4 || !buf_ok(x_buf, 0, n * 4) || !buf_ok(b_buf, 0, n * 4) ||
      !buf_ok(out_buf, 0, n * 4) || !buf_ok(weight_buf, weight_offset, n * 4))
    return seg_note(seg, set_err(ctx, VTB_HIP_EINVAL, "residual_add_rmsnorm: bad range"));
  AddNormArgs a;
  memset(&a, 0, sizeof a);
  a.x = (float*)bptr(x_buf, 0);
  a.b = (const float*)bptr(b_buf, 0);
  a.out = (float*)bptr(out_buf, 0);
  a.w = (const float*)bptr(weight_buf, weight_offset);
  a.n = (int)n;
  a.n4 = (aligned16(a.x) && aligned16(a.b) && aligned16(a.out) && aligned16(a.w)) ? (int)(n / 4) : 0;
  a.eps = eps;
  seg_note(seg, launch(ctx, ctx->f_addnorm, 1, 1, 1, 1024, &a));
}

static void seg_elementwise(VtbHipSeg* seg, hipFunction_t f, const char* what, VtbHipBuf* a_buf, VtbHipBuf* b_buf,
                            size_t n) {
  if (!seg) return;
  VtbHipCtx* ctx = seg->ctx;
  if (n == 0) return;
  if (n > 0x7fffffff / 4 || !buf_ok(a_buf, 0, n * 4) || !buf_ok(b_buf, 0, n * 4))
    return seg_note(seg, set_err(ctx, VTB_HIP_EINVAL, what));
  EltArgs a{(float*)bptr(a_buf, 0), (const float*)bptr(b_buf, 0), (int)n, 0};
  a.n4 = (aligned16(a.a) && aligned16(a.b)) ? (int)(n / 4) : 0;
  const size_t threads = std::max((size_t)a.n4, n - 4 * (size_t)a.n4);
  seg_note(seg, launch(ctx, f, (unsigned)((threads + 255) / 256), 1, 1, 256, &a));
}

extern "C" void vtb_hip_segment_swiglu(VtbHipSeg* seg, VtbHipBuf* gate_buf, VtbHipBuf* up_buf, size_t n) {
  seg_elementwise(seg, seg ? seg->ctx->f_swiglu : nullptr, "swiglu: bad range", gate_buf, up_buf, n);
}

extern "C" void vtb_hip_segment_gelu_approx(VtbHipSeg* seg, VtbHipBuf* gate_buf, VtbHipBuf* up_buf, size_t n) {
  seg_elementwise(seg, seg ? seg->ctx->f_gelu : nullptr, "gelu_approx: bad range", gate_buf, up_buf, n);
}

extern "C" void vtb_hip_segment_residual_add(VtbHipSeg* seg, VtbHipBuf* a_buf, VtbHipBuf* b_buf, size_t n) {
  seg_elementwise(seg, seg ? seg->ctx->f_resadd : nullptr, "residual_add: bad range", a_buf, b_buf, n);
}

extern "C" void vtb_hip_segment_kv_append(VtbHipSeg* seg, VtbHipBuf* kv_buf, size_t slot_offset_bytes,
                                          int kv_dtype, VtbHipBuf* src_buf, size_t src_offset_bytes,
                                          size_t n) {
  if (!seg) return;
  VtbHipCtx* ctx = seg->ctx;
  const int eb = kv_bytes(kv_dtype);
  if (!eb) return seg_note(seg, set_err(ctx, VTB_HIP_EINVAL, "kv_append: bad dtype"));
  if (n == 0) return;
  if (slot_offset_bytes % eb || src_offset_bytes % 4 || n > ((size_t)1 << 40) ||
      !buf_ok(kv_buf, slot_offset_bytes, n * eb) || !buf_ok(src_buf, src_offset_bytes, n * 4))
    return seg_note(seg, set_err(ctx, VTB_HIP_EINVAL, "kv_append: bad range"));
  seg_note(seg, launch_append(ctx, bptr(kv_buf, slot_offset_bytes),
                              (const float*)bptr(src_buf, src_offset_bytes), n, kv_dtype));
}

extern "C" void vtb_hip_segment_attn_decode(VtbHipSeg* seg, VtbHipBuf* out_buf, VtbHipBuf* q_buf,
                                            VtbHipBuf* k_cache_buf, size_t k_cache_offset_bytes,
                                            VtbHipBuf* v_cache_buf, size_t v_cache_offset_bytes,
                                            size_t n_heads, size_t n_kv_heads, size_t head_dim,
                                            size_t seq_len, float inv_sqrt_hd, int kv_dtype) {
  if (!seg) return;
  VtbHipCtx* ctx = seg->ctx;
  const int eb = kv_bytes(kv_dtype);
  if (!eb || n_heads == 0 || n_kv_heads == 0 || head_dim == 0 || n_heads > 65535 ||
      n_kv_heads > 65535 || head_dim > 4096)
    return seg_note(seg, set_err(ctx, VTB_HIP_EINVAL, "attn_decode: bad shape"));
  const size_t qbytes = n_heads * head_dim * 4;
  if (!buf_ok(out_buf, 0, qbytes) || !buf_ok(q_buf, 0, qbytes))
    return seg_note(seg, set_err(ctx, VTB_HIP_EINVAL, "attn_decode: q/out too small"));
  if (seq_len == 0) {
    // Empty softmax: the reference leaves attn_out zeroed (forward.zig:205).
    // A fill kernel, not hipMemsetAsync, so the call can be graph-captured.
    FillArgs fa;
    memset(&fa, 0, sizeof fa);
    fa.dst = (uint32_t*)out_buf->ptr;
    fa.n = (long long)(qbytes / 4);
    return seg_note(seg, launch(ctx, ctx->f_fill, (unsigned)((fa.n + 255) / 256), 1, 1, 256, &fa));
  }
  const size_t kv_rows_bytes = seq_len * n_kv_heads * head_dim * eb;
  if (!buf_ok(k_cache_buf, k_cache_offset_bytes, kv_rows_bytes) ||
      !buf_ok(v_cache_buf, v_cache_offset_bytes, kv_rows_bytes))
    return seg_note(seg, set_err(ctx, VTB_HIP_EINVAL, "attn_decode: K/V range outside buffer"));
  seg_note(seg, launch_decode(ctx, (float*)out_buf->ptr, (const float*)q_buf->ptr,
                              bptr(k_cache_buf, k_cache_offset_bytes),
                              bptr(v_cache_buf, v_cache_offset_bytes), 1, n_heads, n_kv_heads,
                              head_dim, (long long)seq_len - 1, 0, inv_sqrt_hd, kv_dtype));
}

// Shared body of the fused-append decode entries (with or without RoPE).
static void decode_append_entry(const char* name, VtbHipSeg* seg, VtbHipBuf* out_buf, VtbHipBuf* q_buf,
                                VtbHipBuf* k_cache_buf, size_t k_cache_offset_bytes, VtbHipBuf* v_cache_buf,
                                size_t v_cache_offset_bytes, VtbHipBuf* k_cur_buf, VtbHipBuf* v_cur_buf,
                                size_t n_heads, size_t n_kv_heads, size_t head_dim, size_t seq_len,
                                float inv_sqrt_hd, int kv_dtype, const RopeArgs& rope,
                                const DecodeWorkspace* fixed = nullptr) {
  VtbHipCtx* ctx = seg->ctx;
  char msg[128];
  const int eb = kv_bytes(kv_dtype);
  if (!eb || n_heads == 0 || n_kv_heads == 0 || head_dim == 0 || n_heads > 65535 ||
      n_kv_heads > 65535 || head_dim > 4096 || seq_len == 0) {
    snprintf(msg, sizeof msg, "%s: bad shape", name);
    return seg_note(seg, set_err(ctx, VTB_HIP_EINVAL, msg));
  }
  const size_t qbytes = n_heads * head_dim * 4;
  const size_t kv_dim = n_kv_heads * head_dim;
  if (!buf_ok(out_buf, 0, qbytes) || !buf_ok(q_buf, 0, qbytes) || !buf_ok(k_cur_buf, 0, kv_dim * 4) ||
      !buf_ok(v_cur_buf, 0, kv_dim * 4)) {
    snprintf(msg, sizeof msg, "%s: q/out/k_cur/v_cur too small", name);
    return seg_note(seg, set_err(ctx, VTB_HIP_EINVAL, msg));
  }
  const size_t kv_rows_bytes = seq_len * kv_dim * eb;
  if (!buf_ok(k_cache_buf, k_cache_offset_bytes, kv_rows_bytes) ||
      !buf_ok(v_cache_buf, v_cache_offset_bytes, kv_rows_bytes)) {
    snprintf(msg, sizeof msg, "%s: K/V range outside buffer", name);
    return seg_note(seg, set_err(ctx, VTB_HIP_EINVAL, msg));
  }
  seg_note(seg, launch_decode(ctx, (float*)out_buf->ptr, (const float*)q_buf->ptr,
                              bptr(k_cache_buf, k_cache_offset_bytes), bptr(v_cache_buf, v_cache_offset_bytes),
                              1, n_heads, n_kv_heads, head_dim, (long long)seq_len - 1, 0, inv_sqrt_hd,
                              kv_dtype, (const float*)k_cur_buf->ptr, (const float*)v_cur_buf->ptr, rope, fixed));
}

// RoPE arguments for a fused launch, or an error (base must be finite and
// positive, head_dim even, pos within 2^24 so (float)pos is exact).
static int rope_args(VtbHipCtx* ctx, size_t head_dim, size_t pos, float base, int half, RopeArgs* out) {
  if (!(base > 0.0f) || !std::isfinite(base) || head_dim % 2 != 0)
    return set_err(ctx, VTB_HIP_EINVAL, "rope: base must be finite and > 0, head_dim even");
  if (pos > ((size_t)1 << 24)) return set_err(ctx, VTB_HIP_EUNSUPPORTED, "rope: position beyond 2^24");
  const float* t = rope_table(ctx, base, head_dim);
  if (!t) return VTB_HIP_EDEVICE;
  out->inv_freq = t;
  out->pos = (long long)pos;
  out->half = half ? 1 : 0;
  return VTB_HIP_OK;
}

extern "C" void vtb_hip_segment_attn_decode_append(
    VtbHipSeg* seg, VtbHipBuf* out_buf, VtbHipBuf* q_buf, VtbHipBuf* k_cache_buf, size_t k_cache_offset_bytes,
    VtbHipBuf* v_cache_buf, size_t v_cache_offset_bytes, VtbHipBuf* k_cur_buf, VtbHipBuf* v_cur_buf,
    size_t n_heads, size_t n_kv_heads, size_t head_dim, size_t seq_len, float inv_sqrt_hd, int kv_dtype) {
  if (!seg) return;
  decode_append_entry("attn_decode_append", seg, out_buf, q_buf, k_cache_buf, k_cache_offset_bytes, v_cache_buf,
                      v_cache_offset_bytes, k_cur_buf, v_cur_buf, n_heads, n_kv_heads, head_dim, seq_len,
                      inv_sqrt_hd, kv_dtype, RopeArgs());
}

// The no-allocation form: the split-K workspace is the decode code object's
// fixed scratch, so the call allocates nothing (host or device).
extern "C" void vtb_hip_segment_attn_decode_append_noalloc(
    VtbHipSeg* seg, VtbHipBuf* out_buf, VtbHipBuf* q_buf, VtbHipBuf* k_cache_buf, size_t k_cache_offset_bytes,
    VtbHipBuf* v_cache_buf, size_t v_cache_offset_bytes, VtbHipBuf* k_cur_buf, VtbHipBuf* v_cur_buf,
    size_t n_heads, size_t n_kv_heads, size_t head_dim, size_t seq_len, float inv_sqrt_hd, int kv_dtype) {
  if (!seg) return;
  VtbHipCtx* ctx = seg->ctx;
  if (!ctx->dscratch)
    return seg_note(seg, set_err(ctx, VTB_HIP_EUNSUPPORTED, "attn_decode_append_noalloc: no fixed scratch"));
  DecodeWorkspace fixed;
  fixed.counters = (unsigned*)ctx->dscratch;
  fixed.n_counters = vtb::decode_scratch_counter_bytes / sizeof(unsigned);
  fixed.ws = (float*)(ctx->dscratch + vtb::decode_scratch_counter_bytes);
  fixed.ws_bytes = vtb::decode_scratch_bytes - vtb::decode_scratch_counter_bytes;
  decode_append_entry("attn_decode_append_noalloc", seg, out_buf, q_buf, k_cache_buf, k_cache_offset_bytes,
                      v_cache_buf, v_cache_offset_bytes, k_cur_buf, v_cur_buf, n_heads, n_kv_heads, head_dim,
                      seq_len, inv_sqrt_hd, kv_dtype, RopeArgs(), &fixed);
}

extern "C" void vtb_hip_segment_attn_decode_rope_append(
    VtbHipSeg* seg, VtbHipBuf* out_buf, VtbHipBuf* q_buf, VtbHipBuf* k_cache_buf, size_t k_cache_offset_bytes,
    VtbHipBuf* v_cache_buf, size_t v_cache_offset_bytes, VtbHipBuf* k_cur_buf, VtbHipBuf* v_cur_buf,
    size_t n_heads, size_t n_kv_heads, size_t head_dim, size_t seq_len, float inv_sqrt_hd, int kv_dtype,
    size_t rope_pos, float rope_base, int rope_half) {
  if (!seg) return;
  RopeArgs rope;
  const int rc = rope_args(seg->ctx, head_dim, rope_pos, rope_base, rope_half, &rope);
  if (rc) return seg_note(seg, rc);
  decode_append_entry("attn_decode_rope_append", seg, out_buf, q_buf, k_cache_buf, k_cache_offset_bytes,
                      v_cache_buf, v_cache_offset_bytes, k_cur_buf, v_cur_buf, n_heads, n_kv_heads, head_dim,
                      seq_len, inv_sqrt_hd, kv_dtype, rope);
}

extern "C" void vtb_hip_segment_attn_prefill(VtbHipSeg* seg, VtbHipBuf* out_buf, VtbHipBuf* q_buf,
                                             VtbHipBuf* k_cache_buf, VtbHipBuf* v_cache_buf,
                                             size_t layer_offset_bytes, size_t n_tokens, size_t pos0,
                                             size_t sliding_window, size_t n_heads, size_t n_kv_heads,
                                             size_t head_dim, float inv_sqrt_hd, int dtype) {
  if (!seg) return;
  VtbHipCtx* ctx = seg->ctx;
  const int eb = kv_bytes(dtype);
  if (!eb || n_heads == 0 || n_kv_heads == 0 || head_dim == 0 || n_heads > 65535 ||
      n_kv_heads > 65535 || head_dim > 4096 || pos0 > ((size_t)1 << 40) || n_tokens > ((size_t)1 << 31))
    return seg_note(seg, set_err(ctx, VTB_HIP_EINVAL, "attn_prefill: bad shape"));
  if (n_tokens == 0) return;  // prefillCpu returns early for B == 0 (prefill.zig:120)
  const size_t qelems = n_tokens * n_heads * head_dim;
  if (!buf_ok(out_buf, 0, qelems * 4) || !buf_ok(q_buf, 0, qelems * 4))
    return seg_note(seg, set_err(ctx, VTB_HIP_EINVAL, "attn_prefill: q/out too small"));
  const size_t rows = pos0 + n_tokens;
  const size_t kv_rows_bytes = rows * n_kv_heads * head_dim * eb;
  if (!buf_ok(k_cache_buf, layer_offset_bytes, kv_rows_bytes) ||
      !buf_ok(v_cache_buf, layer_offset_bytes, kv_rows_bytes))
    return seg_note(seg, set_err(ctx, VTB_HIP_EINVAL, "attn_prefill: K/V range outside buffer"));
  const long long w = window_arg(sliding_window);
  int rc;
  if (dtype == VTB_HIP_F32)
    rc = launch_decode(ctx, (float*)out_buf->ptr, (const float*)q_buf->ptr,
                       bptr(k_cache_buf, layer_offset_bytes), bptr(v_cache_buf, layer_offset_bytes),
                       n_tokens, n_heads, n_kv_heads, head_dim, (long long)pos0, w, inv_sqrt_hd, dtype);
  else
    rc = launch_prefill_mfma(ctx, (float*)out_buf->ptr, (const float*)q_buf->ptr,
                             bptr(k_cache_buf, layer_offset_bytes),
                             bptr(v_cache_buf, layer_offset_bytes), n_tokens, n_heads, n_kv_heads,
                             head_dim, (long long)pos0, w, inv_sqrt_hd, dtype);
  seg_note(seg, rc);
}

// ============================================================== quantised GEMV

static int matmul_entry(VtbHipCtx* ctx, int qk, VtbHipBuf* out_buf, VtbHipBuf* w_buf, size_t w_offset,
                        VtbHipBuf* acts_buf, size_t m, size_t k) {
  if (!ctx || !out_buf || !w_buf || !acts_buf) return VTB_HIP_EINVAL;
  if (m == 0 || k == 0 || k % kQuantBlockElems[qk] != 0 || m > ((size_t)1 << 31) || k > ((size_t)1 << 31))
    return set_err(ctx, VTB_HIP_EINVAL, "matmul: bad shape");
  const size_t row_bytes = k / kQuantBlockElems[qk] * kQuantBlockBytes[qk];
  if (!buf_ok(w_buf, w_offset, m * row_bytes) || !buf_ok(acts_buf, 0, k * 4) || !buf_ok(out_buf, 0, m * 4))
    return set_err(ctx, VTB_HIP_EINVAL, "matmul: buffer too small");
  return launch_gemv(ctx, qk, (float*)out_buf->ptr, bptr(w_buf, w_offset), (const float*)acts_buf->ptr, m, k);
}

#define VTB_MATMUL_ENTRIES(NAME, QK)                                                                     \
  extern "C" void vtb_hip_segment_matmul_##NAME(VtbHipSeg* seg, VtbHipBuf* out_buf, VtbHipBuf* w_buf,   \
                                                size_t w_offset, VtbHipBuf* acts_buf, size_t m, size_t k) { \
    if (!seg) return;                                                                                   \
    seg_note(seg, matmul_entry(seg->ctx, QK, out_buf, w_buf, w_offset, acts_buf, m, k));                \
  }                                                                                                     \
  extern "C" int vtb_hip_matmul_##NAME(VtbHipCtx* ctx, VtbHipBuf* out_buf, VtbHipBuf* w_buf,           \
                                       size_t w_offset, VtbHipBuf* acts_buf, size_t m, size_t k) {        \
    int rc = matmul_entry(ctx, QK, out_buf, w_buf, w_offset, acts_buf, m, k);                            \
    if (rc) return rc;                                                                                  \
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");                            \
    return VTB_HIP_OK;                                                                                  \
  }

VTB_MATMUL_ENTRIES(q8_0, 0)
VTB_MATMUL_ENTRIES(q4_k, 1)
VTB_MATMUL_ENTRIES(q5_k, 2)
VTB_MATMUL_ENTRIES(q6_k, 3)

// Two or three GEMVs of one format over the same activations in one launch
// (m2 = 0: two).
static int matmul3_entry(VtbHipCtx* ctx, int qk, VtbHipBuf* out0, size_t w_off0, size_t m0, VtbHipBuf* out1,
                         size_t w_off1, size_t m1, VtbHipBuf* out2, size_t w_off2, size_t m2, VtbHipBuf* w_buf,
                         VtbHipBuf* acts_buf, size_t k) {
  if (!ctx || !out0 || !out1 || !w_buf || !acts_buf || (m2 && !out2)) return VTB_HIP_EINVAL;
  if (m0 == 0 || m1 == 0 || k == 0 || k % kQuantBlockElems[qk] != 0 || m0 > ((size_t)1 << 31) ||
      m1 > ((size_t)1 << 31) || m2 > ((size_t)1 << 31) || k > ((size_t)1 << 31))
    return set_err(ctx, VTB_HIP_EINVAL, "matmul3: bad shape");
  const size_t row_bytes = k / kQuantBlockElems[qk] * kQuantBlockBytes[qk];
  VtbHipBuf* outs_b[3] = {out0, out1, out2};
  const size_t offs[3] = {w_off0, w_off1, w_off2}, ms[3] = {m0, m1, m2};
  const int nblk = m2 ? 3 : 2;
  float* outs[3] = {nullptr, nullptr, nullptr};
  const void* ws[3] = {nullptr, nullptr, nullptr};
  if (!buf_ok(acts_buf, 0, k * 4)) return set_err(ctx, VTB_HIP_EINVAL, "matmul3: buffer too small");
  for (int b = 0; b < nblk; ++b) {
    if (!buf_ok(w_buf, offs[b], ms[b] * row_bytes) || !buf_ok(outs_b[b], 0, ms[b] * 4))
      return set_err(ctx, VTB_HIP_EINVAL, "matmul3: buffer too small");
    outs[b] = (float*)outs_b[b]->ptr;
    ws[b] = bptr(w_buf, offs[b]);
  }
  return launch_gemv_blocks(ctx, qk, nblk, outs, ws, ms, (const float*)acts_buf->ptr, k);
}

#define VTB_MATMUL3_ENTRY(NAME, QK)                                                                        \
  extern "C" void vtb_hip_segment_matmul3_##NAME(VtbHipSeg* seg, VtbHipBuf* out0, size_t w_off0, size_t m0, \
                                                 VtbHipBuf* out1, size_t w_off1, size_t m1, VtbHipBuf* out2, \
                                                 size_t w_off2, size_t m2, VtbHipBuf* w_buf,                 \
                                                 VtbHipBuf* acts_buf, size_t k) {                            \
    if (!seg) return;                                                                                     \
    seg_note(seg, matmul3_entry(seg->ctx, QK, out0, w_off0, m0, out1, w_off1, m1, out2, w_off2, m2, w_buf,  \
                                acts_buf, k));                                                            \
  }

#define VTB_MATMUL_GATED_ENTRY(NAME, QK)                                                                  \
  extern "C" void vtb_hip_segment_matmul_gated_##NAME(VtbHipSeg* seg, VtbHipBuf* out_buf, VtbHipBuf* w_buf,    \
                                                      size_t w_off_gate, size_t w_off_up, VtbHipBuf* acts_buf, \
                                                      size_t m, size_t k, int activation) {                    \
    if (!seg) return;                                                                                      \
    VtbHipCtx* ctx = seg->ctx;                                                                             \
    if (!out_buf || !w_buf || !acts_buf || m == 0 || k == 0 || k % kQuantBlockElems[QK] != 0 ||            \
        m > ((size_t)1 << 31) || k > ((size_t)1 << 31))                                                    \
      return seg_note(seg, set_err(ctx, VTB_HIP_EINVAL, "matmul_gated: bad shape"));                       \
    const size_t rb = k / kQuantBlockElems[QK] * kQuantBlockBytes[QK];                                     \
    if (!buf_ok(w_buf, w_off_gate, m * rb) || !buf_ok(w_buf, w_off_up, m * rb) || !buf_ok(acts_buf, 0, k * 4) || \
        !buf_ok(out_buf, 0, m * 4))                                                                        \
      return seg_note(seg, set_err(ctx, VTB_HIP_EINVAL, "matmul_gated: buffer too small"));                \
    seg_note(seg, launch_gemv_gated(ctx, QK, activation == 0 ? 1 : (activation == 1 ? 2 : 0),             \
                                    (float*)out_buf->ptr, bptr(w_buf, w_off_gate), bptr(w_buf, w_off_up),  \
                                    (const float*)acts_buf->ptr, m, k));                                   \
  }

VTB_MATMUL_GATED_ENTRY(q8_0, 0)
VTB_MATMUL_GATED_ENTRY(q4_k, 1)
VTB_MATMUL_GATED_ENTRY(q5_k, 2)
VTB_MATMUL_GATED_ENTRY(q6_k, 3)

VTB_MATMUL3_ENTRY(q8_0, 0)
VTB_MATMUL3_ENTRY(q4_k, 1)
VTB_MATMUL3_ENTRY(q5_k, 2)
VTB_MATMUL3_ENTRY(q6_k, 3)

static int matmul_batched_entry(VtbHipCtx* ctx, int qk, VtbHipBuf* out_buf, VtbHipBuf* w_buf, size_t w_offset,
                                VtbHipBuf* acts_buf, size_t m, size_t k, size_t B) {
  if (!ctx || !out_buf || !w_buf || !acts_buf) return VTB_HIP_EINVAL;
  if (m == 0 || k == 0 || B == 0 || k % kQuantBlockElems[qk] != 0 || m > ((size_t)1 << 31) ||
      k > ((size_t)1 << 31) || B > ((size_t)1 << 31))
    return set_err(ctx, VTB_HIP_EINVAL, "matmul_batched: bad shape");
  const size_t row_bytes = k / kQuantBlockElems[qk] * kQuantBlockBytes[qk];
  if (!buf_ok(w_buf, w_offset, m * row_bytes) || !buf_ok(acts_buf, 0, B * k * 4) || !buf_ok(out_buf, 0, B * m * 4))
    return set_err(ctx, VTB_HIP_EINVAL, "matmul_batched: buffer too small");
  return launch_qgemm(ctx, qk, (float*)out_buf->ptr, bptr(w_buf, w_offset), (const float*)acts_buf->ptr, m, k, B);
}

// Two or three batched matmuls of one format over the same activations,
// one activation pre-pass (m2 = 0: two).
static int matmul_batched3_entry(VtbHipCtx* ctx, int qk, VtbHipBuf* out0, size_t w_off0, size_t m0, VtbHipBuf* out1,
                                 size_t w_off1, size_t m1, VtbHipBuf* out2, size_t w_off2, size_t m2,
                                 VtbHipBuf* w_buf, VtbHipBuf* acts_buf, size_t k, size_t B) {
  if (!ctx || !out0 || !out1 || !w_buf || !acts_buf || (m2 && !out2)) return VTB_HIP_EINVAL;
  if (m0 == 0 || m1 == 0 || k == 0 || B == 0 || k % kQuantBlockElems[qk] != 0 || m0 > ((size_t)1 << 31) ||
      m1 > ((size_t)1 << 31) || m2 > ((size_t)1 << 31) || k > ((size_t)1 << 31) || B > ((size_t)1 << 31))
    return set_err(ctx, VTB_HIP_EINVAL, "matmul_batched3: bad shape");
  const size_t row_bytes = k / kQuantBlockElems[qk] * kQuantBlockBytes[qk];
  VtbHipBuf* outs_b[3] = {out0, out1, out2};
  const size_t offs[3] = {w_off0, w_off1, w_off2}, ms[3] = {m0, m1, m2};
  const int nblk = m2 ? 3 : 2;
  float* outs[3] = {nullptr, nullptr, nullptr};
  const void* ws[3] = {nullptr, nullptr, nullptr};
  if (!buf_ok(acts_buf, 0, B * k * 4)) return set_err(ctx, VTB_HIP_EINVAL, "matmul_batched3: buffer too small");
  for (int b = 0; b < nblk; ++b) {
    if (!buf_ok(w_buf, offs[b], ms[b] * row_bytes) || !buf_ok(outs_b[b], 0, B * ms[b] * 4))
      return set_err(ctx, VTB_HIP_EINVAL, "matmul_batched3: buffer too small");
    outs[b] = (float*)outs_b[b]->ptr;
    ws[b] = bptr(w_buf, offs[b]);
  }
  return launch_qgemm_blocks(ctx, qk, nblk, outs, ws, ms, (const float*)acts_buf->ptr, k, B);
}

#define VTB_MATMUL_BATCHED3_ENTRY(NAME, QK)                                                                   \
  extern "C" void vtb_hip_segment_matmul_batched3_##NAME(                                                    \
      VtbHipSeg* seg, VtbHipBuf* out0, size_t w_off0, size_t m0, VtbHipBuf* out1, size_t w_off1, size_t m1,  \
      VtbHipBuf* out2, size_t w_off2, size_t m2, VtbHipBuf* w_buf, VtbHipBuf* acts_buf, size_t k, size_t B) { \
    if (!seg) return;                                                                                        \
    seg_note(seg, matmul_batched3_entry(seg->ctx, QK, out0, w_off0, m0, out1, w_off1, m1, out2, w_off2, m2,   \
                                        w_buf, acts_buf, k, B));                                             \
  }

VTB_MATMUL_BATCHED3_ENTRY(q8_0, 0)
VTB_MATMUL_BATCHED3_ENTRY(q4_k, 1)
VTB_MATMUL_BATCHED3_ENTRY(q5_k, 2)
VTB_MATMUL_BATCHED3_ENTRY(q6_k, 3)

#define VTB_MATMUL_BATCHED_ENTRIES(NAME, QK)                                                              \
  extern "C" void vtb_hip_segment_matmul_batched_##NAME(VtbHipSeg* seg, VtbHipBuf* out_buf, VtbHipBuf* w_buf, \
                                                        size_t w_offset, VtbHipBuf* acts_buf, size_t m,      \
                                                        size_t k, size_t B) {                                \
    if (!seg) return;                                                                                      \
    seg_note(seg, matmul_batched_entry(seg->ctx, QK, out_buf, w_buf, w_offset, acts_buf, m, k, B));        \
  }                                                                                                        \
  extern "C" int vtb_hip_matmul_batched_##NAME(VtbHipCtx* ctx, VtbHipBuf* out_buf, VtbHipBuf* w_buf,        \
                                               size_t w_offset, VtbHipBuf* acts_buf, size_t m, size_t k,     \
                                               size_t B) {                                                  \
    int rc = matmul_batched_entry(ctx, QK, out_buf, w_buf, w_offset, acts_buf, m, k, B);                    \
    if (rc) return rc;                                                                                     \
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");                               \
    return VTB_HIP_OK;                                                                                     \
  }

VTB_MATMUL_BATCHED_ENTRIES(q8_0, 0)
VTB_MATMUL_BATCHED_ENTRIES(q4_k, 1)
VTB_MATMUL_BATCHED_ENTRIES(q5_k, 2)
VTB_MATMUL_BATCHED_ENTRIES(q6_k, 3)

// ============================================================== KvCache

extern "C" VtbHipKvCache* vtb_hip_kv_cache_init(VtbHipCtx* ctx, size_t n_layers, size_t n_kv_heads,
                                                size_t head_dim, size_t max_seq, int dtype) {
  const int eb = kv_bytes(dtype);
  if (!ctx || !eb || n_layers == 0 || n_kv_heads == 0 || head_dim == 0 || max_seq == 0) return nullptr;
  const double total = (double)n_layers * max_seq * n_kv_heads * head_dim * eb;
  if (total > 1e15) return nullptr;
  const size_t bytes = n_layers * max_seq * n_kv_heads * head_dim * eb;
  VtbHipBuf* k = vtb_hip_alloc(ctx, bytes);
  if (!k) return nullptr;
  VtbHipBuf* v = vtb_hip_alloc(ctx, bytes);
  if (!v) {
    vtb_hip_release(k);
    return nullptr;
  }
  // Unwritten rows are never read (attention stops at pos), but a defined
  // initial state keeps debugging reads deterministic.
  (void)hipMemsetAsync(k->ptr, 0, bytes, ctx->stream);
  (void)hipMemsetAsync(v->ptr, 0, bytes, ctx->stream);
  return new VtbHipKvCache{ctx, n_layers, n_kv_heads, head_dim, max_seq, dtype, 0, k, v};
}

extern "C" void vtb_hip_kv_cache_deinit(VtbHipKvCache* c) {
  if (!c) return;
  vtb_hip_release(c->k);
  vtb_hip_release(c->v);
  delete c;
}

extern "C" void vtb_hip_kv_cache_reset(VtbHipKvCache* c) {
  if (c) c->pos = 0;
}

extern "C" size_t vtb_hip_kv_cache_pos(const VtbHipKvCache* c) { return c ? c->pos : 0; }

extern "C" int vtb_hip_kv_cache_set_pos(VtbHipKvCache* c, size_t pos) {
  if (!c || pos > c->max_seq) return VTB_HIP_EINVAL;
  c->pos = pos;
  return VTB_HIP_OK;
}

extern "C" size_t vtb_hip_kv_cache_max_seq(const VtbHipKvCache* c) { return c ? c->max_seq : 0; }

extern "C" int vtb_hip_kv_cache_dtype(const VtbHipKvCache* c) { return c ? c->dtype : -1; }

extern "C" int vtb_hip_kv_cache_advance(VtbHipKvCache* c) {
  if (!c) return VTB_HIP_EINVAL;
  if (c->pos >= c->max_seq) return VTB_HIP_EFULL;
  c->pos += 1;
  return VTB_HIP_OK;
}

static size_t row_bytes(const VtbHipKvCache* c) { return c->n_kv_heads * c->head_dim * kv_bytes(c->dtype); }

extern "C" size_t vtb_hip_kv_cache_slot_offset(const VtbHipKvCache* c, size_t layer) {
  if (!c || layer >= c->n_layers || c->pos >= c->max_seq) return (size_t)-1;
  return (layer * c->max_seq + c->pos) * row_bytes(c);
}

extern "C" size_t vtb_hip_kv_cache_layer_offset(const VtbHipKvCache* c, size_t layer) {
  if (!c || layer >= c->n_layers) return (size_t)-1;
  return layer * c->max_seq * row_bytes(c);
}

extern "C" VtbHipBuf* vtb_hip_kv_cache_k(VtbHipKvCache* c) { return c ? c->k : nullptr; }
extern "C" VtbHipBuf* vtb_hip_kv_cache_v(VtbHipKvCache* c) { return c ? c->v : nullptr; }

extern "C" int vtb_hip_kv_cache_shrink_to_fit(VtbHipKvCache* c, size_t new_max_seq) {
  if (!c) return VTB_HIP_EINVAL;
  if (new_max_seq >= c->max_seq) return VTB_HIP_OK;
  if (new_max_seq < c->pos) return VTB_HIP_ESHRINK;
  if (new_max_seq == 0) return VTB_HIP_EINVAL;
  VtbHipCtx* ctx = c->ctx;
  const size_t rb = row_bytes(c);
  const size_t new_bytes = c->n_layers * new_max_seq * rb;
  VtbHipBuf* nk = vtb_hip_alloc(ctx, new_bytes);
  if (!nk) return VTB_HIP_EDEVICE;
  VtbHipBuf* nv = vtb_hip_alloc(ctx, new_bytes);
  if (!nv) {
    vtb_hip_release(nk);
    return VTB_HIP_EDEVICE;
  }
  const size_t live = c->pos * rb;
  for (size_t l = 0; l < c->n_layers && live > 0; ++l) {
    const size_t src = l * c->max_seq * rb, dst = l * new_max_seq * rb;
    if (hipMemcpyAsync(bptr(nk, dst), bptr(c->k, src), live, hipMemcpyDeviceToDevice, ctx->stream) != hipSuccess ||
        hipMemcpyAsync(bptr(nv, dst), bptr(c->v, src), live, hipMemcpyDeviceToDevice, ctx->stream) != hipSuccess) {
      vtb_hip_release(nk);
      vtb_hip_release(nv);
      return set_err(ctx, VTB_HIP_EDEVICE, "shrink_to_fit: copy failed");
    }
  }
  vtb_hip_release(c->k);  // hipFree waits for the copies above
  vtb_hip_release(c->v);
  c->k = nk;
  c->v = nv;
  c->max_seq = new_max_seq;
  return VTB_HIP_OK;
}

// ============================================================== layer-level entries

static int check_cfg(const VtbHipKvCache* c, const VtbHipAttnConfig* cfg) {
  if (!c || !cfg) return VTB_HIP_EINVAL;
  if (cfg->n_kv_heads != c->n_kv_heads || cfg->head_dim != c->head_dim || cfg->n_heads == 0)
    return VTB_HIP_EINVAL;
  return VTB_HIP_OK;
}

static int layer_attention_impl(VtbHipSeg* seg, VtbHipKvCache* c, const VtbHipAttnConfig* cfg, size_t layer,
                                VtbHipBuf* q, VtbHipBuf* k_cur, VtbHipBuf* v_cur, VtbHipBuf* attn_out,
                                const float* rope_base, int rope_half) {
  if (!seg) return VTB_HIP_EINVAL;
  VtbHipCtx* ctx = seg->ctx;
  int rc = check_cfg(c, cfg);
  if (rc) return set_err(ctx, rc, "layer_attention: config does not match cache");
  if (layer >= c->n_layers) return set_err(ctx, VTB_HIP_EINVAL, "layer_attention: layer out of range");
  if (c->pos >= c->max_seq) return set_err(ctx, VTB_HIP_EFULL, "KvCacheFull");
  const size_t kv_dim = c->n_kv_heads * c->head_dim;
  const size_t qn = cfg->n_heads * cfg->head_dim;
  if (!buf_ok(q, 0, qn * 4) || !buf_ok(attn_out, 0, qn * 4) || !buf_ok(k_cur, 0, kv_dim * 4) ||
      !buf_ok(v_cur, 0, kv_dim * 4))
    return set_err(ctx, VTB_HIP_EINVAL, "layer_attention: buffer too small");
  RopeArgs rope;
  if (rope_base) {
    rc = rope_args(ctx, cfg->head_dim, c->pos, *rope_base, rope_half, &rope);
    if (rc) return rc;
  }
  // One launch: the decode kernel (rotates q and k_cur at pos when RoPE is
  // fused,) writes the slot at pos (fused append), then attends
  // [window_start(pos), pos].
  const size_t lo = vtb_hip_kv_cache_layer_offset(c, layer);
  const float inv_sqrt_hd = 1.0f / sqrtf((float)cfg->head_dim);
  rc = launch_decode(ctx, (float*)attn_out->ptr, (const float*)q->ptr, bptr(c->k, lo), bptr(c->v, lo), 1,
                     cfg->n_heads, cfg->n_kv_heads, cfg->head_dim, (long long)c->pos,
                     window_arg(cfg->sliding_window), inv_sqrt_hd, c->dtype, (const float*)k_cur->ptr,
                     (const float*)v_cur->ptr, rope);
  seg_note(seg, rc);
  return rc;
}

extern "C" int vtb_hip_layer_attention(VtbHipSeg* seg, VtbHipKvCache* c, const VtbHipAttnConfig* cfg,
                                       size_t layer, VtbHipBuf* q, VtbHipBuf* k_cur, VtbHipBuf* v_cur,
                                       VtbHipBuf* attn_out) {
  return layer_attention_impl(seg, c, cfg, layer, q, k_cur, v_cur, attn_out, nullptr, 0);
}

extern "C" int vtb_hip_layer_attention_rope(VtbHipSeg* seg, VtbHipKvCache* c, const VtbHipAttnConfig* cfg,
                                            size_t layer, VtbHipBuf* q, VtbHipBuf* k_cur, VtbHipBuf* v_cur,
                                            VtbHipBuf* attn_out, float rope_base, int rope_half) {
  return layer_attention_impl(seg, c, cfg, layer, q, k_cur, v_cur, attn_out, &rope_base, rope_half);
}

extern "C" int vtb_hip_prefill_attention(VtbHipSeg* seg, VtbHipKvCache* c, const VtbHipAttnConfig* cfg,
                                         size_t layer, size_t n_tokens, VtbHipBuf* q, VtbHipBuf* k_cur,
                                         VtbHipBuf* v_cur, VtbHipBuf* attn_out) {
  if (!seg) return VTB_HIP_EINVAL;
  VtbHipCtx* ctx = seg->ctx;
  int rc = check_cfg(c, cfg);
  if (rc) return set_err(ctx, rc, "prefill_attention: config does not match cache");
  if (layer >= c->n_layers) return set_err(ctx, VTB_HIP_EINVAL, "prefill_attention: layer out of range");
  if (n_tokens == 0) return VTB_HIP_OK;
  if (n_tokens > c->max_seq || c->pos + n_tokens > c->max_seq) return set_err(ctx, VTB_HIP_EFULL, "KvCacheFull");
  const size_t kv_dim = c->n_kv_heads * c->head_dim;
  const size_t qn = n_tokens * cfg->n_heads * cfg->head_dim;
  if (!buf_ok(q, 0, qn * 4) || !buf_ok(attn_out, 0, qn * 4) || !buf_ok(k_cur, 0, n_tokens * kv_dim * 4) ||
      !buf_ok(v_cur, 0, n_tokens * kv_dim * 4))
    return set_err(ctx, VTB_HIP_EINVAL, "prefill_attention: buffer too small");
  const size_t slot = vtb_hip_kv_cache_slot_offset(c, layer);
  rc = launch_append(ctx, bptr(c->k, slot), (const float*)k_cur->ptr, n_tokens * kv_dim, c->dtype);
  if (!rc) rc = launch_append(ctx, bptr(c->v, slot), (const float*)v_cur->ptr, n_tokens * kv_dim, c->dtype);
  const size_t lo = vtb_hip_kv_cache_layer_offset(c, layer);
  const float inv_sqrt_hd = 1.0f / sqrtf((float)cfg->head_dim);
  const long long w = window_arg(cfg->sliding_window);
  if (!rc && c->dtype == VTB_HIP_F32) {
    rc = launch_decode(ctx, (float*)attn_out->ptr, (const float*)q->ptr, bptr(c->k, lo), bptr(c->v, lo),
                       n_tokens, cfg->n_heads, cfg->n_kv_heads, cfg->head_dim, (long long)c->pos, w,
                       inv_sqrt_hd, c->dtype);
  } else if (!rc) {
    rc = launch_prefill_mfma(ctx, (float*)attn_out->ptr, (const float*)q->ptr, bptr(c->k, lo), bptr(c->v, lo),
                             n_tokens, cfg->n_heads, cfg->n_kv_heads, cfg->head_dim, (long long)c->pos, w,
                             inv_sqrt_hd, c->dtype);
  }
  seg_note(seg, rc);
  return rc;
}

// Pre-size every buffer the context grows on demand, so that later calls
// within these bounds allocate nothing and never drain the stream for a
// growth.  The counterpart of prefill.zig's Scratch.init (prefill.zig:67-88),
// which sizes the batch scratch for B tokens and the score rows for max_seq
// once, before the first forward: here the split-K decode workspace and
// arrival counters (one query, and up to max_batch queries on f32 caches,
// whose prefill runs the decode kernel), the prefill conversion scratch for
// a max_seq-key context (f16/bf16 caches), the batched-matmul activation
// scratch for max_batch tokens of width max_matmul_k (0: none), and the
// RoPE table for rope_base (0: none).
extern "C" int vtb_hip_reserve(VtbHipCtx* ctx, const VtbHipAttnConfig* cfg, int kv_dtype, size_t max_batch,
                               size_t max_matmul_k, float rope_base) {
  if (!ctx || !cfg) return VTB_HIP_EINVAL;
  const size_t D = cfg->head_dim, n_kv = cfg->n_kv_heads, n_heads = cfg->n_heads, max_seq = cfg->max_seq;
  if (d_index(D) < 0) return set_err(ctx, VTB_HIP_EUNSUPPORTED, "reserve: head_dim must be 64, 128 or 256");
  if (!kv_bytes(kv_dtype)) return set_err(ctx, VTB_HIP_EINVAL, "reserve: bad kv dtype");
  if (n_heads == 0 || n_kv == 0 || max_seq == 0 || n_kv > 65535 || n_heads > 65535)
    return set_err(ctx, VTB_HIP_EINVAL, "reserve: bad shape");
  if (max_seq >= ((size_t)1 << 30) || max_batch > max_seq)
    return set_err(ctx, VTB_HIP_EUNSUPPORTED, "reserve: max_seq beyond 2^30 or max_batch beyond max_seq");
  const int gi = decode_group_index(n_heads, n_kv);
  if (gi < 0) return set_err(ctx, VTB_HIP_EUNSUPPORTED, "reserve: GQA group wider than 16");
  const int G = kGs[gi];
  // A query attends at most max_seq rows, and at most the window.
  long long L_hi = (long long)max_seq;
  const long long w = window_arg(cfg->sliding_window);
  if (w > 0) L_hi = std::min(L_hi, w);
  size_t ws = 0, ctr = 0;
  // Query counts from the target split count up plan one split each (no
  // partials; counters grow with the count), so the scan stops there.
  const size_t nq_hi = kv_dtype == VTB_HIP_F32 ? std::max<size_t>(max_batch, 1) : 1;
  const size_t nq_scan = std::min(nq_hi, (size_t)decode_target_splits(ctx, 1, 1));
  for (size_t nq = 1; nq <= nq_scan + 1; ++nq) {
    DecodePlan p;
    const int HG = decode_heads_per_wg(n_heads, n_kv, D, kv_dtype, G);
    decode_bound(ctx, nq <= nq_scan ? nq : nq_hi, n_kv / HG, D, L_hi, kv_dtype, G, HG, &p);
    ws = std::max(ws, p.ws_need);
    ctr = std::max(ctr, p.ctr_need);
  }
  int rc = ensure_workspace(ctx, ws, ctr);
  if (rc) return rc;
  if (kv_dtype != VTB_HIP_F32 && max_batch > 0) {
    const long long vt_ld = ((long long)max_seq + 63) / 64 * 64;
    // With balanced pairs enabled, the d256 kernel's partials for up to
    // max_batch queries.
    const bool bal = env_flag("VTB_PREFILL_BALANCE", true) && D >= 256;
    const size_t bm4 = (size_t)vtb::prefill_block_m((int)D);
    const size_t nblk4 = (max_batch + bm4 - 1) / bm4 + 1;
    rc = ensure_scratch(ctx, &ctx->pf, &ctx->pf_bytes,
                        prefill_scratch(n_kv, D, vt_ld, kv_dtype, bal ? prefill_balance_floats(n_heads, nblk4, D, 256) : 0,
                                        bal ? prefill_balance_ml_floats(n_heads, nblk4, 256) : 0)
                            .bytes,
                        "hipMalloc(prefill scratch)");
    if (rc) return rc;
    if (bal) {
      rc = ensure_workspace(ctx, 0, n_heads * (nblk4 / 2 + 1) * vtb::decode_counter_stride);
      if (rc) return rc;
    }
  }
  if (max_matmul_k > 0 && max_batch > 0) {
    if (max_matmul_k > 32768) return set_err(ctx, VTB_HIP_EUNSUPPORTED, "reserve: matmul k above 32768");
    rc = ensure_scratch(ctx, &ctx->qg, &ctx->qg_bytes, qgemm_scratch_bytes(max_batch, max_matmul_k),
                        "hipMalloc(batched matmul scratch)");
    if (rc) return rc;
  }
  if (rope_base != 0.0f) {
    RopeArgs ra;
    rc = rope_args(ctx, D, 0, rope_base, 0, &ra);
    if (rc) return rc;
  }
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  return VTB_HIP_OK;
}

// Bytes of device scratch the context holds (workspace, counters, prefill
// and batched-matmul scratch); unchanged by any call that needed no growth.
extern "C" size_t vtb_hip_scratch_bytes(VtbHipCtx* ctx) {
  if (!ctx) return 0;
  return ctx->ws_bytes + ctx->n_counters * sizeof(unsigned) + ctx->pf_bytes + ctx->qg_bytes;
}
