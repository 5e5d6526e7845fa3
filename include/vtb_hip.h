/*
 * vtb_hip.h -- C ABI of the MI355X (gfx950) KV-cache attention path for
 * vantablack.  Plain pointers, sizes and opaque handles only.
 *
 * The shape follows vantablack's Metal bridge (src/metal/bridge.h): a
 * process-long context, explicitly released buffers, "segments" that enqueue
 * asynchronously, and a wait_idle drain before the host reads results.
 *   - constructors return NULL on failure (bridge.h:23-35);
 *   - calls returning int use 0 = ok, 1 = bad arguments, 2 = device error
 *     (bridge.m:774, 799-802), plus 3 = KvCacheFull (forward.zig:27-31,161),
 *     4 = NewMaxSeqBelowPos (kv_cache.zig:149), 5 = unsupported shape;
 *   - segment encoders return void; the first error they hit is reported by
 *     vtb_hip_segment_commit (bridge.h:80-89 semantics).
 *
 * Memory is discrete HBM: buffers have no host mapping (unlike the shared
 * MTLBuffers behind KvCache at kv_cache.zig:44-57).  Host data moves only
 * through vtb_hip_upload / vtb_hip_download.
 *
 * One context owns one HIP stream; every call on a context is ordered on it.
 * A context is driven by one host thread (server.zig:463-467 serialises
 * inference the same way).
 */
#ifndef VTB_HIP_H
#define VTB_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct VtbHipCtx VtbHipCtx;
typedef struct VtbHipBuf VtbHipBuf;
typedef struct VtbHipSeg VtbHipSeg;
typedef struct VtbHipKvCache VtbHipKvCache;

enum {
    VTB_HIP_OK = 0,
    VTB_HIP_EINVAL = 1,
    VTB_HIP_EDEVICE = 2,
    VTB_HIP_EFULL = 3,
    VTB_HIP_ESHRINK = 4,
    VTB_HIP_EUNSUPPORTED = 5
};

/* KV cache element type.  vantablack's cache is f32 only
 * (kv_cache.zig:25-27); f16 and bf16 are added here. */
enum { VTB_HIP_F32 = 0, VTB_HIP_F16 = 1, VTB_HIP_BF16 = 2 };

/* LlamaConfig.sliding_window == maxInt(usize): no window (model.zig:59-62). */
#define VTB_HIP_NO_WINDOW ((size_t)-1)

/* The attention fields of LlamaConfig (model.zig:40-70). */
typedef struct {
    size_t n_heads;
    size_t n_kv_heads;
    size_t head_dim;
    size_t max_seq;
    size_t sliding_window; /* VTB_HIP_NO_WINDOW to disable */
} VtbHipAttnConfig;

/* ---- lifecycle: replaces vtb_metal_init / vtb_metal_destroy (bridge.h:23-25).
 * Binds the current HIP device, creates a default-priority stream and loads
 * the gfx950 code objects (hipModuleLoadData).  NULL if no gfx950 device. */
VtbHipCtx *vtb_hip_init(void);
void vtb_hip_destroy(VtbHipCtx *ctx);
/* The hipStream_t every call on ctx is enqueued on. */
void *vtb_hip_stream(VtbHipCtx *ctx);
/* Text of the most recent error on ctx ("" if none). */
const char *vtb_hip_last_error(VtbHipCtx *ctx);
/* Number of compute units of the bound device (0 on error). */
int vtb_hip_cu_count(VtbHipCtx *ctx);
/* No reference counterpart (introspection of a gfx950 launch property).
 * Number of XCDs the workgroups of a launch are dealt over round-robin, as
 * vtb_hip_init measured it (0: the dealing did not check out, or
 * VTB_DECODE_XCD_LOCAL=0).  When nonzero, single-query decode launches whose
 * units divide evenly over the XCDs run every split of a unit on one XCD
 * and hand the split partials over through that XCD's L2. */
int vtb_hip_xcd_map(VtbHipCtx *ctx);
/* The check vtb_hip_init applies to the XCC ids xcc[0..n) of the workgroups
 * of one launch: nx when workgroup i runs on the XCD of workgroup i mod nx
 * and workgroups 0..nx-1 on nx different XCDs (n >= 2 nx), else 0.  Host
 * logic only; no device access. */
int vtb_hip_xcd_deal(const int *xcc, int n);

/* ---- buffers: replaces vtb_metal_alloc / vtb_metal_wrap / vtb_metal_release
 * (bridge.h:27-39).  Device memory, no host pointer. */
VtbHipBuf *vtb_hip_alloc(VtbHipCtx *ctx, size_t bytes);
/* Wrap existing device memory (no copy, not freed on release). */
VtbHipBuf *vtb_hip_wrap(VtbHipCtx *ctx, void *device_ptr, size_t bytes);
void vtb_hip_release(VtbHipBuf *buf);
void *vtb_hip_buf_device_ptr(VtbHipBuf *buf);
size_t vtb_hip_buf_size(VtbHipBuf *buf);
/* Stream-ordered host<->device copies; download blocks until the bytes are
 * on the host.  These replace the host slices of the unified-memory design
 * (forward.zig:56-73). */
int vtb_hip_upload(VtbHipCtx *ctx, VtbHipBuf *dst, size_t dst_offset, const void *src, size_t bytes);
int vtb_hip_download(VtbHipCtx *ctx, void *dst, VtbHipBuf *src, size_t src_offset, size_t bytes);

/* ---- segments: replaces vtb_metal_segment_begin / _commit / vtb_metal_wait_idle
 * (bridge.h:73-89).  Work is enqueued on the context stream as it is encoded;
 * commit reports the first encoding error and does not wait. */
VtbHipSeg *vtb_hip_segment_begin(VtbHipCtx *ctx);
int vtb_hip_segment_commit(VtbHipSeg *seg);
/* Blocks until all work enqueued on ctx has finished (bridge.h:84-87). */
int vtb_hip_wait_idle(VtbHipCtx *ctx);

/* Two or three quantised GEMVs of one format over the same activations in one
 * launch: out_b[i] = W_b[i,:] . acts for the m_b rows of W_b at w_off_b in
 * w_buf (b = 0, 1, 2; m2 = 0 for two).  For the Q/K/V and gate/up
 * projections, which the reference encodes as separate segMatmulQuant calls
 * on one input (forward.zig:459-461, 502-503) or as one call on a fused
 * [Q|K|V] / [gate|up] tensor followed by copies (:443-457, :492-500).  No
 * Metal counterpart: each block is exactly vtb_hip_segment_matmul_<kind>. */
void vtb_hip_segment_matmul3_q8_0(VtbHipSeg *seg, VtbHipBuf *out0, size_t w_off0, size_t m0, VtbHipBuf *out1,
                                  size_t w_off1, size_t m1, VtbHipBuf *out2, size_t w_off2, size_t m2,
                                  VtbHipBuf *w_buf, VtbHipBuf *acts_buf, size_t k);
void vtb_hip_segment_matmul3_q4_k(VtbHipSeg *seg, VtbHipBuf *out0, size_t w_off0, size_t m0, VtbHipBuf *out1,
                                  size_t w_off1, size_t m1, VtbHipBuf *out2, size_t w_off2, size_t m2,
                                  VtbHipBuf *w_buf, VtbHipBuf *acts_buf, size_t k);
void vtb_hip_segment_matmul3_q5_k(VtbHipSeg *seg, VtbHipBuf *out0, size_t w_off0, size_t m0, VtbHipBuf *out1,
                                  size_t w_off1, size_t m1, VtbHipBuf *out2, size_t w_off2, size_t m2,
                                  VtbHipBuf *w_buf, VtbHipBuf *acts_buf, size_t k);
void vtb_hip_segment_matmul3_q6_k(VtbHipSeg *seg, VtbHipBuf *out0, size_t w_off0, size_t m0, VtbHipBuf *out1,
                                  size_t w_off1, size_t m1, VtbHipBuf *out2, size_t w_off2, size_t m2,
                                  VtbHipBuf *w_buf, VtbHipBuf *acts_buf, size_t k);

/* Two or three batched matmuls of one format over the same B tokens of
 * activations (the Q/K/V or gate/up projections of prefillLayer,
 * prefill.zig:167-169 and 216-217): out_b[B][m_b] = acts . W_b^T, each
 * block exactly vtb_hip_segment_matmul_batched_<kind>, with the activation
 * pre-pass run once for all blocks (m2 = 0 for two).  No reference
 * counterpart: a launch-count reduction over matmulBatched's calls. */
void vtb_hip_segment_matmul_batched3_q8_0(VtbHipSeg *seg, VtbHipBuf *out0, size_t w_off0, size_t m0,
                                         VtbHipBuf *out1, size_t w_off1, size_t m1, VtbHipBuf *out2, size_t w_off2,
                                         size_t m2, VtbHipBuf *w_buf, VtbHipBuf *acts_buf, size_t k, size_t B);
void vtb_hip_segment_matmul_batched3_q4_k(VtbHipSeg *seg, VtbHipBuf *out0, size_t w_off0, size_t m0,
                                         VtbHipBuf *out1, size_t w_off1, size_t m1, VtbHipBuf *out2, size_t w_off2,
                                         size_t m2, VtbHipBuf *w_buf, VtbHipBuf *acts_buf, size_t k, size_t B);
void vtb_hip_segment_matmul_batched3_q5_k(VtbHipSeg *seg, VtbHipBuf *out0, size_t w_off0, size_t m0,
                                         VtbHipBuf *out1, size_t w_off1, size_t m1, VtbHipBuf *out2, size_t w_off2,
                                         size_t m2, VtbHipBuf *w_buf, VtbHipBuf *acts_buf, size_t k, size_t B);
void vtb_hip_segment_matmul_batched3_q6_k(VtbHipSeg *seg, VtbHipBuf *out0, size_t w_off0, size_t m0,
                                         VtbHipBuf *out1, size_t w_off1, size_t m1, VtbHipBuf *out2, size_t w_off2,
                                         size_t m2, VtbHipBuf *w_buf, VtbHipBuf *acts_buf, size_t k, size_t B);

/* The FFN's gate and up GEMVs and its activation in one launch:
 * out[i] = act(W_gate[i,:] . acts) * (W_up[i,:] . acts) for the m rows of the
 * two matrices at w_off_gate / w_off_up in w_buf; activation 0 = silu
 * (math.swiglu, math.zig:154-161), 1 = tanh-approximate gelu
 * (math.gegluApprox, :166-175).  Replaces the gate/up segMatmulQuant calls
 * and the swiglu / gegluApprox encoder of gpuLayerStep
 * (forward.zig:502-507); no Metal counterpart (a fusion of those three). */
void vtb_hip_segment_matmul_gated_q8_0(VtbHipSeg *seg, VtbHipBuf *out_buf, VtbHipBuf *w_buf, size_t w_off_gate,
                                       size_t w_off_up, VtbHipBuf *acts_buf, size_t m, size_t k, int activation);
void vtb_hip_segment_matmul_gated_q4_k(VtbHipSeg *seg, VtbHipBuf *out_buf, VtbHipBuf *w_buf, size_t w_off_gate,
                                       size_t w_off_up, VtbHipBuf *acts_buf, size_t m, size_t k, int activation);
void vtb_hip_segment_matmul_gated_q5_k(VtbHipSeg *seg, VtbHipBuf *out_buf, VtbHipBuf *w_buf, size_t w_off_gate,
                                       size_t w_off_up, VtbHipBuf *acts_buf, size_t m, size_t k, int activation);
void vtb_hip_segment_matmul_gated_q6_k(VtbHipSeg *seg, VtbHipBuf *out_buf, VtbHipBuf *w_buf, size_t w_off_gate,
                                       size_t w_off_up, VtbHipBuf *acts_buf, size_t m, size_t k, int activation);

/* The small ops a full-GPU decode layer chains between its matmuls
 * (gpuLayerStep, src/runtime/forward.zig:419-513), over f32 arrays of n
 * elements.  Bad ranges are recorded on the segment (commit reports them).
 *   rmsnorm:      out = in * w * inv, inv = 1/sqrt(sum(in^2)/n + eps), w the
 *                 f32 weights at weight_offset bytes (out may be in).  Replaces
 *                 vtb_metal_segment_rmsnorm (bridge.h:115-122); math.rmsNorm
 *                 (src/kernels/math.zig:11-32).
 *   swiglu:       gate = gate / (1 + exp(-gate)) * up.  Replaces
 *                 vtb_metal_segment_swiglu (bridge.h:132-136); math.swiglu
 *                 (math.zig:154-161).
 *   gelu_approx:  gate = 0.5 g (1 + tanh(sqrt(2/pi) (g + 0.044715 g^3))) * up.
 *                 Replaces vtb_metal_segment_gelu_approx (bridge.h:138-143);
 *                 math.gegluApprox (math.zig:166-175).
 *   residual_add: a += b.  Replaces vtb_metal_segment_residual_add
 *                 (bridge.h:145-149); math.addInto. */
void vtb_hip_segment_rmsnorm(VtbHipSeg *seg, VtbHipBuf *out_buf, VtbHipBuf *in_buf, VtbHipBuf *weight_buf,
                             size_t weight_offset, size_t n, float eps);
/* rmsnorm of each of `rows` consecutive rows of n (the prefill's per-token
 * norm, prefill.zig:159-164 and 207-212), same weights for every row. */
void vtb_hip_segment_rmsnorm_rows(VtbHipSeg *seg, VtbHipBuf *out_buf, VtbHipBuf *in_buf, VtbHipBuf *weight_buf,
                                  size_t weight_offset, size_t n, size_t rows, float eps);
/* RoPE in place of x = f32 [rows][n_heads][head_dim], row t at position
 * pos0 + t: math.rope (half = 0) or math.ropeHalf (half = 1) per (token,
 * head), as prefillLayer applies them (prefill.zig:177-189).  The same
 * angles, sin/cos and operation order as the decode kernel's fused RoPE. */
void vtb_hip_segment_rope_rows(VtbHipSeg *seg, VtbHipBuf *x_buf, size_t rows, size_t n_heads, size_t head_dim,
                               size_t pos0, float base, int half);
void vtb_hip_segment_swiglu(VtbHipSeg *seg, VtbHipBuf *gate_buf, VtbHipBuf *up_buf, size_t n);
void vtb_hip_segment_gelu_approx(VtbHipSeg *seg, VtbHipBuf *gate_buf, VtbHipBuf *up_buf, size_t n);
void vtb_hip_segment_residual_add(VtbHipSeg *seg, VtbHipBuf *a_buf, VtbHipBuf *b_buf, size_t n);
/* x += b, then out = rmsnorm(x) * w (out may be x): the residual add and the
 * rmsnorm that follows it in gpuLayerStep (forward.zig:487 and 510, each
 * followed by an rmsnorm of x at :490 / the next layer's :441, or
 * gpuFinalStep's :517) in one launch, with the same arithmetic as the two
 * encoders above.  No counterpart in the Metal bridge: a fusion of
 * vtb_metal_segment_residual_add and vtb_metal_segment_rmsnorm. */
void vtb_hip_segment_residual_add_rmsnorm(VtbHipSeg *seg, VtbHipBuf *x_buf, VtbHipBuf *b_buf, VtbHipBuf *out_buf,
                                          VtbHipBuf *weight_buf, size_t weight_offset, size_t n, float eps);

/* f32 copy, dst[dst_off + i] = src[src_off + i] for i < n_floats.
 * Replaces vtb_metal_segment_copy (bridge.h:148-155). */
void vtb_hip_segment_copy(VtbHipSeg *seg, VtbHipBuf *dst_buf, size_t dst_offset_bytes,
                          VtbHipBuf *src_buf, size_t src_offset_bytes, size_t n_floats);

/* KV-slot append: kv[slot_off + i] = round(src[src_off + i]) for i < n,
 * rounding f32 to the cache dtype (nearest even).  Replaces the two
 * seg.copy splices into kv_k / kv_v (forward.zig:466-468) and the CPU
 * @memcpy into keySlot/valueSlot (forward.zig:267-269).  n may span several
 * consecutive slots (a prefill's B rows, prefill.zig:175-191). */
void vtb_hip_segment_kv_append(VtbHipSeg *seg, VtbHipBuf *kv_buf, size_t slot_offset_bytes,
                               int kv_dtype, VtbHipBuf *src_buf, size_t src_offset_bytes,
                               size_t n);

/* Decode attention for one token, one layer:
 *   out[h,:] = sum_t softmax_t((q[h] . K[t,kv_h]) * inv_sqrt_hd) V[t,kv_h,:]
 * for t in [0, seq_len), kv_h = (h*n_kv_heads)/n_heads.  q and out are f32
 * [n_heads*head_dim]; K/V rows are [n_kv_heads*head_dim] of kv_dtype starting
 * at the given byte offsets (the caller applies the sliding window by moving
 * the offset forward window_start rows and passing attended_len as seq_len,
 * exactly as forward.zig:470-483 does).  Replaces vtb_metal_segment_attn_scores,
 * _softmax_rows and _attn_weighted_sum (bridge.h:157-183) with one split-K
 * launch; no score buffer exists.  head_dim in {64,128,256}; offsets 16-byte
 * aligned. */
void vtb_hip_segment_attn_decode(VtbHipSeg *seg, VtbHipBuf *out_buf, VtbHipBuf *q_buf,
                                 VtbHipBuf *k_cache_buf, size_t k_cache_offset_bytes,
                                 VtbHipBuf *v_cache_buf, size_t v_cache_offset_bytes,
                                 size_t n_heads, size_t n_kv_heads, size_t head_dim,
                                 size_t seq_len, float inv_sqrt_hd, int kv_dtype);

/* Decode with the KV-slot append fused into the same launch: writes k_cur /
 * v_cur (f32 [n_kv_heads*head_dim]), rounded to kv_dtype, into row
 * seq_len-1 of the K/V views at the given offsets, then computes exactly
 * what vtb_hip_segment_attn_decode computes over rows [0, seq_len).
 * Replaces the Metal sequence seg.copy(kv_k slot), seg.copy(kv_v slot),
 * attention trio (forward.zig:466-483) with one launch. */
void vtb_hip_segment_attn_decode_append(VtbHipSeg *seg, VtbHipBuf *out_buf, VtbHipBuf *q_buf,
                                        VtbHipBuf *k_cache_buf, size_t k_cache_offset_bytes,
                                        VtbHipBuf *v_cache_buf, size_t v_cache_offset_bytes,
                                        VtbHipBuf *k_cur_buf, VtbHipBuf *v_cur_buf,
                                        size_t n_heads, size_t n_kv_heads, size_t head_dim,
                                        size_t seq_len, float inv_sqrt_hd, int kv_dtype);

/* vtb_hip_segment_attn_decode_append computing the same outputs, allocating
 * nothing: no counterpart in the reference.  For callers that cannot allocate
 * device or host memory mid-stream (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  The split-K partials and
 * arrival counters live in a fixed 8 MiB array of the decode code object
 * (256 KiB of counters, the rest partials; each context holds its own copy
 * until it is destroyed), not in the context's growable workspace.  A shape
 * whose workspace would exceed it is rejected with 5 (EUNSUPPORTED) at
 * commit.  A shape fits when its split plan keeps
 * (n_part + n_gpart) * (head_dim + 2) * 4 <= 8 MiB - 256 KiB and its
 * arrival counters within 256 KiB, where n_part = units * n_splits * G and
 * n_gpart = units * ceil(n_splits / 16) * G (units: KV heads, or head pairs
 * for the head-group kernels; G: the kernel's query slots per unit).  The
 * split count depends on the CU count and VTB_DECODE_TARGET_WGS, so this is
 * not a fixed set of shapes; the BASELINE decode shapes (C1, C2, C3, C5)
 * fit on a 256-CU MI355X with the default plan, and wider ones can be
 * rejected (e.g. 200 KV heads with 16-query groups at head_dim 256).  Calls
 * that overlap on one context race on the array; calls on one stream do
 * not (each launch leaves its counters at zero for the next). */
void vtb_hip_segment_attn_decode_append_noalloc(VtbHipSeg *seg, VtbHipBuf *out_buf, VtbHipBuf *q_buf,
                                                VtbHipBuf *k_cache_buf, size_t k_cache_offset_bytes,
                                                VtbHipBuf *v_cache_buf, size_t v_cache_offset_bytes,
                                                VtbHipBuf *k_cur_buf, VtbHipBuf *v_cur_buf,
                                                size_t n_heads, size_t n_kv_heads, size_t head_dim,
                                                size_t seq_len, float inv_sqrt_hd, int kv_dtype);

/* vtb_hip_segment_attn_decode_append with RoPE fused in front: q (all
 * n_heads) and k_cur (all n_kv_heads) are rotated at absolute position
 * rope_pos -- math.rope, interleaved pairs, or with rope_half math.ropeHalf,
 * pairs (i, i + head_dim/2) (src/kernels/math.zig:85-133), angle
 * rope_pos / rope_base^(2j/head_dim) -- before the slot write and the
 * attention.  Replaces the Metal sequence seg.rope(q), seg.rope(k_cur)
 * (forward.zig:463-464; kernel rope_inplace, bridge.m:130-150, which has
 * only the interleaved form), seg.copy x2 (:467-468) and the attention trio
 * (:481-483) with one launch.  q_buf and k_cur_buf are read, not rotated in
 * place (nothing reads them afterwards in the reference).  rope_pos is
 * separate from seq_len because a sliding window shifts the K/V view.  The
 * first call per (rope_base, head_dim) uploads a head_dim/2-float table.
 * rope_base finite and > 0; rope_pos <= 2^24. */
void vtb_hip_segment_attn_decode_rope_append(VtbHipSeg *seg, VtbHipBuf *out_buf, VtbHipBuf *q_buf,
                                             VtbHipBuf *k_cache_buf, size_t k_cache_offset_bytes,
                                             VtbHipBuf *v_cache_buf, size_t v_cache_offset_bytes,
                                             VtbHipBuf *k_cur_buf, VtbHipBuf *v_cur_buf,
                                             size_t n_heads, size_t n_kv_heads, size_t head_dim,
                                             size_t seq_len, float inv_sqrt_hd, int kv_dtype,
                                             size_t rope_pos, float rope_base, int rope_half);

/* Causal prefill attention for n_tokens queries of one layer.  Query b sits
 * at absolute position pos0 + b and attends rows [window_start(pos0+b),
 * pos0+b] of the layer whose row 0 is at layer_offset_bytes in k/v, where
 * window_start follows forward.zig:195-203.  Replaces the per-position loop
 * `for b: attentionCausal` (prefill.zig:193-197, 237-287), which has no Metal
 * counterpart.  q: f32 [n_tokens][n_heads*head_dim], as prefill.zig's s.q
 * (:167-189); out: f32, same shape.  For f16/bf16 caches the kernel runs on
 * f16 MFMA: each (query, head) row of q is scaled by a power of two and
 * rounded to f16, K and V are converted to f16 per 64-key tile with a
 * power-of-two scale where a bf16 tile exceeds f16's range, and P is
 * rounded to f16 for the PV product; the scales are exact and taken back
 * out.  For f32 caches the exact f32 decode kernel runs per query.  The
 * context keeps a prefill scratch of about 2*n_kv*head_dim*(pos0+n_tokens)
 * bytes (twice that for bf16), grown on demand. */
void vtb_hip_segment_attn_prefill(VtbHipSeg *seg, VtbHipBuf *out_buf, VtbHipBuf *q_buf,
                                  VtbHipBuf *k_cache_buf, VtbHipBuf *v_cache_buf,
                                  size_t layer_offset_bytes, size_t n_tokens, size_t pos0,
                                  size_t sliding_window, size_t n_heads, size_t n_kv_heads,
                                  size_t head_dim, float inv_sqrt_hd, int dtype);

/* ---- Quantised matrix-vector products: out[i] = sum_j W[i, j] * acts[j] for
 * m rows of k weights stored as GGUF blocks (layouts of src/kernels/simd.zig:
 * Q8_0 34 B / 32 weights, Q4_K 144 B / 256, Q5_K 176 B / 256, Q6_K 210 B / 256),
 * row 0 at w_offset in w_buf; acts f32 [k] (16-byte aligned), out f32 [m].
 * Each weight is dequantised exactly as the CPU reference does; the dot runs
 * in f32 (results agree with the CPU path to ~1e-6 relative; the Metal path's
 * own bar is 1e-4, bridge.zig:466-470).  k a multiple of the block size; the
 * weights 4-byte aligned and below 2 GiB.
 * Segment encoders replace vtb_metal_segment_matmul_{q8_0,q4_k,q5_k,q6_k}
 * (bridge.h:93-113, dispatched by segMatmulQuant, forward.zig:400-417); the
 * vtb_hip_matmul_* forms run synchronously, as vtb_metal_matmul_* do
 * (bridge.h:41-70): 0 on success. */
void vtb_hip_segment_matmul_q8_0(VtbHipSeg *seg, VtbHipBuf *out_buf, VtbHipBuf *w_buf, size_t w_offset,
                                 VtbHipBuf *acts_buf, size_t m, size_t k);
void vtb_hip_segment_matmul_q4_k(VtbHipSeg *seg, VtbHipBuf *out_buf, VtbHipBuf *w_buf, size_t w_offset,
                                 VtbHipBuf *acts_buf, size_t m, size_t k);
void vtb_hip_segment_matmul_q5_k(VtbHipSeg *seg, VtbHipBuf *out_buf, VtbHipBuf *w_buf, size_t w_offset,
                                 VtbHipBuf *acts_buf, size_t m, size_t k);
void vtb_hip_segment_matmul_q6_k(VtbHipSeg *seg, VtbHipBuf *out_buf, VtbHipBuf *w_buf, size_t w_offset,
                                 VtbHipBuf *acts_buf, size_t m, size_t k);
int vtb_hip_matmul_q8_0(VtbHipCtx *ctx, VtbHipBuf *out_buf, VtbHipBuf *w_buf, size_t w_offset,
                        VtbHipBuf *acts_buf, size_t m, size_t k);
int vtb_hip_matmul_q4_k(VtbHipCtx *ctx, VtbHipBuf *out_buf, VtbHipBuf *w_buf, size_t w_offset,
                        VtbHipBuf *acts_buf, size_t m, size_t k);
int vtb_hip_matmul_q5_k(VtbHipCtx *ctx, VtbHipBuf *out_buf, VtbHipBuf *w_buf, size_t w_offset,
                        VtbHipBuf *acts_buf, size_t m, size_t k);
int vtb_hip_matmul_q6_k(VtbHipCtx *ctx, VtbHipBuf *out_buf, VtbHipBuf *w_buf, size_t w_offset,
                        VtbHipBuf *acts_buf, size_t m, size_t k);

/* ---- Batched quantised matmuls (prefill projections): out[b][i] =
 * sum_j W[i, j] * acts[b][j] for B tokens; W as above (m rows of k weights in
 * GGUF blocks at w_offset), acts f32 [B][k] (16-byte aligned), out f32
 * [B][m].  Replace matmulBatched (prefill.zig:325-378, called at :170-226 for
 * the q/k/v/o and FFN projections of a prompt), which dequantises each row
 * (dequantToF32, forward.zig:654-730) and takes simd.dot_f32 with every
 * token.  Computed on MFMA from a two-piece f16 split of each token's acts
 * scaled by a power of two (22 significant bits per activation); products
 * are exact and sums f32 (results agree with the CPU path to ~1e-6 of
 * sum |W||x|).  k a multiple of the block size and at most 32768 (the
 * reference's MAX_K: error 5 above it); weights 4-byte aligned, below 2 GiB.
 * The context keeps a scratch of 4*Bp*k + Bp*k/4 + 4*Bp bytes (Bp = B
 * rounded up to 128), grown on demand.  vtb_hip_matmul_batched_* run synchronously. */
void vtb_hip_segment_matmul_batched_q8_0(VtbHipSeg *seg, VtbHipBuf *out_buf, VtbHipBuf *w_buf, size_t w_offset,
                                         VtbHipBuf *acts_buf, size_t m, size_t k, size_t B);
void vtb_hip_segment_matmul_batched_q4_k(VtbHipSeg *seg, VtbHipBuf *out_buf, VtbHipBuf *w_buf, size_t w_offset,
                                         VtbHipBuf *acts_buf, size_t m, size_t k, size_t B);
void vtb_hip_segment_matmul_batched_q5_k(VtbHipSeg *seg, VtbHipBuf *out_buf, VtbHipBuf *w_buf, size_t w_offset,
                                         VtbHipBuf *acts_buf, size_t m, size_t k, size_t B);
void vtb_hip_segment_matmul_batched_q6_k(VtbHipSeg *seg, VtbHipBuf *out_buf, VtbHipBuf *w_buf, size_t w_offset,
                                         VtbHipBuf *acts_buf, size_t m, size_t k, size_t B);
int vtb_hip_matmul_batched_q8_0(VtbHipCtx *ctx, VtbHipBuf *out_buf, VtbHipBuf *w_buf, size_t w_offset,
                                VtbHipBuf *acts_buf, size_t m, size_t k, size_t B);
int vtb_hip_matmul_batched_q4_k(VtbHipCtx *ctx, VtbHipBuf *out_buf, VtbHipBuf *w_buf, size_t w_offset,
                                VtbHipBuf *acts_buf, size_t m, size_t k, size_t B);
int vtb_hip_matmul_batched_q5_k(VtbHipCtx *ctx, VtbHipBuf *out_buf, VtbHipBuf *w_buf, size_t w_offset,
                                VtbHipBuf *acts_buf, size_t m, size_t k, size_t B);
int vtb_hip_matmul_batched_q6_k(VtbHipCtx *ctx, VtbHipBuf *out_buf, VtbHipBuf *w_buf, size_t w_offset,
                                VtbHipBuf *acts_buf, size_t m, size_t k, size_t B);

/* ---- KvCache, device-handle mode (kv_cache.zig:20-196).  Layer-major
 * [n_layers][max_seq][n_kv_heads][head_dim] of dtype in HBM; no host slices. */
VtbHipKvCache *vtb_hip_kv_cache_init(VtbHipCtx *ctx, size_t n_layers, size_t n_kv_heads,
                                     size_t head_dim, size_t max_seq, int dtype); /* :33-73 */
void vtb_hip_kv_cache_deinit(VtbHipKvCache *cache);                              /* :75-81 */
void vtb_hip_kv_cache_reset(VtbHipKvCache *cache);                               /* :83-85 */
size_t vtb_hip_kv_cache_pos(const VtbHipKvCache *cache);
/* Set pos directly (tests and prefill's `cache.pos += B`, prefill.zig:141). */
int vtb_hip_kv_cache_set_pos(VtbHipKvCache *cache, size_t pos);
size_t vtb_hip_kv_cache_max_seq(const VtbHipKvCache *cache);
int vtb_hip_kv_cache_dtype(const VtbHipKvCache *cache);
int vtb_hip_kv_cache_advance(VtbHipKvCache *cache);                              /* :130-133 */
/* Byte offset of the slot at pos in layer (keySlot/valueSlot, :97-111);
 * (size_t)-1 where the reference asserts. */
size_t vtb_hip_kv_cache_slot_offset(const VtbHipKvCache *cache, size_t layer);
/* Byte offset of row 0 of layer (keysFor/valuesFor, :116-128). */
size_t vtb_hip_kv_cache_layer_offset(const VtbHipKvCache *cache, size_t layer);
VtbHipBuf *vtb_hip_kv_cache_k(VtbHipKvCache *cache);
VtbHipBuf *vtb_hip_kv_cache_v(VtbHipKvCache *cache);
/* :147-195.  Compacts every layer's live prefix into a new allocation of
 * new_max_seq rows per layer and frees the old one (the HBM tail is returned,
 * unlike the Metal path).  0, or 4 if new_max_seq < pos. */
int vtb_hip_kv_cache_shrink_to_fit(VtbHipKvCache *cache, size_t new_max_seq);

/* ---- scratch reservation: the counterpart of prefill.zig Scratch.init
 * (prefill.zig:67-88), which sizes the batch scratch for B tokens and the
 * score rows for max_seq once, before the first forward.  Grows, once, every
 * buffer the context otherwise grows on demand (which drains the stream and
 * calls hipMalloc inside the call that needs it): the split-K decode
 * workspace and counters for one query (and, on f32 caches, whose prefill
 * runs the decode kernel, up to max_batch queries) over up to c->max_seq
 * keys or the window; the prefill conversion scratch for a c->max_seq-key
 * context (f16/bf16 caches, max_batch > 0); the batched-matmul activation
 * scratch for max_batch tokens of width max_matmul_k (0: none); the RoPE
 * table of rope_base (0: none).  Later calls within these bounds allocate
 * nothing.  Waits for the stream.  5 if a bound is beyond what the kernels
 * take (max_batch > max_seq, max_matmul_k > 32768). */
int vtb_hip_reserve(VtbHipCtx *ctx, const VtbHipAttnConfig *c, int kv_dtype, size_t max_batch,
                    size_t max_matmul_k, float rope_base);
/* Bytes of device scratch ctx holds: unchanged by calls that needed no
 * growth. */
size_t vtb_hip_scratch_bytes(VtbHipCtx *ctx);

/* ---- Layer-level entries mirroring the reference call sites.
 *
 * Decode, one layer (forward.zig:267-270 then cpuAttention :187-228): write
 * k_cur/v_cur (f32 [n_kv_heads*head_dim]) into the slot at cache->pos, then
 * attend [window_start(pos), pos] with q (f32 [n_heads*head_dim]) into
 * attn_out (f32), in one launch (the slot write is fused into the decode
 * kernel).  Does not advance pos (stepWithBackend advances once after
 * all layers, forward.zig:168).  3 if pos >= max_seq. */
int vtb_hip_layer_attention(VtbHipSeg *seg, VtbHipKvCache *cache, const VtbHipAttnConfig *c,
                            size_t layer, VtbHipBuf *q, VtbHipBuf *k_cur, VtbHipBuf *v_cur,
                            VtbHipBuf *attn_out);

/* vtb_hip_layer_attention with the layer's RoPE fused in: the whole of
 * forward.zig:250-270 -- math.rope / math.ropeHalf (rope_half, LlamaConfig
 * .rope_half, model.zig:57) of q per head and of k_cur per KV head at
 * cache->pos with rope_base (LlamaConfig.rope_base, model.zig:50), the slot
 * write, cpuAttention -- in one launch.  q and k_cur are not modified. */
int vtb_hip_layer_attention_rope(VtbHipSeg *seg, VtbHipKvCache *cache, const VtbHipAttnConfig *c,
                                 size_t layer, VtbHipBuf *q, VtbHipBuf *k_cur, VtbHipBuf *v_cur,
                                 VtbHipBuf *attn_out, float rope_base, int rope_half);

/* Prefill, one layer (prefill.zig:174-197): write the n_tokens rows of
 * k_cur/v_cur (f32 [n_tokens][kv_dim]) into slots pos..pos+n_tokens-1, then
 * causal attention for every query (q f32 [n_tokens][n_heads*head_dim]) into
 * attn_out, exactly as vtb_hip_segment_attn_prefill computes it.  Does not
 * advance pos.  3 if pos + n_tokens > max_seq. */
int vtb_hip_prefill_attention(VtbHipSeg *seg, VtbHipKvCache *cache, const VtbHipAttnConfig *c,
                              size_t layer, size_t n_tokens, VtbHipBuf *q, VtbHipBuf *k_cur,
                              VtbHipBuf *v_cur, VtbHipBuf *attn_out);

#ifdef __cplusplus
}
#endif

#endif /* VTB_HIP_H */
