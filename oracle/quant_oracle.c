/* CPU restatement of vantablack's quantised matmuls (TEST INFRASTRUCTURE ONLY:
 * loaded by tests/ and never by the product path).
 *
 * Follows src/kernels/simd.zig:
 *   Q8_0  block = { f16 d; i8 qs[32] }                      :145-190
 *   Q4_K  block = { f16 d, dmin; u8 scales[12]; u8 qs[128] } :192-273
 *   Q5_K  block = Q4_K + u8 qh[32] before qs                 :275-347
 *   Q6_K  block = { u8 ql[128], qh[64]; i8 sc[16]; f16 d }   :349-433
 * Dequantisation keeps the reference's f32 products in the same order (no
 * contraction: -ffp-contract=off).  The matmuls keep its structure: Q8_0 sums
 * four 8-wide chunk reductions per block and scales the block sum; the K-quants
 * dequantise a block, accumulate 8 lanes over it and add the lane reduction
 * to the row total.  The order inside a Zig @reduce(.Add) is not specified by
 * the language; it is taken as lane order here (parity unpinned at the ULP
 * level only; the GPU bar is 1e-4 relative, bridge.zig:466-470). */
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>

float vtb_oracle_f16_to_f32(uint16_t h); /* attn_oracle.c */

enum { VTB_Q8_0 = 0, VTB_Q4_K = 1, VTB_Q5_K = 2, VTB_Q6_K = 3 };

static const size_t block_bytes[4] = {34, 144, 176, 210};
static const size_t block_elems[4] = {32, 256, 256, 256};

size_t vtb_oracle_quant_block_bytes(int kind) { return (kind >= 0 && kind < 4) ? block_bytes[kind] : 0; }
size_t vtb_oracle_quant_block_elems(int kind) { return (kind >= 0 && kind < 4) ? block_elems[kind] : 0; }

static float f16_at(const uint8_t *p) { return vtb_oracle_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* simd.zig:153-157 */
static void dequant_q8_0(const uint8_t *blk, float *out) {
    const float scale = f16_at(blk);
    for (int j = 0; j < 32; j++) out[j] = scale * (float)(int8_t)blk[2 + j];
}

/* simd.zig:211-219 (q4kScaleMin): 6-bit scale and min of sub-block s. */
static void scale_min_k4(int s, const uint8_t *scales, uint8_t *sc, uint8_t *mn) {
    if (s < 4) {
        *sc = scales[s] & 0x3F;
        *mn = scales[s + 4] & 0x3F;
    } else {
        *sc = (uint8_t)((scales[s + 4] & 0x0F) | ((scales[s - 4] >> 6) << 4));
        *mn = (uint8_t)((scales[s + 4] >> 4) | ((scales[s] >> 6) << 4));
    }
}

/* simd.zig:221-243 (Q4_K) and :290-317 (Q5_K: qh supplies the fifth bit). */
static void dequant_q45_k(const uint8_t *blk, float *out, int five) {
    const float d = f16_at(blk), dmin = f16_at(blk + 2);
    const uint8_t *scales = blk + 4;
    const uint8_t *qh = blk + 16;
    const uint8_t *qs = blk + (five ? 48 : 16);
    int y = 0;
    for (int s = 0; s < 8; s += 2) {
        uint8_t sa, ma, sb, mb;
        scale_min_k4(s, scales, &sa, &ma);
        scale_min_k4(s + 1, scales, &sb, &mb);
        const float d1 = d * (float)sa, m1 = dmin * (float)ma;
        const float d2 = d * (float)sb, m2 = dmin * (float)mb;
        const uint8_t *q = qs + (s / 2) * 32;
        for (int l = 0; l < 32; l++) {
            unsigned w0 = q[l] & 0x0F, w1 = q[l] >> 4;
            if (five) {
                w0 += (qh[l] & (1u << s)) ? 16u : 0u;
                w1 += (qh[l] & (1u << (s + 1))) ? 16u : 0u;
            }
            out[y + l] = d1 * (float)w0 - m1;
            out[y + 32 + l] = d2 * (float)w1 - m2;
        }
        y += 64;
    }
}

/* simd.zig:366-404: two halves of 128; for l < 32 four weights at l, l+32,
 * l+64, l+96 from ql/qh, biased by -32, scaled by d * sc[is + {0,2,4,6}]. */
static void dequant_q6_k(const uint8_t *blk, float *out) {
    const float d = f16_at(blk + 208);
    const uint8_t *ql = blk, *qh = blk + 128;
    const int8_t *sc = (const int8_t *)(blk + 192);
    for (int half = 0; half < 2; half++) {
        const uint8_t *qlh = ql + 64 * half, *qhh = qh + 32 * half;
        const int8_t *sch = sc + 8 * half;
        float *y = out + 128 * half;
        for (int l = 0; l < 32; l++) {
            const int is = l / 16;
            const int q1 = (int)((qlh[l] & 0x0F) | (((qhh[l] >> 0) & 3) << 4)) - 32;
            const int q2 = (int)((qlh[l + 32] & 0x0F) | (((qhh[l] >> 2) & 3) << 4)) - 32;
            const int q3 = (int)((qlh[l] >> 4) | (((qhh[l] >> 4) & 3) << 4)) - 32;
            const int q4 = (int)((qlh[l + 32] >> 4) | (((qhh[l] >> 6) & 3) << 4)) - 32;
            y[l] = d * (float)sch[is + 0] * (float)q1;
            y[l + 32] = d * (float)sch[is + 2] * (float)q2;
            y[l + 64] = d * (float)sch[is + 4] * (float)q3;
            y[l + 96] = d * (float)sch[is + 6] * (float)q4;
        }
    }
}

/* One block of `kind` -> block_elems f32.  0, or -1 for an unknown kind. */
int vtb_oracle_dequant_block(int kind, const uint8_t *blk, float *out) {
    switch (kind) {
    case VTB_Q8_0: dequant_q8_0(blk, out); return 0;
    case VTB_Q4_K: dequant_q45_k(blk, out, 0); return 0;
    case VTB_Q5_K: dequant_q45_k(blk, out, 1); return 0;
    case VTB_Q6_K: dequant_q6_k(blk, out); return 0;
    default: return -1;
    }
}

static float reduce8(const float *v) {
    float s = v[0];
    for (int i = 1; i < 8; i++) s += v[i];
    return s;
}

/* out[i] = row i of W (m rows of k/block_elems blocks) . acts[0..k).
 * simd.zig:159-190 (Q8_0), :245-273 / :319-347 / :406-433 (K-quants).
 * 0, or -1 if k is not a whole number of blocks / kind is unknown. */
int vtb_oracle_matmul_quant(int kind, float *out, const uint8_t *w, const float *acts, size_t m, size_t k) {
    if (kind < 0 || kind > 3 || k % block_elems[kind] != 0) return -1;
    const size_t be = block_elems[kind], bb = block_bytes[kind];
    const size_t nb = k / be, row_bytes = nb * bb;
    float dq[256];
    for (size_t i = 0; i < m; i++) {
        const uint8_t *row = w + i * row_bytes;
        float total = 0.0f;
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *blk = row + b * bb;
            const float *x = acts + b * be;
            if (kind == VTB_Q8_0) {
                const float scale = f16_at(blk);
                float block_dot = 0.0f;
                for (int chunk = 0; chunk < 4; chunk++) {
                    float p[8];
                    for (int li = 0; li < 8; li++)
                        p[li] = (float)(int8_t)blk[2 + chunk * 8 + li] * x[chunk * 8 + li];
                    block_dot += reduce8(p);
                }
                total += scale * block_dot;
            } else {
                vtb_oracle_dequant_block(kind, blk, dq);
                float acc[8] = {0};
                for (size_t j = 0; j < be; j += 8)
                    for (int li = 0; li < 8; li++) acc[li] += dq[j + li] * x[j + li];
                total += reduce8(acc);
            }
        }
        out[i] = total;
    }
    return 0;
}

/* simd.zig:13-29 (dot_f32): eight lane accumulators over the whole length,
 * each product rounded then added (no contraction), reduced in lane order,
 * then the tail (none for whole blocks). */
static float dot_f32(const float *a, const float *b, size_t n) {
    float acc[8] = {0};
    size_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++) acc[l] += a[i + l] * b[i + l];
    float sum = reduce8(acc);
    for (; i < n; i++) sum += a[i] * b[i];
    return sum;
}

/* prefill.zig:325-378 (matmulBatched / matmulBatchedWorker): for each weight
 * row, dequantise the whole row (forward.zig:654-730 dequantToF32, block by
 * block) and take dot_f32 with every token's activations:
 *   out[b*m + row] = dot_f32(dequant(W[row]), acts[b*k .. b*k + k]).
 * 0, or -1 for an unknown kind, k not a whole number of blocks or k above
 * the reference's MAX_K of 32768 (which returns DimTooLarge). */
int vtb_oracle_matmul_batched(int kind, float *out, const uint8_t *w, const float *acts, size_t m, size_t k,
                              size_t B) {
    if (kind < 0 || kind > 3 || k % block_elems[kind] != 0 || k > 32768) return -1;
    const size_t be = block_elems[kind], bb = block_bytes[kind];
    const size_t nb = k / be, row_bytes = nb * bb;
    float *dq = (float *)malloc(k * sizeof(float));
    if (!dq) return -1;
    for (size_t row = 0; row < m; row++) {
        for (size_t b = 0; b < nb; b++) vtb_oracle_dequant_block(kind, w + row * row_bytes + b * bb, dq + b * be);
        for (size_t t = 0; t < B; t++) out[t * m + row] = dot_f32(dq, acts + t * k, k);
    }
    free(dq);
    return 0;
}
