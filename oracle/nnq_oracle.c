/*
 * CPU oracle for the quantized-linear hot path — TEST INFRASTRUCTURE ONLY.
 *
 * Restates, in plain C, the reference's (alabsystems/nn) CPU arithmetic for the
 * dequant-fused matmul path.  Each function cites the Rust source it follows
 * (paths relative to the reference repository root).  This file is the checker
 * for the HIP product path and the timed CPU baseline; the product never links
 * or calls it.
 *
 * Build: see oracle/Makefile (-O2 -ffp-contract=off, no fast-math).
 */
#include "nnq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------------ */
/* half-precision conversions.  The reference uses the `half` 2.x crate      */
/* (Cargo.toml:151): f16->f32 is exact widening, f32->f16 is IEEE 754        */
/* round-to-nearest-even with overflow to infinity and quiet NaNs.           */
/* ------------------------------------------------------------------------ */

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    if (exp == 0) {
        /* zero or subnormal: man * 2^-24, exact in binary32 */
        float v = (float)man * 5.9604644775390625e-8f;
        return u2f(f2u(v) | sign);
    }
    if (exp == 31) {
        if (man == 0) return u2f(sign | 0x7F800000u);
        return u2f(sign | 0x7FC00000u | (man << 13));
    }
    return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t orc_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) {
        if (ax == 0x7F800000u) return sign | 0x7C00u;
        return (uint16_t)(sign | 0x7E00u | ((ax & 0x7FFFFFu) >> 13));
    }
    int e = (int)(ax >> 23) - 127;
    uint32_t mant = ax & 0x7FFFFFu;
    if (e >= -14) {
        if (e > 15) return sign | 0x7C00u;
        uint32_t half = ((uint32_t)(e + 15) << 10) | (mant >> 13);
        uint32_t rem = mant & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half += 1u; /* may carry into inf */
        return (uint16_t)(sign | half);
    }
    /* f16 subnormal (or underflow to zero); f32 subnormals are < 2^-126 and round to 0 */
    if (ax < 0x00800000u) return sign;
    uint32_t m = mant | 0x800000u;       /* value = m * 2^(e-23) = m * 2^(e+1) units of 2^-24 */
    int shift = -(e + 1);                /* >= 14 */
    if (shift > 24) return sign;
    uint32_t half = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (half & 1u))) half += 1u;
    return (uint16_t)(sign | half);
}

float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t orc_f32_to_bf16(float f) {
    uint32_t x = f2u(f);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x0040u);
    uint32_t lsb = (x >> 16) & 1u;
    return (uint16_t)((x + 0x7FFFu + lsb) >> 16);
}

void orc_f16_to_f32_array(const uint16_t *in, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f16_to_f32(in[i]);
}
void orc_f32_to_f16_array(const float *in, size_t n, uint16_t *out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f32_to_f16(in[i]);
}
void orc_f32_to_bf16_array(const float *in, size_t n, uint16_t *out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f32_to_bf16(in[i]);
}

static inline float ld_f16(const uint8_t *p) { return orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* validate_dequant_input: crates/nn-gguf/src/dequant.rs:123-139 — a short
 * buffer clamps the number of decoded blocks instead of failing. */
static size_t clamp_blocks(size_t nbytes, size_t num_elements, size_t bs, size_t bpb) {
    size_t nb = num_elements / bs;
    if (nbytes < nb * bpb) return nbytes / bpb;
    return nb;
}

/* ------------------------------------------------------------------------ */
/* Q8_0                                                                      */
/* ------------------------------------------------------------------------ */

/* dequantize_q8_0: crates/nn-core/src/dyn_tensor/quantized.rs:237-253 and
 * crates/nn-gguf/src/dequant.rs:178-196.  v = f32(d) * f32(q). */
size_t orc_dequant_q8_0(const uint8_t *data, size_t nbytes, size_t num_elements, float *out) {
    size_t nb = clamp_blocks(nbytes, num_elements, 32, 34);
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *p = data + b * 34;
        float scale = ld_f16(p);
        for (int j = 0; j < 32; j++) out[b * 32 + j] = scale * (float)(int8_t)p[2 + j];
    }
    return nb * 32;
}

/* quantized_matmul_core -> quantized_dot_row -> dot_q8_0_block:
 * crates/nn-core/src/dyn_tensor/quantized_matmul.rs:173-187, 191-220, 232-272.
 * Per block: acc_b = sum_{j=0..31} x * (d * q) sequentially from 0; the row
 * accumulates the block sums sequentially.  `rows` is batch*M (rank folding). */
int orc_q8_0_matmul(const float *x, size_t rows, size_t k, const uint8_t *w, size_t n, float *y) {
    if (k % 32) return -1;
    size_t nblk = k / 32;
    for (size_t r = 0; r < rows; r++) {
        const float *xr = x + r * k;
        for (size_t oc = 0; oc < n; oc++) {
            const uint8_t *wr = w + oc * nblk * 34;
            float acc = 0.0f;
            for (size_t b = 0; b < nblk; b++) {
                const uint8_t *p = wr + b * 34;
                float scale = ld_f16(p);
                float bacc = 0.0f;
                for (int j = 0; j < 32; j++) {
                    float wv = scale * (float)(int8_t)p[2 + j];
                    float prod = xr[b * 32 + j] * wv;
                    bacc = bacc + prod;
                }
                acc = acc + bacc;
            }
            y[r * n + oc] = acc;
        }
    }
    return 0;
}

/* Q8_0 encoder.  The reference ships none (its tests hand-build blocks,
 * crates/nn-core/src/dyn_tensor/quantized_matmul_tests.rs:37-46); this is the
 * build-defined input generator: d = amax/127 stored as f16, q = round(v/d). */
void orc_quantize_q8_0(const float *v, size_t n, uint8_t *out) {
    size_t nb = n / 32;
    for (size_t b = 0; b < nb; b++) {
        const float *x = v + b * 32;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) {
            float a = fabsf(x[j]);
            if (a > amax) amax = a;
        }
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint16_t dh = orc_f32_to_f16(d);
        uint8_t *p = out + b * 34;
        p[0] = (uint8_t)(dh & 0xFF);
        p[1] = (uint8_t)(dh >> 8);
        for (int j = 0; j < 32; j++) {
            float q = roundf(x[j] * id);
            if (q > 127.0f) q = 127.0f;
            if (q < -127.0f) q = -127.0f;
            p[2 + j] = (uint8_t)(int8_t)q;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Q4_K, GGUF-spec layout (nn-core BlockQ4K)                                 */
/* ------------------------------------------------------------------------ */

/* get_scale_min_k4: crates/nn-core/src/layers/quantized/linear.rs:166-176 */
void orc_q4k_get_scale_min(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* BlockQ4K::dequantize: crates/nn-core/src/layers/quantized/linear.rs:63-92.
 * Block bytes: d u16 | dmin u16 | scales[12] | qs[128] (repr(C), :49-56). */
void orc_q4k_dequant_block(const uint8_t *blk, float *out) {
    float d = ld_f16(blk);
    float dmin = ld_f16(blk + 2);
    const uint8_t *scales = blk + 4;
    const uint8_t *qs = blk + 16;
    int oi = 0;
    for (int j = 0; j < 256; j += 64) {
        int q_off = j / 2;
        int is = j / 32;
        uint8_t sc1, mm1, sc2, mm2;
        orc_q4k_get_scale_min(is, scales, &sc1, &mm1);
        float d1 = d * (float)sc1;
        float m1 = dmin * (float)mm1;
        orc_q4k_get_scale_min(is + 1, scales, &sc2, &mm2);
        float d2 = d * (float)sc2;
        float m2 = dmin * (float)mm2;
        for (int i = 0; i < 32; i++) {
            float t = d1 * (float)(qs[q_off + i] & 0xF);
            out[oi++] = t - m1;
        }
        for (int i = 0; i < 32; i++) {
            float t = d2 * (float)(qs[q_off + i] >> 4);
            out[oi++] = t - m2;
        }
    }
}

/* QuantizedWeight::dequantize_to_f32: crates/nn-core/src/layers/quantized/linear.rs:268-281
 * (block after block; the storage is validated, the clamp only guards callers). */
size_t orc_dequant_q4_k_gguf(const uint8_t *data, size_t nbytes, size_t num_elements, float *out) {
    size_t nb = clamp_blocks(nbytes, num_elements, 256, 144);
    for (size_t b = 0; b < nb; b++) orc_q4k_dequant_block(data + b * 144, out + b * 256);
    return nb * 256;
}

/* dequantize_q4_k (nn-gguf layout): crates/nn-gguf/src/dequant.rs:335-398.
 * Different scale packing and lo/hi nibble interleave from BlockQ4K. */
size_t orc_dequant_q4_k_legacy(const uint8_t *data, size_t nbytes, size_t num_elements, float *out) {
    size_t nb = clamp_blocks(nbytes, num_elements, 256, 144);
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *p = data + b * 144;
        float d = ld_f16(p);
        float dmin = ld_f16(p + 2);
        const uint8_t *sd = p + 4;
        uint8_t scales[8], mins[8];
        for (int j = 0; j < 8; j++) scales[j] = (uint8_t)((sd[j / 2] >> (4 * (j % 2))) & 0x0F);
        for (int j = 0; j < 8; j++) mins[j] = (uint8_t)((sd[4 + j / 2] >> (4 * (j % 2))) & 0x0F);
        for (int j = 0; j < 4; j++) scales[j] |= (uint8_t)(((sd[8] >> (2 * j)) & 3) << 4);
        for (int j = 0; j < 4; j++) scales[4 + j] |= (uint8_t)(((sd[9] >> (2 * j)) & 3) << 4);
        for (int j = 0; j < 4; j++) mins[j] |= (uint8_t)(((sd[10] >> (2 * j)) & 3) << 4);
        for (int j = 0; j < 4; j++) mins[4 + j] |= (uint8_t)(((sd[11] >> (2 * j)) & 3) << 4);
        const uint8_t *qs = p + 16;
        float *o = out + b * 256;
        for (int j = 0; j < 8; j++) {
            float sc = d * (float)scales[j];
            float m = dmin * (float)mins[j];
            for (int i = 0; i < 16; i++) {
                uint8_t byte = qs[j * 16 + i];
                float lo = (float)(byte & 0x0F);
                float hi = (float)((byte >> 4) & 0x0F);
                float a = sc * lo;
                float c = sc * hi;
                o[j * 32 + 2 * i] = a - m;
                o[j * 32 + 2 * i + 1] = c - m;
            }
        }
    }
    return nb * 256;
}

/* nearest_int: crates/nn-core/src/layers/quantized/linear.rs:179-192.
 * f32::round (half away from zero); non-finite or out-of-i32 -> error (-1).
 * `r as i32` saturates at i32::MAX for r == 2^31. */
int orc_q4k_nearest_int(float v, int32_t *out) {
    if (!isfinite(v)) return -1;
    float r = roundf(v);
    if (r < -2147483648.0f || r > 2147483648.0f) return -1;
    if (r >= 2147483648.0f) *out = 2147483647;
    else *out = (int32_t)r;
    return 0;
}

/* f32::min / f32::max ignore a NaN operand (IEEE minNum/maxNum) like fminf/fmaxf. */

/* make_qkx1_quants: crates/nn-core/src/layers/quantized/linear.rs:195-254.
 * Returns (scale, -min) through *scale / *neg_min. */
int orc_q4k_make_qkx1_quants(int nmax, int ntry, const float *x, size_t n, float *scale_out, float *neg_min) {
    uint8_t l[256];
    if (n > 256) return -1;
    memset(l, 0, n);
    float mn = INFINITY, mx = -INFINITY;
    for (size_t i = 0; i < n; i++) mn = fminf(mn, x[i]);
    for (size_t i = 0; i < n; i++) mx = fmaxf(mx, x[i]);
    if (mx == mn) {
        float c = mn;
        if (c >= 0.0f) {
            *scale_out = nmax > 0 ? c / (float)nmax : 0.0f;
            *neg_min = 0.0f;
        } else {
            *scale_out = 0.0f;
            *neg_min = -c;
        }
        return 0;
    }
    float min = fminf(mn, 0.0f);
    float iscale = (float)nmax / (mx - min);
    float scale = 1.0f / iscale;
    for (int it = 0; it < ntry; it++) {
        float sumlx = 0.0f;
        int32_t suml2 = 0;
        int did_change = 0;
        for (size_t i = 0; i < n; i++) {
            int32_t li;
            if (orc_q4k_nearest_int(iscale * (x[i] - min), &li)) return -1;
            if (li < 0) li = 0;
            if (li > nmax) li = nmax;
            if ((uint8_t)li != l[i]) {
                l[i] = (uint8_t)li;
                did_change = 1;
            }
            float t = (x[i] - min) * (float)(uint8_t)li;
            sumlx = sumlx + t;
            suml2 += li * li;
        }
        if (suml2 == 0) {
            *scale_out = 0.0f;
            *neg_min = 0.0f;
            return 0;
        }
        scale = sumlx / (float)suml2;
        if (scale == 0.0f) {
            *scale_out = 0.0f;
            *neg_min = -min;
            return 0;
        }
        /* Iterator::sum over f32 (sequential) */
        float sum = -0.0f;
        for (size_t i = 0; i < n; i++) {
            float t = scale * (float)l[i];
            sum = sum + (x[i] - t);
        }
        min = fminf(sum / (float)n, 0.0f);
        iscale = 1.0f / scale;
        if (!did_change) break;
    }
    *scale_out = scale;
    *neg_min = -min;
    return 0;
}

/* BlockQ4K::quantize: crates/nn-core/src/layers/quantized/linear.rs:95-162 */
int orc_quantize_q4_k_block(const float *v, uint8_t *blk) {
    float sub_scales[8], sub_mins[8];
    uint8_t scales[12];
    uint8_t qs[128];
    memset(scales, 0, sizeof scales);
    memset(qs, 0, sizeof qs);
    for (int j = 0; j < 8; j++)
        if (orc_q4k_make_qkx1_quants(15, 5, v + 32 * j, 32, &sub_scales[j], &sub_mins[j])) return -1;
    float max_scale = 0.0f, max_min = 0.0f;
    for (int j = 0; j < 8; j++) max_scale = fmaxf(max_scale, sub_scales[j]);
    for (int j = 0; j < 8; j++) max_min = fmaxf(max_min, sub_mins[j]);
    float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
    float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
    for (int j = 0; j < 8; j++) {
        int32_t a, b;
        if (orc_q4k_nearest_int(inv_scale * sub_scales[j], &a)) return -1;
        if (orc_q4k_nearest_int(inv_min * sub_mins[j], &b)) return -1;
        uint8_t ls = (uint8_t)a;
        uint8_t lm = (uint8_t)b;
        if (ls > 63) ls = 63;
        if (lm > 63) lm = 63;
        if (j < 4) {
            scales[j] = ls;
            scales[j + 4] = lm;
        } else {
            scales[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
            scales[j - 4] |= (uint8_t)((ls >> 4) << 6);
            scales[j] |= (uint8_t)((lm >> 4) << 6);
        }
    }
    uint16_t d = orc_f32_to_f16(max_scale / 63.0f);
    uint16_t dmin = orc_f32_to_f16(max_min / 63.0f);
    uint8_t l[256];
    memset(l, 0, sizeof l);
    for (int j = 0; j < 8; j++) {
        uint8_t sc, m;
        orc_q4k_get_scale_min(j, scales, &sc, &m);
        float bd = orc_f16_to_f32(d) * (float)sc;
        if (bd != 0.0f) {
            float bm = orc_f16_to_f32(dmin) * (float)m;
            for (int ii = 0; ii < 32; ii++) {
                int32_t q;
                if (orc_q4k_nearest_int((v[32 * j + ii] + bm) / bd, &q)) return -1;
                if (q < 0) q = 0;
                if (q > 15) q = 15;
                l[32 * j + ii] = (uint8_t)q;
            }
        }
    }
    for (int j = 0; j < 256; j += 64)
        for (int k = 0; k < 32; k++) qs[j / 2 + k] = (uint8_t)(l[j + k] | (l[j + k + 32] << 4));
    blk[0] = (uint8_t)(d & 0xFF);
    blk[1] = (uint8_t)(d >> 8);
    blk[2] = (uint8_t)(dmin & 0xFF);
    blk[3] = (uint8_t)(dmin >> 8);
    memcpy(blk + 4, scales, 12);
    memcpy(blk + 16, qs, 128);
    return 0;
}

/* QLinear::from_linear(Q4K): crates/nn-core/src/layers/quantized/linear.rs:309-346 —
 * flatten, zero-pad to a multiple of 256, quantize block by block. */
int orc_quantize_q4_k(const float *v, size_t n_total, uint8_t *out) {
    size_t nb = (n_total + 255) / 256;
    float buf[256];
    for (size_t b = 0; b < nb; b++) {
        size_t base = b * 256;
        size_t cnt = n_total - base < 256 ? n_total - base : 256;
        memcpy(buf, v + base, cnt * sizeof(float));
        for (size_t i = cnt; i < 256; i++) buf[i] = 0.0f;
        if (orc_quantize_q4_k_block(buf, out + b * 144)) return -1;
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Q6_K, nn-gguf layout                                                      */
/* ------------------------------------------------------------------------ */

/* dequantize_q6_k: crates/nn-gguf/src/dequant.rs:415-459.
 * ql[128] | qh[64] | scales[16] i8 | d f16 @208; element idx:
 * lo4 = nibble idx of ql, hi2 = crumb idx of qh, v = (d * sc[idx/16]) * (q6 - 32). */
size_t orc_dequant_q6_k_legacy(const uint8_t *data, size_t nbytes, size_t num_elements, float *out) {
    size_t nb = clamp_blocks(nbytes, num_elements, 256, 210);
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *p = data + b * 210;
        const uint8_t *ql = p;
        const uint8_t *qh = p + 128;
        const uint8_t *sc = p + 192;
        float d = ld_f16(p + 208);
        for (int sub = 0; sub < 16; sub++) {
            float s = (float)(int8_t)sc[sub];
            for (int kk = 0; kk < 16; kk++) {
                int idx = sub * 16 + kk;
                uint8_t qlb = ql[idx / 2];
                uint8_t lo4 = (idx % 2 == 0) ? (qlb & 0x0F) : ((qlb >> 4) & 0x0F);
                uint8_t hi2 = (qh[idx / 4] >> ((idx % 4) * 2)) & 0x03;
                int q6 = lo4 | (hi2 << 4);
                float ds = d * s;
                out[b * 256 + idx] = ds * (float)(q6 - 32);
            }
        }
    }
    return nb * 256;
}

/* Q6_K encoder for the nn-gguf layout.  The reference has none (its tests hand-build blocks);
 * build-defined: per 16-value sub-block scale amax/31, d = f16(max/127),
 * int8 sub-scales, q6 = clamp(round(v / (d*sc)), -32, 31) + 32. */
void orc_quantize_q6_k_legacy(const float *v, size_t n, uint8_t *out) {
    size_t nb = n / 256;
    for (size_t b = 0; b < nb; b++) {
        const float *x = v + b * 256;
        uint8_t *p = out + b * 210;
        memset(p, 0, 210);
        float sub_scale[16];
        float maxs = 0.0f;
        for (int s = 0; s < 16; s++) {
            float amax = 0.0f;
            for (int k = 0; k < 16; k++) {
                float a = fabsf(x[s * 16 + k]);
                if (a > amax) amax = a;
            }
            sub_scale[s] = amax / 31.0f;
            if (sub_scale[s] > maxs) maxs = sub_scale[s];
        }
        uint16_t dh = orc_f32_to_f16(maxs / 127.0f);
        float df = orc_f16_to_f32(dh);
        p[208] = (uint8_t)(dh & 0xFF);
        p[209] = (uint8_t)(dh >> 8);
        for (int s = 0; s < 16; s++) {
            float scf = df > 0.0f ? roundf(sub_scale[s] / df) : 0.0f;
            if (scf > 127.0f) scf = 127.0f;
            int8_t sc = (int8_t)scf;
            p[192 + s] = (uint8_t)sc;
            float eff = df * (float)sc;
            for (int k = 0; k < 16; k++) {
                int idx = s * 16 + k;
                int q = 32;
                if (eff != 0.0f) {
                    float r = roundf(x[idx] / eff);
                    if (r < -32.0f) r = -32.0f;
                    if (r > 31.0f) r = 31.0f;
                    q = (int)r + 32;
                }
                p[idx / 2] |= (uint8_t)((q & 0x0F) << (4 * (idx % 2)));
                p[128 + idx / 4] |= (uint8_t)(((q >> 4) & 0x03) << (2 * (idx % 4)));
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* GPT-OSS MXFP4 (crates/nn-gptoss/src/quantize.rs)                         */
/* ------------------------------------------------------------------------ */

/* FP4_LUT: crates/nn-gptoss/src/quantize.rs:28-45 */
static const float FP4_LUT[16] = {0.0f,  0.5f,  1.0f,  1.5f,  2.0f,  3.0f,  4.0f,  6.0f,
                                  -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};
static const float FP4_ABS[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};

float orc_mxfp4_lut(int code) { return FP4_LUT[code & 15]; }

/* compute_e8m0_scale: crates/nn-gptoss/src/quantize.rs:68-81 */
uint8_t orc_mxfp4_e8m0_from_max(float max_abs) {
    if (!isfinite(max_abs) || max_abs <= 0.0f) return 0;
    uint32_t bits = f2u(max_abs);
    uint8_t be = (uint8_t)((bits >> 23) & 0xFF);
    if (be == 0) return 0;
    uint8_t se = be >= 2 ? (uint8_t)(be - 2) : 0;
    return se < 254 ? se : 254;
}

/* decode_e8m0_scale: crates/nn-gptoss/src/quantize.rs:84-90 (byte 0 -> 2^-126) */
float orc_mxfp4_decode_e8m0(uint8_t e) {
    if (e == 0) return u2f(0x00800000u);
    return u2f((uint32_t)e << 23);
}

/* quantize_to_fp4: crates/nn-gptoss/src/quantize.rs:93-116 (strict `<`: ties keep
 * the lower magnitude; non-finite -> code 0) */
uint8_t orc_mxfp4_quantize_fp4(float val, float scale) {
    if (!isfinite(val) || scale <= 0.0f) return 0;
    int sign = val < 0.0f;
    float a = fabsf(val) / scale;
    int best = 0;
    float bestd = 3.40282347e+38f;
    for (int i = 0; i < 8; i++) {
        float dd = fabsf(a - FP4_ABS[i]);
        if (dd < bestd) {
            bestd = dd;
            best = i;
        }
    }
    return (uint8_t)(sign ? (best | 8) : best);
}

/* Mxfp4Tensor::quantize: crates/nn-gptoss/src/quantize.rs:122-163.
 * Pair p of a block: HIGH nibble = element 2p, LOW nibble = element 2p+1. */
void orc_mxfp4_quantize(const float *data, size_t n, uint8_t *packed, uint8_t *scales) {
    size_t nb = (n + 31) / 32;
    for (size_t b = 0; b < nb; b++) {
        size_t start = b * 32;
        float max_abs = 0.0f;
        for (int i = 0; i < 32; i++) {
            size_t idx = start + i;
            float val = idx < n ? data[idx] : 0.0f;
            float a = fabsf(val);
            if (isfinite(a) && a > max_abs) max_abs = a;
        }
        uint8_t sb = orc_mxfp4_e8m0_from_max(max_abs);
        scales[b] = sb;
        float scale = orc_mxfp4_decode_e8m0(sb);
        for (int p = 0; p < 16; p++) {
            size_t ih = start + 2 * p, il = start + 2 * p + 1;
            float vh = ih < n ? data[ih] : 0.0f;
            float vl = il < n ? data[il] : 0.0f;
            uint8_t ch = orc_mxfp4_quantize_fp4(vh, scale);
            uint8_t cl = orc_mxfp4_quantize_fp4(vl, scale);
            packed[b * 16 + p] = (uint8_t)((ch << 4) | cl);
        }
    }
}

/* Mxfp4Tensor::dequantize: crates/nn-gptoss/src/quantize.rs:167-188 (LUT * scale) */
void orc_mxfp4_dequantize(const uint8_t *packed, const uint8_t *scales, size_t nblocks, size_t total, float *out) {
    size_t o = 0;
    for (size_t b = 0; b < nblocks && o < total; b++) {
        float scale = orc_mxfp4_decode_e8m0(scales[b]);
        for (int p = 0; p < 16 && o < total; p++) {
            uint8_t byte = packed[b * 16 + p];
            out[o++] = FP4_LUT[(byte >> 4) & 0xF] * scale;
            if (o < total) out[o++] = FP4_LUT[byte & 0xF] * scale;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* f32 compute sinks                                                         */
/* ------------------------------------------------------------------------ */

/* x @ W^T, W [n, k] row-major (Linear::forward / QLinear::forward, crates/nn-core/
 * src/layers/core_layers.rs:118-135, crates/nn-core/src/dyn_tensor/ops/matmul.rs:18-52).
 * The reference's sgemm (ndarray/matrixmultiply) accumulation order is not pinned;
 * this restatement sums k in order from 0. */
void orc_matmul_xwt(const float *x, size_t m, size_t k, const float *w, size_t n, float *y) {
    for (size_t i = 0; i < m; i++)
        for (size_t j = 0; j < n; j++) {
            const float *xr = x + i * k, *wr = w + j * k;
            float acc = 0.0f;
            for (size_t t = 0; t < k; t++) acc = acc + xr[t] * wr[t];
            y[i * n + j] = acc;
        }
}

/* x @ W, W [k, n] row-major (expert matmuls, crates/nn-gptoss/src/quantized_model.rs:112,126) */
void orc_matmul_xw(const float *x, size_t m, size_t k, const float *w, size_t n, float *y) {
    float *acc = (float *)malloc(n * sizeof(float));
    for (size_t i = 0; i < m; i++) {
        for (size_t j = 0; j < n; j++) acc[j] = 0.0f;
        for (size_t t = 0; t < k; t++) {
            float xv = x[i * k + t];
            const float *wr = w + t * n;
            for (size_t j = 0; j < n; j++) acc[j] = acc[j] + xv * wr[j];
        }
        memcpy(y + i * n, acc, n * sizeof(float));
    }
    free(acc);
}

/* argmax: crates/nn-core/src/dyn_tensor/ops_ext/argreduce.rs:94-118 — NaN is an
 * error; best starts at -inf with index 0; strict `>` keeps the first maximum. */
int orc_argmax(const float *v, size_t n, uint32_t *idx) {
    if (n == 0) return -2;
    for (size_t i = 0; i < n; i++)
        if (isnan(v[i])) return -1;
    uint32_t bi = 0;
    float bv = -INFINITY;
    for (size_t i = 0; i < n; i++)
        if (v[i] > bv) {
            bv = v[i];
            bi = (uint32_t)i;
        }
    *idx = bi;
    return 0;
}

/* softmax over the last dim, CPU path: crates/nn-core/src/dyn_tensor/ops/softmax.rs:143-182 */
int orc_softmax_rows(const float *x, size_t rows, size_t cols, float *out) {
    for (size_t i = 0; i < rows * cols; i++)
        if (isnan(x[i])) return -1;
    for (size_t r = 0; r < rows; r++) {
        const float *xr = x + r * cols;
        float *o = out + r * cols;
        float mx = -INFINITY;
        for (size_t c = 0; c < cols; c++) mx = fmaxf(mx, xr[c]);
        if (mx == -INFINITY) {
            for (size_t c = 0; c < cols; c++) o[c] = 0.0f;
            continue;
        }
        if (mx == INFINITY) {
            size_t cnt = 0;
            for (size_t c = 0; c < cols; c++) cnt += xr[c] == INFINITY;
            float prob = 1.0f / (float)cnt;
            for (size_t c = 0; c < cols; c++) o[c] = xr[c] == INFINITY ? prob : 0.0f;
            continue;
        }
        for (size_t c = 0; c < cols; c++) o[c] = expf(xr[c] - mx);
        float sum = -0.0f;
        for (size_t c = 0; c < cols; c++) sum = sum + o[c];
        for (size_t c = 0; c < cols; c++) o[c] = o[c] / sum;
    }
    return 0;
}

/* f32::total_cmp key */
static inline int32_t total_key(float f) {
    int32_t b = (int32_t)f2u(f);
    b ^= (int32_t)(((uint32_t)(b >> 31)) >> 1);
    return b;
}

/* topk along the last dim: crates/nn-core/src/dyn_tensor/ops_ext/sorting.rs:63-104 —
 * descending by total_cmp.  The reference's select_nth_unstable/sort_unstable leave
 * the order of exactly-equal values unspecified; this restatement breaks ties by
 * ascending index. */
int orc_topk_rows(const float *x, size_t rows, size_t cols, size_t k, float *vals, uint32_t *idx) {
    if (k == 0 || k > cols) return -2;
    for (size_t i = 0; i < rows * cols; i++)
        if (isnan(x[i])) return -1;
    for (size_t r = 0; r < rows; r++) {
        const float *xr = x + r * cols;
        for (size_t s = 0; s < k; s++) {
            /* selection: s-th best not yet taken */
            size_t best = (size_t)-1;
            for (size_t c = 0; c < cols; c++) {
                int taken = 0;
                for (size_t q = 0; q < s; q++)
                    if (idx[r * k + q] == c) taken = 1;
                if (taken) continue;
                if (best == (size_t)-1 || total_key(xr[c]) > total_key(xr[best])) best = c;
            }
            idx[r * k + s] = (uint32_t)best;
            vals[r * k + s] = xr[best];
        }
    }
    return 0;
}

/* QLinear::forward with Q4_K weights (full dequant then f32 x @ W^T):
 * crates/nn-core/src/layers/quantized/linear.rs:366-400. */
int orc_q4k_linear(const float *x, size_t rows, size_t k, const uint8_t *w, size_t n, float *y) {
    if (k % 256) return -1;
    float *wf = (float *)malloc(n * k * sizeof(float));
    if (!wf) return -3;
    orc_dequant_q4_k_gguf(w, (n * k / 256) * 144, n * k, wf);
    orc_matmul_xwt(x, rows, k, wf, n, y);
    free(wf);
    return 0;
}

/* GGUF Q6_K load-time decode then f32 Linear (LM head): crates/nn-gguf/src/reader.rs:282,
 * crates/nn-qwen3/src/lib.rs:124-133. */
int orc_q6k_linear(const float *x, size_t rows, size_t k, const uint8_t *w, size_t n, float *y) {
    if (k % 256) return -1;
    float *wf = (float *)malloc(n * k * sizeof(float));
    if (!wf) return -3;
    orc_dequant_q6_k_legacy(w, (n * k / 256) * 210, n * k, wf);
    orc_matmul_xwt(x, rows, k, wf, n, y);
    free(wf);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* GPT-OSS MXFP4 MoE layer                                                    */
/* ------------------------------------------------------------------------ */

/* QuantizedDecoderLayer::moe_forward + expert_forward:
 * crates/nn-gptoss/src/quantized_model.rs:99-194.  The router Linear is
 * replaced by the given logits (the benchmark feeds N(0,1) logits directly).
 * gate_up is [E, hidden, 2*inter] flat MXFP4, down is [E, inter, hidden] flat
 * MXFP4 (blocks of 32 along the flattened, i.e. output, dimension).
 * faithful_full_dequant=1 dequantizes every expert's weights on every
 * expert_forward call (:107, :123), as the reference does; 0 decodes only the
 * expert in use (identical values, less work). */
int orc_moe_forward_mxfp4(const float *x, size_t T, size_t H, const float *logits, size_t E, size_t K,
                          const uint8_t *gu_packed, const uint8_t *gu_scales, const float *gu_bias,
                          const uint8_t *dn_packed, const uint8_t *dn_scales, const float *dn_bias, size_t I,
                          float limit, int faithful, float *out, uint32_t *topk_idx_out, float *topk_w_out) {
    int rc = 0;
    size_t gu_per = H * 2 * I, dn_per = I * H;
    if (gu_per % 32 || dn_per % 32) return -2;
    float *probs = (float *)malloc(T * E * sizeof(float));
    float *tw = (float *)malloc(T * K * sizeof(float));
    uint32_t *ti = (uint32_t *)malloc(T * K * sizeof(uint32_t));
    float *wgu = (float *)malloc((faithful ? E : 1) * gu_per * sizeof(float));
    float *wdn = (float *)malloc((faithful ? E : 1) * dn_per * sizeof(float));
    float *xg = (float *)malloc(T * H * sizeof(float));
    float *gu = (float *)malloc(T * 2 * I * sizeof(float));
    float *hid = (float *)malloc(T * I * sizeof(float));
    float *yo = (float *)malloc(T * H * sizeof(float));
    uint32_t *ids = (uint32_t *)malloc(T * K * sizeof(uint32_t));
    float *wts = (float *)malloc(T * K * sizeof(float));
    if (!probs || !tw || !ti || !wgu || !wdn || !xg || !gu || !hid || !yo || !ids || !wts) {
        rc = -3;
        goto done;
    }
    if (orc_softmax_rows(logits, T, E, probs)) { rc = -1; goto done; }
    if (orc_topk_rows(probs, T, E, K, tw, ti)) { rc = -1; goto done; }
    for (size_t t = 0; t < T; t++) {
        float s = -0.0f;
        for (size_t j = 0; j < K; j++) s = s + tw[t * K + j];
        for (size_t j = 0; j < K; j++) tw[t * K + j] = tw[t * K + j] / s;
    }
    if (topk_idx_out) memcpy(topk_idx_out, ti, T * K * sizeof(uint32_t));
    if (topk_w_out) memcpy(topk_w_out, tw, T * K * sizeof(float));
    for (size_t i = 0; i < T * H; i++) out[i] = 0.0f;
    for (size_t e = 0; e < E; e++) {
        size_t cnt = 0;
        for (size_t t = 0; t < T; t++)
            for (size_t s = 0; s < K; s++)
                if (ti[t * K + s] == e) {
                    ids[cnt] = (uint32_t)t;
                    wts[cnt] = tw[t * K + s];
                    cnt++;
                }
        if (cnt == 0) continue;
        for (size_t r = 0; r < cnt; r++) memcpy(xg + r * H, x + (size_t)ids[r] * H, H * sizeof(float));
        const float *Wg, *Wd;
        if (faithful) {
            orc_mxfp4_dequantize(gu_packed, gu_scales, E * gu_per / 32, E * gu_per, wgu);
            orc_mxfp4_dequantize(dn_packed, dn_scales, E * dn_per / 32, E * dn_per, wdn);
            Wg = wgu + e * gu_per;
            Wd = wdn + e * dn_per;
        } else {
            orc_mxfp4_dequantize(gu_packed + e * gu_per / 2, gu_scales + e * gu_per / 32, gu_per / 32, gu_per, wgu);
            orc_mxfp4_dequantize(dn_packed + e * dn_per / 2, dn_scales + e * dn_per / 32, dn_per / 32, dn_per, wdn);
            Wg = wgu;
            Wd = wdn;
        }
        orc_matmul_xw(xg, cnt, H, Wg, 2 * I, gu);
        for (size_t r = 0; r < cnt; r++)
            for (size_t c = 0; c < 2 * I; c++) gu[r * 2 * I + c] = gu[r * 2 * I + c] + gu_bias[e * 2 * I + c];
        for (size_t r = 0; r < cnt; r++)
            for (size_t c = 0; c < I; c++) {
                float g = gu[r * 2 * I + c];
                float up = gu[r * 2 * I + I + c];
                float sg = g / (1.0f + expf(-g)); /* silu: crates/nn-core/src/dyn_tensor/ops/math.rs:140 */
                if (sg < -limit) sg = -limit;
                if (sg > limit) sg = limit;
                hid[r * I + c] = sg * up;
            }
        orc_matmul_xw(hid, cnt, I, Wd, H, yo);
        for (size_t r = 0; r < cnt; r++)
            for (size_t c = 0; c < H; c++) {
                float v = yo[r * H + c] + dn_bias[e * H + c];
                if (!isfinite(v)) { rc = -4; goto done; }
                yo[r * H + c] = v;
            }
        for (size_t r = 0; r < cnt; r++)
            for (size_t c = 0; c < H; c++) {
                float wv = yo[r * H + c] * wts[r];
                out[(size_t)ids[r] * H + c] = out[(size_t)ids[r] * H + c] + wv;
            }
    }
    for (size_t i = 0; i < T * H; i++)
        if (!isfinite(out[i])) { rc = -4; goto done; }
done:
    free(probs); free(tw); free(ti); free(wgu); free(wdn); free(xg); free(gu); free(hid); free(yo);
    free(ids); free(wts);
    return rc;
}

/* ------------------------------------------------------------------------ */
/* nn-core OCP MXFP4: crates/nn-core/src/layers/quantized/mxfp4.rs.          */
/* A block is [shared_exp u8][16 packed bytes] (Mxfp4Block, :70-84, 17 bytes, */
/* BLOCK_STORAGE_BYTES :52); element 2i is the LOW nibble of byte i (:209-213,*/
/* :232-237); blocks run along the flattened order, the last one zero-padded  */
/* (quantize_tensor :293-315).  The 4-bit codes are the e2m1 values the file */
/* calls E1M2 (:58-64).                                                       */
/* ------------------------------------------------------------------------ */

static const float OCP_MAG[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};

/* block_scale_from_exp (:177-186): 2^(e - 127) in f64, cast to f32 (e = 0 gives the
 * f32 subnormal 2^-127, e = 255 overflows to +inf) */
float orc_ocp_block_scale(uint8_t shared_exp) { return (float)ldexp(1.0, (int)shared_exp - 127); }

/* compute_shared_exponent (:142-170): ceil(log2(max|v| / 6)) + 127 in f32, clamped to
 * [0, 254]; 0 for an all-zero block.  The values are finite (quantize_block checks
 * first). */
uint8_t orc_ocp_shared_exp(const float *v32) {
    float max_abs = 0.0f;
    for (int i = 0; i < 32; i++) {
        const float a = fabsf(v32[i]);
        if (a > max_abs) max_abs = a;
    }
    if (max_abs == 0.0f) return 0;
    const float log2_ratio = log2f(max_abs / 6.0f);
    const int exp_biased = (int)ceilf(log2_ratio) + 127;
    return (uint8_t)(exp_biased < 0 ? 0 : (exp_biased > 254 ? 254 : exp_biased));
}

/* encode_e1m2 (:96-117): 0 for a zero value or scale; else the nearest magnitude of
 * |v| / scale (strict <, so ties keep the lower index) with the sign in bit 3 */
uint8_t orc_ocp_encode(float v, float block_scale) {
    if (v == 0.0f || block_scale == 0.0f) return 0;
    const int sign = v < 0.0f;
    const float abs_scaled = fabsf(v) / block_scale;
    uint8_t best = 0;
    float best_dist = 3.40282347e38f;
    for (uint8_t i = 0; i < 8; i++) {
        const float dist = fabsf(abs_scaled - OCP_MAG[i]);
        if (dist < best_dist) {
            best_dist = dist;
            best = i;
        }
    }
    return (uint8_t)((sign ? 0x8 : 0x0) | best);
}

/* decode_e1m2 (:124-134): magnitude * scale, negated when bit 3 is set */
float orc_ocp_decode(uint8_t code, float block_scale) {
    const float value = OCP_MAG[code & 7] * block_scale;
    return (code >> 3) & 1 ? -value : value;
}

/* quantize_tensor (:293-315) over quantize_block (:194-220); blocks holds
 * ceil(n / 32) * 17 bytes.  Returns -1 (ValueOutOfRange) on a non-finite value. */
int orc_ocp_quantize_tensor(const float *data, size_t n, uint8_t *blocks) {
    for (size_t i = 0; i < n; i++)
        if (!isfinite(data[i])) return -1;
    const size_t nb = (n + 31) / 32;
    for (size_t b = 0; b < nb; b++) {
        float v[32] = {0};
        for (size_t i = 0; i < 32 && b * 32 + i < n; i++) v[i] = data[b * 32 + i];
        const uint8_t e = orc_ocp_shared_exp(v);
        const float scale = orc_ocp_block_scale(e);
        uint8_t *blk = blocks + b * 17;
        blk[0] = e;
        memset(blk + 1, 0, 16);
        for (int i = 0; i < 32; i++) {
            const uint8_t code = orc_ocp_encode(v[i], scale);
            blk[1 + i / 2] |= (i % 2 == 0) ? code : (uint8_t)(code << 4);
        }
    }
    return 0;
}

/* dequantize_tensor (:320-333) over dequantize_block (:226-244): the first n values */
void orc_ocp_dequantize_tensor(const uint8_t *blocks, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) {
        const uint8_t *blk = blocks + (i / 32) * 17;
        const size_t j = i % 32;
        const uint8_t byte = blk[1 + j / 2];
        out[i] = orc_ocp_decode(j % 2 == 0 ? (byte & 0x0F) : (byte >> 4), orc_ocp_block_scale(blk[0]));
    }
}

/* splitmix64 mixer: crates/nn-core/src/test_prng.rs:18-22 */
uint64_t orc_splitmix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* ------------------------------------------------------------------------ */
/* Qwen3 SwiGLU MLP glue (crates/nn-qwen3/src/layers.rs:40-47):              */
/*   gate = silu(gate_proj(x)), up = up_proj(x), out = down_proj(gate * up), */
/* silu(x) = x / (1 + exp(-x)) in f32 (crates/nn-core/src/dyn_tensor/ops/    */
/* math.rs:140), the product elementwise in f32 (broadcast_mul).             */
/* ------------------------------------------------------------------------ */

void orc_silu_mul(const float *g, const float *u, size_t n, float *h) {
    for (size_t i = 0; i < n; i++) {
        const float s = g[i] / (1.0f + expf(-g[i]));
        h[i] = s * u[i];
    }
}

/* check_output_finite (crates/nn-core/src/layers/nan_check.rs:113): 1 when any value is NaN or infinite */
int orc_any_nonfinite(const float *v, size_t n) {
    for (size_t i = 0; i < n; i++)
        if (!isfinite(v[i])) return 1;
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Token sampling: sample_token (crates/nn-gptoss/src/sampling.rs:136-185)   */
/* and its steps.  top_k < 0 means None; use_top_p = 0 means None.           */
/* Top-k ties: the reference sorts with sort_unstable_by, whose order among  */
/* equal logits is unspecified; here equal values keep the lower index       */
/* first (parity unpinned for exact ties at the k-th place).  NaN logits are */
/* ordered below -inf for the selection and never become candidates.  With   */
/* top_k Some(k) the candidates are the finite logits among the k largest    */
/* (apply_top_k, :245-275); with top_k None every logit v > -inf is one,     */
/* +inf included (:158-165), which makes softmax_candidates uniform.         */
/* ------------------------------------------------------------------------ */

typedef struct { uint32_t idx; float v; } orc_cand;

/* descending value, then ascending index; NaN last */
static int cand_desc(const void *a, const void *b) {
    const orc_cand *x = (const orc_cand *)a, *y = (const orc_cand *)b;
    const int xn = x->v != x->v, yn = y->v != y->v;
    if (xn != yn) return xn - yn;
    if (!xn && x->v != y->v) return x->v > y->v ? -1 : 1;
    return x->idx < y->idx ? -1 : (x->idx > y->idx);
}

/* softmax_candidates (sampling.rs:371-391): probabilities in candidate order */
static void softmax_cands(const orc_cand *c, size_t n, float *p) {
    float mx = -INFINITY;
    for (size_t i = 0; i < n; i++) mx = fmaxf(mx, c[i].v);
    if (!isfinite(mx)) {
        for (size_t i = 0; i < n; i++) p[i] = 1.0f / (float)n;
        return;
    }
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        p[i] = expf(c[i].v - mx);
        sum += p[i];
    }
    if (!isfinite(sum) || sum == 0.0f) {
        for (size_t i = 0; i < n; i++) p[i] = 1.0f / (float)n;
        return;
    }
    for (size_t i = 0; i < n; i++) p[i] = p[i] / sum;
}

/* argmax_slice (sampling.rs:394-400): Iterator::max_by with partial_cmp, i.e. the
 * running maximum is replaced unless it compares Greater (ties and NaN move on) */
size_t orc_argmax_slice(const float *v, size_t n) {
    size_t best = 0;
    for (size_t j = 1; j < n; j++)
        if (!(v[best] > v[j])) best = j;
    return best;
}

/* softmax_sample (sampling.rs:340-365) */
static uint32_t softmax_sample_c(const orc_cand *c, size_t n, uint64_t seed) {
    if (n == 1) return c[0].idx;
    float *p = (float *)malloc(n * sizeof(float));
    softmax_cands(c, n, p);
    const float selector = (float)(seed % 10000u) / 10000.0f;
    float cum = 0.0f;
    uint32_t out = c[n - 1].idx;
    for (size_t i = 0; i < n; i++) {
        cum += p[i];
        if (selector < cum) {
            out = c[i].idx;
            break;
        }
    }
    free(p);
    return out;
}

int orc_sample_token(const float *logits, size_t n, const uint32_t *past, size_t n_past, float temperature,
                     int64_t top_k, int use_top_p, float top_p, float rep_penalty, float freq_penalty, uint64_t seed,
                     uint32_t *token) {
    if (n == 0 || !(temperature > 0.0f) || !isfinite(temperature)) return -1;
    float *s = (float *)malloc(n * sizeof(float));
    memcpy(s, logits, n * sizeof(float));
    /* apply_repetition_penalty (:277-290), per occurrence */
    if (fabsf(rep_penalty - 1.0f) > 1.1920929e-7f)
        for (size_t i = 0; i < n_past; i++)
            if (past[i] < n) {
                const float l = s[past[i]];
                if (l > 0.0f) s[past[i]] = l / rep_penalty;
                else if (l < 0.0f) s[past[i]] = l * rep_penalty;
            }
    /* apply_frequency_penalty (:297-306) */
    if (fabsf(freq_penalty) > 1.1920929e-7f)
        for (size_t i = 0; i < n_past; i++)
            if (past[i] < n) s[past[i]] -= freq_penalty;
    /* apply_temperature (:193-199) */
    for (size_t i = 0; i < n; i++)
        if (isfinite(s[i])) s[i] /= temperature;
    orc_cand *c = (orc_cand *)malloc(n * sizeof(orc_cand));
    size_t nc = 0;
    if (top_k < 0) {
        /* top_k None (:160-164): every v > -inf in index order; NaN compares false */
        for (size_t i = 0; i < n; i++)
            if (s[i] > -INFINITY) c[nc++] = (orc_cand){(uint32_t)i, s[i]};
    } else if ((size_t)top_k >= n) {
        /* apply_top_k with k >= len (:250-256): the finite logits in index order */
        for (size_t i = 0; i < n; i++)
            if (isfinite(s[i])) c[nc++] = (orc_cand){(uint32_t)i, s[i]};
    } else if (top_k > 0) {
        /* apply_top_k (:258-275): the k largest, then the finite ones in index order */
        orc_cand *all = (orc_cand *)malloc(n * sizeof(orc_cand));
        for (size_t i = 0; i < n; i++) all[i] = (orc_cand){(uint32_t)i, s[i]};
        qsort(all, n, sizeof(orc_cand), cand_desc);
        unsigned char *keep = (unsigned char *)calloc(n, 1);
        for (int64_t i = 0; i < top_k; i++) keep[all[i].idx] = 1;
        for (size_t i = 0; i < n; i++)
            if (keep[i] && isfinite(s[i])) c[nc++] = (orc_cand){(uint32_t)i, s[i]};
        free(keep);
        free(all);
    }
    /* apply_top_p_candidates (:211-238) */
    if (use_top_p && nc > 0) {
        qsort(c, nc, sizeof(orc_cand), cand_desc); /* stable order: ties keep index order */
        float *p = (float *)malloc(nc * sizeof(float));
        softmax_cands(c, nc, p);
        float cum = 0.0f;
        size_t keepn = 0;
        for (size_t i = 0; i < nc; i++) {
            cum += p[i];
            keepn = i + 1;
            if (cum >= top_p) break;
        }
        nc = keepn;
        free(p);
    }
    /* Step 6 (:178-184) */
    if (nc == 0)
        *token = (uint32_t)orc_argmax_slice(logits, n);
    else
        *token = softmax_sample_c(c, nc, seed);
    free(c);
    free(s);
    return 0;
}

