// Host-side upload repack: GGUF / nn-gguf block bytes -> the tile16 device image.
//
// Every transform here is a bijection on the block bytes (plus zero padding of
// the last row tile and, for Q8_0, of the last group of 8 blocks), so the
// algorithmic bytes a kernel streams equal the bytes of the source blocks.
#include <cmath>
#include <cstring>
#include <vector>

#include "nnq_internal.h"

namespace nnq {

bool make_layout(int fmt, int layout, int64_t n, int64_t k, Layout *L, const char **err) {
    *L = Layout{};
    L->fmt = fmt;
    L->layout = layout;
    L->n = n;
    L->k = k;
    L->ntile = (n + kTile - 1) / kTile;
    switch (fmt) {
    case NNQ_FMT_Q4_K:
        if (layout != NNQ_LAYOUT_GGUF && layout != NNQ_LAYOUT_NN_GGUF) {
            *err = "Q4_K supports the GGUF (BlockQ4K) and nn-gguf layouts";
            return false;
        }
        if (k % 256) {
            *err = "Q4_K in_features must be a multiple of 256 (row-aligned super-blocks)";
            return false;
        }
        L->nblk = k / 256;
        L->qs_bytes = (size_t)L->ntile * L->nblk * 2048;
        L->hdr_bytes = (size_t)L->ntile * L->nblk * 256;
        L->aux_bytes = (size_t)L->ntile * L->nblk * 512 + (size_t)L->ntile * kTile * 4;
        return true;
    case NNQ_FMT_Q8_0:
        if (layout != NNQ_LAYOUT_GGUF && layout != NNQ_LAYOUT_NN_GGUF) {
            *err = "Q8_0 supports the GGUF layout";
            return false;
        }
        if (k % 32) {
            *err = "Q8_0 in_features must be a multiple of 32";
            return false;
        }
        L->nblk = ((k / 32) + 7) / 8 * 8;
        L->qs_bytes = (size_t)L->ntile * (L->nblk / 2) * 1024;
        L->hdr_bytes = (size_t)L->ntile * (L->nblk / 8) * 256;
        return true;
    case NNQ_FMT_Q6_K:
        if (layout != NNQ_LAYOUT_NN_GGUF) {
            *err = "Q6_K is supported in the nn-gguf layout (the reference's only Q6_K decoder)";
            return false;
        }
        if (k % 256) {
            *err = "Q6_K in_features must be a multiple of 256";
            return false;
        }
        L->nblk = k / 256;
        L->qs_bytes = (size_t)L->ntile * L->nblk * 3072;
        L->hdr_bytes = (size_t)L->ntile * L->nblk * 288;
        return true;
    default:
        *err = "unsupported block format for a linear weight";
        return false;
    }
}

// Byte order inside each 4-byte word of the quant plane: source bytes (e0,e1,e2,e3)
// are stored as (e0,e2,e1,e3) so that `w & 0x000F000F` / `(w >> 8) & 0x000F000F`
// (and the 0x00FF00FF variants) yield element pairs (e0,e1) and (e2,e3).
static inline void put_perm8(uint8_t *dst, const uint8_t *src) {
    for (int w = 0; w < 2; w++) {
        dst[4 * w + 0] = src[4 * w + 0];
        dst[4 * w + 1] = src[4 * w + 2];
        dst[4 * w + 2] = src[4 * w + 1];
        dst[4 * w + 3] = src[4 * w + 3];
    }
}

// nn-gguf Q4_K (crates/nn-gguf/src/dequant.rs:335-398) -> BlockQ4K packing
// (crates/nn-core/src/layers/quantized/linear.rs:121-157).  Both decode as
// (d*sc_j)*q - dmin*m_j over sub-block j = element/32, so moving the 6-bit
// scales/mins and the nibbles yields identical f32 values.
void q4k_legacy_to_gguf(const uint8_t *p, uint8_t *o) {
    const uint8_t *sd = p + 4;
    uint8_t sc[8], mn[8], q[256];
    for (int j = 0; j < 8; j++) sc[j] = (sd[j / 2] >> (4 * (j % 2))) & 0x0F;
    for (int j = 0; j < 8; j++) mn[j] = (sd[4 + j / 2] >> (4 * (j % 2))) & 0x0F;
    for (int j = 0; j < 4; j++) sc[j] |= ((sd[8] >> (2 * j)) & 3) << 4;
    for (int j = 0; j < 4; j++) sc[4 + j] |= ((sd[9] >> (2 * j)) & 3) << 4;
    for (int j = 0; j < 4; j++) mn[j] |= ((sd[10] >> (2 * j)) & 3) << 4;
    for (int j = 0; j < 4; j++) mn[4 + j] |= ((sd[11] >> (2 * j)) & 3) << 4;
    const uint8_t *qs = p + 16;
    for (int j = 0; j < 8; j++)
        for (int i = 0; i < 16; i++) {
            q[32 * j + 2 * i] = qs[16 * j + i] & 0x0F;
            q[32 * j + 2 * i + 1] = qs[16 * j + i] >> 4;
        }
    std::memcpy(o, p, 4);
    uint8_t *s = o + 4;
    std::memset(s, 0, 12);
    for (int j = 0; j < 8; j++) {
        uint8_t ls = sc[j], lm = mn[j];
        if (j < 4) {
            s[j] = ls;
            s[j + 4] = lm;
        } else {
            s[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
            s[j - 4] |= (uint8_t)((ls >> 4) << 6);
            s[j] |= (uint8_t)((lm >> 4) << 6);
        }
    }
    for (int g = 0; g < 4; g++)
        for (int i = 0; i < 32; i++) o[16 + 32 * g + i] = (uint8_t)(q[64 * g + i] | (q[64 * g + 32 + i] << 4));
}

void repack_q4k(const uint8_t *src, int legacy, const Layout &L, uint8_t *dst) {
    uint8_t *qs = dst;
    uint8_t *hdr = dst + L.qs_bytes;
    std::memset(dst, 0, L.total());
    uint8_t tmp[144];
    for (int64_t t = 0; t < L.ntile; t++)
        for (int64_t b = 0; b < L.nblk; b++)
            for (int r = 0; r < kTile; r++) {
                int64_t row = t * kTile + r;
                if (row >= L.n) continue;
                const uint8_t *blk = src + (row * L.nblk + b) * 144;
                if (legacy) {
                    q4k_legacy_to_gguf(blk, tmp);
                    blk = tmp;
                }
                std::memcpy(hdr + (t * L.nblk + b) * 256 + 16 * r, blk, 16);
                // lane l = 16p + r of plane h holds bytes [16h, 16h + 16) of group p (the 32
                // bytes whose low / high nibbles are sub-blocks 2p / 2p + 1) of row r
                uint8_t *qb = qs + (t * L.nblk + b) * 2048;
                for (int h = 0; h < 2; h++)
                    for (int p = 0; p < 4; p++) {
                        uint8_t *d = qb + 1024 * h + 16 * (16 * p + r);
                        put_perm8(d, blk + 16 + 32 * p + 16 * h);
                        put_perm8(d + 8, blk + 16 + 32 * p + 16 * h + 8);
                    }
            }
}

void repack_q8_0(const uint8_t *src, const Layout &L, uint8_t *dst) {
    uint8_t *qs = dst;
    uint8_t *hdr = dst + L.qs_bytes;
    std::memset(dst, 0, L.total());
    const int64_t nb = L.k / 32;
    const int64_t npair = L.nblk / 2, ngrp = L.nblk / 8;
    static const uint8_t zeros[34] = {0};
    for (int64_t t = 0; t < L.ntile; t++)
        for (int r = 0; r < kTile; r++) {
            int64_t row = t * kTile + r;
            if (row >= L.n) continue;
            for (int64_t b = 0; b < L.nblk; b++) {
                const uint8_t *blk = b < nb ? src + (row * nb + b) * 34 : zeros;
                // scales: (tile, group of 8 blocks) -> 16 rows x 8 f16
                uint8_t *h = hdr + (t * ngrp + b / 8) * 256 + 16 * r + 2 * (b % 8);
                h[0] = blk[0];
                h[1] = blk[1];
                int64_t bp = b / 2;
                int half = (int)(b % 2);
                for (int p = 0; p < 4; p++) {
                    uint8_t *d = qs + (t * npair + bp) * 1024 + 16 * (16 * p + r) + 8 * half;
                    put_perm8(d, blk + 2 + 8 * p);
                }
            }
        }
    (void)npair;
}

// Q6_K (nn-gguf layout, crates/nn-gguf/src/dequant.rs:415-459).  For each
// (tile, block, 64-value chunk c) lane l = 16p + r holds 12 bytes:
//   word A: low nibbles of v0..v7, word B: low nibbles of v8..v15, word C: the
//   16 two-bit high parts, where v_s = q[64c + 8p + s] and v_{8+s} = q[64c + 32 + 8p + s].
// Pair j = (v_{2j}, v_{2j+1}) keeps its nibbles at bits 4j' and 16+4j' (j' = j mod 4) of
// A or B, and its crumbs at bits 2j and 16+2j of C.
void repack_q6k(const uint8_t *src, const Layout &L, uint8_t *dst) {
    uint8_t *qs = dst;
    uint8_t *hdr = dst + L.qs_bytes;
    std::memset(dst, 0, L.total());
    uint8_t q[256];
    for (int64_t t = 0; t < L.ntile; t++)
        for (int64_t b = 0; b < L.nblk; b++)
            for (int r = 0; r < kTile; r++) {
                int64_t row = t * kTile + r;
                if (row >= L.n) continue;
                const uint8_t *blk = src + (row * L.nblk + b) * 210;
                const uint8_t *ql = blk, *qh = blk + 128;
                for (int idx = 0; idx < 256; idx++) {
                    uint8_t lo = (idx % 2 == 0) ? (ql[idx / 2] & 0x0F) : ((ql[idx / 2] >> 4) & 0x0F);
                    uint8_t hi = (qh[idx / 4] >> ((idx % 4) * 2)) & 0x03;
                    q[idx] = (uint8_t)(lo | (hi << 4));
                }
                uint8_t *h = hdr + (t * L.nblk + b) * 288;
                std::memcpy(h + 16 * r, blk + 192, 16);
                h[256 + 2 * r] = blk[208];
                h[256 + 2 * r + 1] = blk[209];
                for (int c = 0; c < 4; c++)
                    for (int p = 0; p < 4; p++) {
                        uint32_t A = 0, B = 0, C = 0;
                        for (int s = 0; s < 16; s++) {
                            int kk = s < 8 ? 64 * c + 8 * p + s : 64 * c + 32 + 8 * p + (s - 8);
                            uint32_t v = q[kk];
                            int j = s / 2, which = s % 2;
                            uint32_t nib = v & 0xF, crumb = v >> 4;
                            int jj = j % 4;
                            uint32_t npos = 4 * jj + 16 * which;
                            if (j < 4)
                                A |= nib << npos;
                            else
                                B |= nib << npos;
                            C |= crumb << (2 * j + 16 * which);
                        }
                        uint8_t *d = qs + ((t * L.nblk + b) * 4 + c) * 768 + 12 * (16 * p + r);
                        std::memcpy(d, &A, 4);
                        std::memcpy(d + 4, &B, 4);
                        std::memcpy(d + 8, &C, 4);
                    }
            }
}

}  // namespace nnq

namespace nnq {

// GPT-OSS MXFP4 expert weights (Mxfp4Tensor of the flat [E][K][N] tensor,
// crates/nn-gptoss/src/quantize.rs:122-163: byte p of a 32-element block holds
// element 2p in the high nibble and 2p + 1 in the low nibble, one E8M0 scale per
// block) -> per (expert, 32-column block, 32-row block) fragments whose bytes each
// lane of a 16x16x32 MFMA wave needs; see MoeDev.
void moe_repack(const uint8_t *packed, const uint8_t *scales, int64_t E, int64_t K, int64_t N, uint8_t *dc,
                uint8_t *ds, bool gptoss_scales) {
    const int64_t NB = N / 32, KB = K / 32;
    for (int64_t e = 0; e < E; e++)
        for (int64_t nb = 0; nb < NB; nb++)
            for (int64_t kb = 0; kb < KB; kb++) {
                const int64_t frag = (e * NB + nb) * KB + kb;
                uint8_t *c = dc + frag * 512;
                for (int p = 0; p < 4; p++)
                    for (int col = 0; col < 16; col++)
                        for (int i = 0; i < 8; i++) {
                            const int64_t row = kb * 32 + 8 * p + i;
                            c[(16 * p + col) * 8 + i] = packed[(e * K + row) * (N / 2) + nb * 16 + col];
                        }
                uint8_t *s = ds + frag * 32;
                for (int r = 0; r < 32; r++) {
                    const uint8_t v = scales[(e * K + kb * 32 + r) * NB + nb];
                    s[r] = (gptoss_scales && v == 0) ? 1 : v;
                }
            }
}

void ocp_split(const uint8_t *blocks, size_t nblocks, uint8_t *packed, uint8_t *scales) {
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t *blk = blocks + b * 17;
        scales[b] = blk[0];
        for (int p = 0; p < 16; p++) packed[b * 16 + p] = (uint8_t)((blk[1 + p] << 4) | (blk[1 + p] >> 4));
    }
}

}  // namespace nnq

namespace nnq {

// Power of two s with amax * s in [2^14, 2^15) (1 for amax = 0, NaN for a non-finite
// amax), exponent clamped to +-126: the device f16_prescale.
static float prescale_pow2(float amax) {
    if (!(amax <= 3.0e38f)) return std::nanf("");
    if (amax == 0.0f) return 1.0f;
    uint32_t u;
    std::memcpy(&u, &amax, 4);
    int eb = (int)((u >> 23) & 0xFF);
    int se = 141 - (eb > 1 ? eb : 1);
    se = se > 126 ? 126 : (se < -126 ? -126 : se);
    return std::ldexp(1.0f, se);
}

void q4k_aux_plane(const uint8_t *hdr, const Layout &L, uint8_t *aux, int64_t t0, int64_t t1) {
    float *srow = reinterpret_cast<float *>(aux + (size_t)L.ntile * L.nblk * 512);
    for (int64_t t = t0; t < t1; t++)
        for (int r = 0; r < kTile; r++) {
            auto dmin_of = [&](int64_t b) {
                uint16_t h;
                std::memcpy(&h, hdr + (t * L.nblk + b) * 256 + 16 * r + 2, 2);
                _Float16 f;
                std::memcpy(&f, &h, 2);
                return (float)f;
            };
            float dmax = 0.0f;
            for (int64_t b = 0; b < L.nblk; b++) dmax = std::fmax(dmax, std::fabs(dmin_of(b)));
            const float s = prescale_pow2(dmax * 63.0f);
            srow[t * kTile + r] = s;
            for (int64_t b = 0; b < L.nblk; b++) {
                const uint8_t *q = hdr + (t * L.nblk + b) * 256 + 16 * r + 4;  // scales[12]
                const float dm = dmin_of(b) * s;
                uint8_t *hi = aux + (t * L.nblk + b) * 512 + 16 * r, *lo = hi + 256;
                for (int j = 0; j < 8; j++) {
                    // get_scale_min_k4 (crates/nn-core/src/layers/quantized/linear.rs:166-176): the min
                    const uint8_t m = j < 4 ? (q[j + 4] & 63) : (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
                    const float v = dm * (float)m;  // exact: 11 + 6 significant bits
                    const _Float16 h = (_Float16)v, l = (_Float16)(v - (float)h);
                    std::memcpy(hi + 2 * j, &h, 2);
                    std::memcpy(lo + 2 * j, &l, 2);
                }
            }
        }
}

}  // namespace nnq
