// Host-side encoders and the seeded input generator of the C ABI.
//
// The Q4_K and MXFP4 encoders restate the reference's quantizers (cited per
// function); Q8_0 and Q6_K have no reference encoder, so these are this
// library's own input generators.  All of them run on the CPU and are
// parallelised over independent blocks (results do not depend on threading).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/nnq.h"
#include "nnq_internal.h"

namespace {

template <class F>
void parallel_blocks(size_t nblocks, F &&fn) {
    size_t hw = std::max(1u, std::thread::hardware_concurrency());
    size_t nt = std::min<size_t>(hw, std::max<size_t>(1, nblocks / 4096));
    if (nt <= 1) {
        fn(0, nblocks);
        return;
    }
    std::vector<std::thread> th;
    size_t per = (nblocks + nt - 1) / nt;
    for (size_t t = 0; t < nt; t++) {
        size_t lo = t * per, hi = std::min(nblocks, lo + per);
        if (lo >= hi) break;
        th.emplace_back([&fn, lo, hi] { fn(lo, hi); });
    }
    for (auto &x : th) x.join();
}

inline uint32_t f2u(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
inline float u2f(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }

// IEEE binary32 -> binary16, round to nearest even (the `half` crate's from_f32).
uint16_t to_f16(float f) {
    uint32_t x = f2u(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return ax == 0x7F800000u ? (uint16_t)(sign | 0x7C00u) : (uint16_t)(sign | 0x7E00u | ((ax & 0x7FFFFFu) >> 13));
    int e = (int)(ax >> 23) - 127;
    uint32_t mant = ax & 0x7FFFFFu;
    if (e >= -14) {
        if (e > 15) return sign | 0x7C00u;
        uint32_t h = ((uint32_t)(e + 15) << 10) | (mant >> 13);
        uint32_t rem = mant & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    if (ax < 0x00800000u) return sign;
    uint32_t m = mant | 0x800000u;
    int sh = -(e + 1);
    if (sh > 24) return sign;
    uint32_t h = m >> sh, rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float from_f16(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1F, m = h & 0x3FF;
    if (e == 0) return u2f(f2u((float)m * 5.9604644775390625e-8f) | sign);
    if (e == 31) return u2f(sign | (m ? 0x7FC00000u | (m << 13) : 0x7F800000u));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

// ---- Q4_K: BlockQ4K::quantize (crates/nn-core/src/layers/quantized/linear.rs:95-162) ----

// nearest_int (:179-192): round half away from zero; error on non-finite / out of i32.
bool nearest_int(float v, int32_t *o) {
    if (!std::isfinite(v)) return false;
    float r = std::round(v);
    if (r < -2147483648.0f || r > 2147483648.0f) return false;
    *o = r >= 2147483648.0f ? 2147483647 : (int32_t)r;
    return true;
}

// make_qkx1_quants (:195-254) with nmax = 15, ntry = 5 over 32 values.
bool qkx1(const float *x, float *scale_out, float *negmin_out) {
    const int n = 32, nmax = 15, ntry = 5;
    uint8_t l[32] = {0};
    float mn = INFINITY, mx = -INFINITY;
    for (int i = 0; i < n; i++) mn = std::fmin(mn, x[i]);
    for (int i = 0; i < n; i++) mx = std::fmax(mx, x[i]);
    if (mx == mn) {
        if (mn >= 0.0f) {
            *scale_out = mn / (float)nmax;
            *negmin_out = 0.0f;
        } else {
            *scale_out = 0.0f;
            *negmin_out = -mn;
        }
        return true;
    }
    float min = std::fmin(mn, 0.0f);
    float iscale = (float)nmax / (mx - min);
    float scale = 1.0f / iscale;
    for (int it = 0; it < ntry; it++) {
        float sumlx = 0.0f;
        int32_t suml2 = 0;
        bool changed = false;
        for (int i = 0; i < n; i++) {
            int32_t li;
            if (!nearest_int(iscale * (x[i] - min), &li)) return false;
            li = std::min(std::max(li, 0), nmax);
            if ((uint8_t)li != l[i]) {
                l[i] = (uint8_t)li;
                changed = true;
            }
            volatile float prod = (x[i] - min) * (float)li;  // no FMA contraction
            sumlx = sumlx + prod;
            suml2 += li * li;
        }
        if (suml2 == 0) {
            *scale_out = 0.0f;
            *negmin_out = 0.0f;
            return true;
        }
        scale = sumlx / (float)suml2;
        if (scale == 0.0f) {
            *scale_out = 0.0f;
            *negmin_out = -min;
            return true;
        }
        float sum = -0.0f;
        for (int i = 0; i < n; i++) {
            volatile float t = scale * (float)l[i];
            sum = sum + (x[i] - t);
        }
        min = std::fmin(sum / (float)n, 0.0f);
        iscale = 1.0f / scale;
        if (!changed) break;
    }
    *scale_out = scale;
    *negmin_out = -min;
    return true;
}

void scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

bool quantize_q4k_block(const float *v, uint8_t *blk) {
    float ss[8], sm[8];
    for (int j = 0; j < 8; j++)
        if (!qkx1(v + 32 * j, &ss[j], &sm[j])) return false;
    float max_scale = 0.0f, max_min = 0.0f;
    for (int j = 0; j < 8; j++) max_scale = std::fmax(max_scale, ss[j]);
    for (int j = 0; j < 8; j++) max_min = std::fmax(max_min, sm[j]);
    float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
    float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
    uint8_t s[12] = {0};
    for (int j = 0; j < 8; j++) {
        int32_t a, b;
        if (!nearest_int(inv_scale * ss[j], &a) || !nearest_int(inv_min * sm[j], &b)) return false;
        uint8_t ls = std::min<uint8_t>((uint8_t)a, 63), lm = std::min<uint8_t>((uint8_t)b, 63);
        if (j < 4) {
            s[j] = ls;
            s[j + 4] = lm;
        } else {
            s[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
            s[j - 4] |= (uint8_t)((ls >> 4) << 6);
            s[j] |= (uint8_t)((lm >> 4) << 6);
        }
    }
    uint16_t d = to_f16(max_scale / 63.0f), dmin = to_f16(max_min / 63.0f);
    uint8_t l[256] = {0};
    for (int j = 0; j < 8; j++) {
        uint8_t sc, m;
        scale_min_k4(j, s, &sc, &m);
        float bd = from_f16(d) * (float)sc;
        if (bd == 0.0f) continue;
        float bm = from_f16(dmin) * (float)m;
        for (int i = 0; i < 32; i++) {
            int32_t q;
            if (!nearest_int((v[32 * j + i] + bm) / bd, &q)) return false;
            l[32 * j + i] = (uint8_t)std::min(std::max(q, 0), 15);
        }
    }
    blk[0] = (uint8_t)d;
    blk[1] = (uint8_t)(d >> 8);
    blk[2] = (uint8_t)dmin;
    blk[3] = (uint8_t)(dmin >> 8);
    std::memcpy(blk + 4, s, 12);
    for (int g = 0; g < 4; g++)
        for (int i = 0; i < 32; i++) blk[16 + 32 * g + i] = (uint8_t)(l[64 * g + i] | (l[64 * g + 32 + i] << 4));
    return true;
}

// ---- MXFP4 (crates/nn-gptoss/src/quantize.rs:68-163) ----
const float kFp4Abs[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};

uint8_t e8m0_from_max(float a) {  // compute_e8m0_scale (:68-81)
    if (!std::isfinite(a) || a <= 0.0f) return 0;
    uint8_t be = (uint8_t)((f2u(a) >> 23) & 0xFF);
    if (be == 0) return 0;
    uint8_t se = be >= 2 ? (uint8_t)(be - 2) : 0;
    return std::min<uint8_t>(se, 254);
}
float e8m0_decode(uint8_t e) { return e == 0 ? u2f(0x00800000u) : u2f((uint32_t)e << 23); }  // (:84-90)
uint8_t fp4_code(float v, float scale) {  // quantize_to_fp4 (:93-116)
    if (!std::isfinite(v) || scale <= 0.0f) return 0;
    bool neg = v < 0.0f;
    float a = std::fabs(v) / scale;
    int best = 0;
    float bd = 3.40282347e+38f;
    for (int i = 0; i < 8; i++) {
        float d = std::fabs(a - kFp4Abs[i]);
        if (d < bd) {
            bd = d;
            best = i;
        }
    }
    return (uint8_t)(neg ? best | 8 : best);
}

}  // namespace

extern "C" {

int nnq_quantize_q4_k(const float *v, size_t n, uint8_t *out) {
    if (!v || !out) return NNQ_ERR_INVALID_ARGUMENT;
    size_t nb = (n + 255) / 256;
    std::vector<char> bad(nb, 0);
    parallel_blocks(nb, [&](size_t lo, size_t hi) {
        float buf[256];
        for (size_t b = lo; b < hi; b++) {
            size_t base = b * 256, cnt = std::min<size_t>(256, n - base);
            std::memcpy(buf, v + base, cnt * sizeof(float));
            std::fill(buf + cnt, buf + 256, 0.0f);
            if (!quantize_q4k_block(buf, out + b * 144)) bad[b] = 1;
        }
    });
    for (char c : bad)
        if (c) return NNQ_ERR_NON_FINITE;
    return NNQ_OK;
}

int nnq_quantize_mxfp4(const float *v, size_t n, uint8_t *packed, uint8_t *scales) {
    if (!v || !packed || !scales) return NNQ_ERR_INVALID_ARGUMENT;
    size_t nb = (n + 31) / 32;
    parallel_blocks(nb, [&](size_t lo, size_t hi) {
        for (size_t b = lo; b < hi; b++) {
            size_t s0 = b * 32;
            float mx = 0.0f;
            for (int i = 0; i < 32; i++) {
                float a = s0 + i < n ? std::fabs(v[s0 + i]) : 0.0f;
                if (std::isfinite(a) && a > mx) mx = a;
            }
            uint8_t e = e8m0_from_max(mx);
            scales[b] = e;
            float sc = e8m0_decode(e);
            for (int p = 0; p < 16; p++) {
                size_t ih = s0 + 2 * p, il = ih + 1;
                uint8_t ch = fp4_code(ih < n ? v[ih] : 0.0f, sc), cl = fp4_code(il < n ? v[il] : 0.0f, sc);
                packed[b * 16 + p] = (uint8_t)((ch << 4) | cl);
            }
        }
    });
    return NNQ_OK;
}

// nn-core OCP MXFP4 quantize_tensor (crates/nn-core/src/layers/quantized/mxfp4.rs:194-220,
// 293-315): 17-byte blocks [shared_exp][16 packed, element 2i in the low nibble of byte
// i], shared_exp = clamp(ceil(log2(max|v| / 6)) + 127, 0, 254) (0 for an all-zero block),
// codes the nearest e2m1 magnitude of |v| / 2^(e - 127) (strict <: ties keep the lower).
int nnq_quantize_mxfp4_ocp(const float *v, size_t n, uint8_t *blocks) {
    if ((!v && n) || (!blocks && n)) return NNQ_ERR_INVALID_ARGUMENT;
    for (size_t i = 0; i < n; i++)
        if (!std::isfinite(v[i])) return nnq::set_error(NNQ_ERR_NON_FINITE, "mxfp4 quantize_block: non-finite input value");
    static const float kMag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
    const size_t nb = (n + 31) / 32;
    parallel_blocks(nb, [&](size_t lo, size_t hi) {
        for (size_t b = lo; b < hi; b++) {
            float x[32];
            float mx = 0.0f;
            for (int i = 0; i < 32; i++) {
                x[i] = b * 32 + i < n ? v[b * 32 + i] : 0.0f;
                const float a = std::fabs(x[i]);
                if (a > mx) mx = a;
            }
            uint8_t e = 0;
            if (mx != 0.0f) {
                const int eb = (int)std::ceil(std::log2(mx / 6.0f)) + 127;
                e = (uint8_t)std::min(254, std::max(0, eb));
            }
            const float scale = (float)std::ldexp(1.0, (int)e - 127);
            uint8_t *blk = blocks + b * 17;
            blk[0] = e;
            for (int p = 0; p < 16; p++) blk[1 + p] = 0;
            for (int i = 0; i < 32; i++) {
                uint8_t code = 0;
                if (x[i] != 0.0f && scale != 0.0f) {
                    const float q = std::fabs(x[i]) / scale;
                    float best = 3.40282347e38f;
                    for (uint8_t j = 0; j < 8; j++) {
                        const float d = std::fabs(q - kMag[j]);
                        if (d < best) {
                            best = d;
                            code = j;
                        }
                    }
                    if (x[i] < 0.0f) code |= 0x8;
                }
                blk[1 + i / 2] |= (i % 2 == 0) ? code : (uint8_t)(code << 4);
            }
        }
    });
    return NNQ_OK;
}

int nnq_quantize_q8_0(const float *v, size_t n, uint8_t *out) {
    if (!v || !out) return NNQ_ERR_INVALID_ARGUMENT;
    if (n % 32) return NNQ_ERR_INVALID_SHAPE;
    parallel_blocks(n / 32, [&](size_t lo, size_t hi) {
        for (size_t b = lo; b < hi; b++) {
            const float *x = v + b * 32;
            float amax = 0.0f;
            for (int j = 0; j < 32; j++) amax = std::max(amax, std::fabs(x[j]));
            float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
            uint16_t dh = to_f16(d);
            uint8_t *p = out + b * 34;
            p[0] = (uint8_t)dh;
            p[1] = (uint8_t)(dh >> 8);
            for (int j = 0; j < 32; j++) {
                float q = std::round(x[j] * id);
                q = std::min(127.0f, std::max(-127.0f, q));
                p[2 + j] = (uint8_t)(int8_t)q;
            }
        }
    });
    return NNQ_OK;
}

int nnq_quantize_q6_k(const float *v, size_t n, uint8_t *out) {
    if (!v || !out) return NNQ_ERR_INVALID_ARGUMENT;
    if (n % 256) return NNQ_ERR_INVALID_SHAPE;
    parallel_blocks(n / 256, [&](size_t lo, size_t hi) {
        for (size_t b = lo; b < hi; b++) {
            const float *x = v + b * 256;
            uint8_t *p = out + b * 210;
            std::memset(p, 0, 210);
            float ss[16], maxs = 0.0f;
            for (int s = 0; s < 16; s++) {
                float amax = 0.0f;
                for (int k = 0; k < 16; k++) amax = std::max(amax, std::fabs(x[16 * s + k]));
                ss[s] = amax / 31.0f;
                maxs = std::max(maxs, ss[s]);
            }
            uint16_t dh = to_f16(maxs / 127.0f);
            float df = from_f16(dh);
            p[208] = (uint8_t)dh;
            p[209] = (uint8_t)(dh >> 8);
            for (int s = 0; s < 16; s++) {
                float scf = df > 0.0f ? std::min(127.0f, std::round(ss[s] / df)) : 0.0f;
                int8_t sc = (int8_t)scf;
                p[192 + s] = (uint8_t)sc;
                float eff = df * (float)sc;
                for (int k = 0; k < 16; k++) {
                    int idx = 16 * s + k, q = 32;
                    if (eff != 0.0f) q = (int)std::min(31.0f, std::max(-32.0f, std::round(x[idx] / eff))) + 32;
                    p[idx / 2] |= (uint8_t)((q & 0x0F) << (4 * (idx % 2)));
                    p[128 + idx / 4] |= (uint8_t)(((q >> 4) & 3) << (2 * (idx % 4)));
                }
            }
        }
    });
    return NNQ_OK;
}

int nnq_synth_normal(uint64_t seed, uint64_t tensor_id, size_t n, double sigma, float *out) {
    if (!out && n) return NNQ_ERR_INVALID_ARGUMENT;
    auto mix = [](uint64_t z) {  // splitmix64, crates/nn-core/src/test_prng.rs:18-22
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    };
    const uint64_t base = seed + tensor_id * 0xD1B54A32D192ED03ull;
    auto uni = [&](uint64_t i) {  // top 53 bits -> [0, 1)
        return (double)(mix(base + i * 0x9E3779B97F4A7C15ull) >> 11) * (1.0 / 9007199254740992.0);
    };
    size_t npairs = (n + 1) / 2;
    parallel_blocks((npairs + 255) / 256, [&](size_t lo, size_t hi) {
        for (size_t blk = lo; blk < hi; blk++)
            for (size_t j = blk * 256; j < std::min(npairs, blk * 256 + 256); j++) {
                double u1 = uni(2 * j), u2 = uni(2 * j + 1);
                double r = std::sqrt(-2.0 * std::log(1.0 - u1));
                double a = 6.283185307179586 * u2;
                out[2 * j] = (float)(sigma * r * std::cos(a));
                if (2 * j + 1 < n) out[2 * j + 1] = (float)(sigma * r * std::sin(a));
            }
    });
    return NNQ_OK;
}

}  // extern "C"
