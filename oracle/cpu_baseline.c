/* CPU baseline of the quantized-linear path (benchmark infrastructure, not product code):
 * the reference's flow restated for bench.py's cpu_baseline leg.  QLinear::forward decodes
 * the whole quantized matrix to f32 and then multiplies (crates/nn-core/src/layers/quantized/
 * linear.rs:366-400 -> crates/nn-core/src/dyn_tensor/ops/matmul.rs:18-52); the decoders here
 * are the oracle's own (nnq_oracle.c, compiled into the same library), run over block ranges
 * under OpenMP, and the f32 product is a register-blocked, cache-blocked loop vectorized by
 * the compiler (-O3, one clone per x86-64 level), standing in for matrixmultiply's sgemm.
 *
 * Decoded values are bit-identical to the oracle's at any thread count; products differ from
 * the oracle's sequential sums by f32 rounding only (another summation order), so this is a
 * speed baseline, never a parity reference.  Only bench.py and tests/ load it. */
#include <omp.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#include "nnq_oracle.h"

int cb_max_threads(void) { return omp_get_max_threads(); }

/* contiguous block ranges, one per thread; every decoder is block-local */
void cb_dequant_q4k(const uint8_t *wb, size_t nblocks, float *out, int threads) {
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t b = 0; b < (int64_t)nblocks; b += 64) {
        const size_t nb = (size_t)((int64_t)nblocks - b < 64 ? (int64_t)nblocks - b : 64);
        orc_dequant_q4_k_gguf(wb + (size_t)b * 144, nb * 144, nb * 256, out + (size_t)b * 256);
    }
}

void cb_dequant_q6k(const uint8_t *wb, size_t nblocks, float *out, int threads) {
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t b = 0; b < (int64_t)nblocks; b += 64) {
        const size_t nb = (size_t)((int64_t)nblocks - b < 64 ? (int64_t)nblocks - b : 64);
        orc_dequant_q6_k_legacy(wb + (size_t)b * 210, nb * 210, nb * 256, out + (size_t)b * 256);
    }
}

void cb_dequant_mxfp4(const uint8_t *packed, const uint8_t *scales, size_t nblocks, float *out, int threads) {
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t b = 0; b < (int64_t)nblocks; b += 1024) {
        const size_t nb = (size_t)((int64_t)nblocks - b < 1024 ? (int64_t)nblocks - b : 1024);
        orc_mxfp4_dequantize(packed + (size_t)b * 16, scales + b, nb, nb * 32, out + (size_t)b * 32);
    }
}

/* ---- f32 product y[m][n] = x[m][k] . w[n][k]^T -------------------------------------- */
#define VW 16
typedef float vf __attribute__((vector_size(VW * 4)));

static inline vf ldv(const float *p) {
    vf v;
    memcpy(&v, p, sizeof v);
    return v;
}
static inline float hsum(vf v) {
    float s = 0.0f;
    for (int i = 0; i < VW; i++) s += v[i];
    return s;
}

/* R rows of x against C rows of w over k in [k0, k1) (k1 - k0 a multiple of VW), added to y */
#define MICRO(R, C)                                                                                        \
    static inline __attribute__((always_inline)) void micro_##R##x##C(const float *x, int64_t ldx, const float *w, int64_t ldw, int64_t k0,      \
                                int64_t k1, float *y, int64_t ldy) {                                       \
        vf acc[R][C];                                                                                      \
        for (int r = 0; r < R; r++)                                                                        \
            for (int c = 0; c < C; c++) acc[r][c] = (vf){0};                                               \
        for (int64_t kk = k0; kk < k1; kk += VW) {                                                         \
            vf wv[C];                                                                                      \
            for (int c = 0; c < C; c++) wv[c] = ldv(w + c * ldw + kk);                                     \
            for (int r = 0; r < R; r++) {                                                                  \
                const vf xv = ldv(x + r * ldx + kk);                                                       \
                for (int c = 0; c < C; c++) acc[r][c] += xv * wv[c];                                       \
            }                                                                                              \
        }                                                                                                  \
        for (int r = 0; r < R; r++)                                                                        \
            for (int c = 0; c < C; c++) y[r * ldy + c] += hsum(acc[r][c]);                                 \
    }
MICRO(4, 4)
MICRO(1, 4)
MICRO(1, 1)
MICRO(4, 1)

/* scalar tail for k not a multiple of VW */
static inline __attribute__((always_inline)) void tail(const float *x, int64_t ldx, int64_t rows, const float *w, int64_t ldw, int64_t cols, int64_t k0,
                 int64_t k1, float *y, int64_t ldy) {
    for (int64_t r = 0; r < rows; r++)
        for (int64_t c = 0; c < cols; c++) {
            float s = 0.0f;
            for (int64_t kk = k0; kk < k1; kk++) s += x[r * ldx + kk] * w[c * ldw + kk];
            y[r * ldy + c] += s;
        }
}

/* Columns j0 .. j1 (rows of w) of y over all of k, in k blocks of 1024 (m >= 4), so the block
 * of w (64 rows, 256 KB) and the x slice stay in the core's caches while every row of x passes.
 * One clone per x86 vector level, picked at load time: the library is built on another host
 * than the one that runs it, so -march=native cannot be used. */
__attribute__((target_clones("avx512f", "avx2", "default"))) static void matmul_cols(
    const float *x, int64_t m, const float *w, int64_t n, int64_t k, float *y, int64_t j0, int64_t j1) {
    const int64_t kv = k / VW * VW, KC = m < 4 ? kv : 1024;  /* a GEMV streams each row whole */
    for (int64_t i = 0; i < m; i++) memset(y + i * n + j0, 0, (size_t)(j1 - j0) * sizeof(float));
    for (int64_t k0 = 0; k0 < kv; k0 += KC) {
        const int64_t k1 = k0 + KC < kv ? k0 + KC : kv;
        int64_t i = 0;
        for (; i + 4 <= m; i += 4) {
            int64_t j = j0;
            for (; j + 4 <= j1; j += 4) micro_4x4(x + i * k, k, w + j * k, k, k0, k1, y + i * n + j, n);
            for (; j < j1; j++) micro_4x1(x + i * k, k, w + j * k, k, k0, k1, y + i * n + j, n);
        }
        for (; i < m; i++) {
            int64_t j = j0;
            for (; j + 4 <= j1; j += 4) micro_1x4(x + i * k, k, w + j * k, k, k0, k1, y + i * n + j, n);
            for (; j < j1; j++) micro_1x1(x + i * k, k, w + j * k, k, k0, k1, y + i * n + j, n);
        }
    }
    if (kv < k) tail(x, k, m, w + j0 * k, k, j1 - j0, kv, k, y + j0, n);
}

/* columns split over the threads in blocks of 64 */
void cb_matmul_xwt(const float *x, int64_t m, const float *w, int64_t n, int64_t k, float *y, int threads) {
    const int64_t NC = 64, nblk = (n + NC - 1) / NC;
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t jb = 0; jb < nblk; jb++) matmul_cols(x, m, w, n, k, y, jb * NC, jb * NC + NC < n ? jb * NC + NC : n);
}

/* ---- f32 product y[m][n] = x[m][k] . w[k][n] (w row-major, as the MoE experts' f32
 * weights are laid out after decoding) ------------------------------------------------
 * Column strips of 4 VW, rows 4 at a time: the strip's accumulators stay in registers
 * over a k block of 256 while each row of w contributes one broadcast FMA per vector. */
__attribute__((target_clones("avx512f", "avx2", "default"))) static void matmul_xw_cols(
    const float *x, int64_t m, const float *w, int64_t k, int64_t n, float *y, int64_t j0, int64_t j1) {
    const int64_t KC = 256;
    for (int64_t i = 0; i < m; i++) memset(y + i * n + j0, 0, (size_t)(j1 - j0) * sizeof(float));
    for (int64_t k0 = 0; k0 < k; k0 += KC) {
        const int64_t k1 = k0 + KC < k ? k0 + KC : k;
        for (int64_t i0 = 0; i0 < m; i0 += 4) {
            const int64_t rows = m - i0 < 4 ? m - i0 : 4;
            int64_t j = j0;
            for (; j + 4 * VW <= j1; j += 4 * VW) {
                vf acc[4][4];
                for (int r = 0; r < 4; r++)
                    for (int c = 0; c < 4; c++) acc[r][c] = (vf){0};
                for (int64_t kk = k0; kk < k1; kk++) {
                    vf wv[4];
                    for (int c = 0; c < 4; c++) wv[c] = ldv(w + kk * n + j + c * VW);
                    for (int r = 0; r < 4; r++) {
                        if (r >= rows) break;
                        const float xs = x[(i0 + r) * k + kk];
                        for (int c = 0; c < 4; c++) acc[r][c] += xs * wv[c];
                    }
                }
                for (int r = 0; r < rows; r++)
                    for (int c = 0; c < 4; c++) {
                        float *yp = y + (i0 + r) * n + j + c * VW;
                        vf yv = ldv(yp);
                        yv += acc[r][c];
                        memcpy(yp, &yv, sizeof yv);
                    }
            }
            for (; j < j1; j++)  /* scalar columns past the last whole strip */
                for (int64_t r = 0; r < rows; r++) {
                    float s = 0.0f;
                    for (int64_t kk = k0; kk < k1; kk++) s += x[(i0 + r) * k + kk] * w[kk * n + j];
                    y[(i0 + r) * n + j] += s;
                }
        }
    }
}

/* columns split over the threads in blocks of 256 */
void cb_matmul_xw(const float *x, int64_t m, const float *w, int64_t k, int64_t n, float *y, int threads) {
    const int64_t NC = 256, nblk = (n + NC - 1) / NC;
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t jb = 0; jb < nblk; jb++) matmul_xw_cols(x, m, w, k, n, y, jb * NC, jb * NC + NC < n ? jb * NC + NC : n);
}

/* QLinear::forward with a Q4_K weight, as the reference runs it: decode all of W into the
 * caller's f32 buffer (allocated once by the caller), then y = x . W^T */
void cb_q4k_qlinear(const uint8_t *wb, int64_t n, int64_t k, const float *x, int64_t m, float *wbuf, float *y,
                    int threads) {
    cb_dequant_q4k(wb, (size_t)(n * k / 256), wbuf, threads);
    cb_matmul_xwt(x, m, wbuf, n, k, y, threads);
}

/* first index of the maximum (argreduce.rs:105-118; the inputs here are finite) */
int64_t cb_argmax(const float *v, int64_t n) {
    int64_t best = 0;
    for (int64_t i = 1; i < n; i++)
        if (v[i] > v[best]) best = i;
    return best;
}
