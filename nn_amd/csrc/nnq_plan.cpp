// Host arithmetic of the C ABI's calls: the byte sizes of token arrays, the layout of a
// call's workspace regions, and how long batches are cut into launches.  It is kept apart
// from nnq_abi.cpp (which makes the HIP runtime calls) so that the sanitizer harness
// (tests/sanitize) runs the same code on the CPU over ragged and extreme shapes.
#include <algorithm>

#include "nnq_internal.h"

namespace nnq {

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

bool array_bytes(int64_t rows, int64_t cols, size_t elem, size_t *out) {
    *out = 0;
    if (rows < 0 || cols < 0) return false;
    size_t a = 0;
    if (__builtin_mul_overflow((size_t)rows, (size_t)cols, &a)) return false;
    return !__builtin_mul_overflow(a, elem, out);
}

bool plan_regions(const size_t *sizes, int n, size_t *offsets, size_t *total) {
    size_t at = 0;
    for (int i = 0; i < n; i++) {
        offsets[i] = at;
        if (sizes[i] == 0) continue;  // an absent region takes no space
        // the next region starts at the 256-byte boundary after this one
        size_t end = 0;
        if (__builtin_add_overflow(at, sizes[i], &end) || end > SIZE_MAX - 255) return false;
        at = align256(end);
    }
    *total = at;
    return true;
}

int64_t moe_chunk_tokens(int64_t tokens, int top_k) {
    if (tokens <= 0 || top_k <= 0) return 0;
    return std::max<int64_t>(1, std::min<int64_t>(tokens, kMoeChunkAssign / top_k));
}

int64_t gemm_chunk_rows(int64_t m, int64_t k) {
    if (m <= 0 || k <= 0) return 0;
    // the GEMMs address an activation plane (and its f32 hi + lo pair) with 32-bit byte
    // offsets: 2 planes * rows * K * 2 bytes stays below 2^31
    const int64_t lim = ((int64_t)1 << 31) - 1;
    int64_t rows = lim / (4 * k);
    if (rows >= 256) rows = rows / 256 * 256;  // whole 256-row tiles per launch
    return std::min(m, std::max<int64_t>(1, rows));
}

}  // namespace nnq
