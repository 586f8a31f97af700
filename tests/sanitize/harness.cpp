// Host code of the nnq library and the CPU oracle under AddressSanitizer and
// UndefinedBehaviorSanitizer (built by tests/sanitize/Makefile with ROCm's clang as a
// plain host compiler; no device code is built or run).
//
// Covered: the GGUF reader on a valid file and on thousands of mutated copies of it
// (bit flips, byte overwrites with extreme values, truncations, grown length fields),
// including tensor-data lookups and the device-weight path up to the repack; the repacks
// of every weight format and layout over random bytes and ragged shapes; the host
// encoders over random, zero, tiny, huge and non-finite inputs; the ABI calls' size,
// workspace-layout and chunking arithmetic (nnq_plan.cpp) over random and extreme
// shapes; and the oracle's decoders, linears, MoE and sampling on small random cases.
// Any sanitizer report aborts the run (exit code != 0).
//
// nnq_abi.cpp (HIP) is not linked: this file provides the two symbols the host sources
// take from it, with nnq_weight_create validating as the library does and then running
// the real layout and repack code into host memory instead of uploading.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include <unistd.h>

#include "../../nn_amd/csrc/nnq_internal.h"

extern "C" {
#include "../../oracle/nnq_oracle.h"
}

namespace nnq {
thread_local std::string g_err;
int set_error(int code, const char *msg) {
    g_err = msg;
    return code;
}
}  // namespace nnq

struct nnq_weight {
    std::vector<uint8_t> image;
};

static size_t blk_elems(int fmt) { return fmt == NNQ_FMT_Q8_0 ? 32 : 256; }
static size_t blk_bytes(int fmt) { return fmt == NNQ_FMT_Q8_0 ? 34 : (fmt == NNQ_FMT_Q4_K ? 144 : 210); }

extern "C" int nnq_weight_create(nnq_format fmt, nnq_layout layout, const uint8_t *bytes, size_t nbytes, int64_t n,
                                 int64_t k, nnq_weight **out) {
    *out = nullptr;
    if (fmt != NNQ_FMT_Q8_0 && fmt != NNQ_FMT_Q4_K && fmt != NNQ_FMT_Q6_K) return NNQ_ERR_WRONG_FORMAT;
    if (n <= 0 || k <= 0) return NNQ_ERR_INVALID_ARGUMENT;
    if ((size_t)k % blk_elems(fmt)) return NNQ_ERR_INVALID_SHAPE;
    if (nbytes != (size_t)n * ((size_t)k / blk_elems(fmt)) * blk_bytes(fmt)) return NNQ_ERR_DATA_LENGTH;
    nnq::Layout L;
    const char *err = nullptr;
    if (!nnq::make_layout(fmt, layout, n, k, &L, &err)) return NNQ_ERR_WRONG_FORMAT;
    nnq_weight *w = new nnq_weight;
    w->image.assign(L.total(), 0);
    uint8_t *d = w->image.data();
    if (fmt == NNQ_FMT_Q4_K) {
        nnq::repack_q4k(bytes, layout == NNQ_LAYOUT_NN_GGUF, L, d);
        nnq::q4k_aux_plane(d + L.qs_bytes, L, d + L.qs_bytes + L.hdr_bytes, 0, L.ntile);
    } else if (fmt == NNQ_FMT_Q6_K) {
        nnq::repack_q6k(bytes, L, d);
    } else {
        nnq::repack_q8_0(bytes, L, d);
    }
    *out = w;
    return NNQ_OK;
}

static std::mt19937_64 rng(20261202);

static void put(std::vector<uint8_t> &b, const void *p, size_t n) {
    const uint8_t *q = static_cast<const uint8_t *>(p);
    b.insert(b.end(), q, q + n);
}
template <class T>
static void put(std::vector<uint8_t> &b, T v) {
    put(b, &v, sizeof v);
}
static void put_str(std::vector<uint8_t> &b, const std::string &s) {
    put<uint64_t>(b, s.size());
    put(b, s.data(), s.size());
}

// a valid GGUF v3 file: metadata of every scalar type, a string, an array of strings, a
// nested array; Q4_K, Q6_K and Q8_0 tensors with random block bytes
static std::vector<uint8_t> valid_gguf() {
    std::vector<uint8_t> b;
    put<uint32_t>(b, 0x46554747u);
    put<uint32_t>(b, 3);
    put<uint64_t>(b, 3);   // tensors
    put<uint64_t>(b, 14);  // metadata
    const uint32_t scalar_types[] = {0, 1, 2, 3, 4, 5, 6, 7, 10, 11, 12};
    const size_t sizes[] = {1, 1, 2, 2, 4, 4, 4, 1, 8, 8, 8};
    for (int i = 0; i < 11; i++) {
        put_str(b, "key." + std::to_string(i));
        put<uint32_t>(b, scalar_types[i]);
        uint64_t v = rng();
        put(b, &v, sizes[i]);
    }
    put_str(b, "general.architecture");
    put<uint32_t>(b, 8);
    put_str(b, "qwen3");
    put_str(b, "tokens");
    put<uint32_t>(b, 9);
    put<uint32_t>(b, 8);
    put<uint64_t>(b, 3);
    for (const char *t : {"a", "bc", "def"}) put_str(b, t);
    put_str(b, "nested");
    put<uint32_t>(b, 9);
    put<uint32_t>(b, 9);
    put<uint64_t>(b, 2);
    for (int i = 0; i < 2; i++) {
        put<uint32_t>(b, 4);
        put<uint64_t>(b, 2);
        put<uint32_t>(b, 7);
        put<uint32_t>(b, 9);
    }
    struct T { const char *name; uint32_t type; uint64_t ne0, ne1, bytes; };
    const T ts[] = {{"blk.0.ffn_down.weight", 12, 512, 32, 32 * 2 * 144},
                    {"output.weight", 14, 256, 48, 48 * 210},
                    {"blk.0.attn_q.weight", 8, 64, 16, 16 * 2 * 34}};
    uint64_t off = 0;
    for (const T &t : ts) {
        put_str(b, t.name);
        put<uint32_t>(b, 2);
        put<uint64_t>(b, t.ne0);
        put<uint64_t>(b, t.ne1);
        put<uint32_t>(b, t.type);
        put<uint64_t>(b, off);
        off += (t.bytes + 31) / 32 * 32;
    }
    while (b.size() % 32) b.push_back(0);
    const size_t base = b.size();
    b.resize(base + off);
    for (size_t i = base; i < b.size(); i++) b[i] = (uint8_t)rng();
    // finite f16 scales (d, dmin of Q4_K; d of Q6_K; d of Q8_0)
    for (size_t i = base; i + 1 < b.size(); i += 2) b[i + 1] &= 0x3B;
    return b;
}

// every query on an opened file, and the device-weight path for every tensor
static void exercise(const nnq_gguf *g) {
    uint32_t ver;
    int64_t nt, nkv;
    uint64_t doff;
    nnq_gguf_info(g, &ver, &nt, &nkv, &doff);
    for (int64_t i = -1; i <= nt; i++) {
        const char *name = nullptr;
        int32_t nd = 0;
        uint64_t dims[8], off, nb;
        uint32_t dt;
        if (nnq_gguf_tensor_info(g, i, &name, &nd, dims, &dt, &off, &nb) != NNQ_OK) continue;
        const uint8_t *data;
        uint64_t n;
        if (nnq_gguf_tensor_data(g, name, &data, &n) == NNQ_OK) {
            volatile uint8_t sink = 0;
            for (uint64_t j = 0; j < n; j += 61) sink ^= data[j];
            if (n) sink ^= data[n - 1];
        }
        for (int order = 0; order < 2; order++)
            for (int lay = 0; lay < 2; lay++) {
                nnq_weight *w = nullptr;
                if (nnq_gguf_weight_create(g, name, (nnq_layout)lay, order, &w) == NNQ_OK) delete w;
            }
    }
    for (const char *key : {"general.architecture", "tokens", "nested", "key.3", "key.10", "missing"}) {
        uint32_t type, at;
        uint64_t u, ac;
        int64_t iv;
        double f;
        const char *str;
        nnq_gguf_metadata(g, key, &type, &u, &iv, &f, &str, &at, &ac);
    }
}

static int fuzz_gguf(int iters, const char *dir) {
    const std::vector<uint8_t> seed = valid_gguf();
    const std::string path = std::string(dir) + "/fuzz.gguf";
    int opened = 0;
    for (int it = 0; it < iters; it++) {
        std::vector<uint8_t> b = seed;
        if (it > 0) {
            const int muts = 1 + (int)(rng() % 6);
            for (int k = 0; k < muts; k++) {
                const size_t pos = rng() % b.size();
                switch (rng() % 6) {
                case 0: b[pos] ^= (uint8_t)(1u << (rng() % 8)); break;
                case 1: b[pos] = (uint8_t)rng(); break;
                case 2: {  // an extreme 64-bit value (lengths, counts, offsets, dims)
                    const uint64_t vals[] = {0, 1, 0x7FFFFFFFull, 0xFFFFFFFFull, 0x8000000000000000ull, ~0ull,
                                             (uint64_t)1 << 33, 100001, 16777217};
                    const uint64_t v = vals[rng() % 9];
                    for (int j = 0; j < 8 && pos + j < b.size(); j++) b[pos + j] = (uint8_t)(v >> (8 * j));
                    break;
                }
                case 3: b.resize(pos); break;
                case 4: b.insert(b.begin() + (ptrdiff_t)pos, (size_t)(rng() % 64), (uint8_t)rng()); break;
                default: b.erase(b.begin() + (ptrdiff_t)pos, b.begin() + (ptrdiff_t)std::min(b.size(), pos + 1 + rng() % 16));
                }
                if (b.empty()) b.push_back(0);
            }
        }
        FILE *f = std::fopen(path.c_str(), "wb");
        if (!f) return 2;
        std::fwrite(b.data(), 1, b.size(), f);
        std::fclose(f);
        nnq_gguf *g = nullptr;
        if (nnq_gguf_open(path.c_str(), &g) == NNQ_OK) {
            opened++;
            exercise(g);
            nnq_gguf_close(g);
        }
    }
    unlink(path.c_str());
    std::printf("gguf: %d files, %d opened\n", iters, opened);
    return opened >= 1 ? 0 : 3;  // the unmutated file must open
}

static std::vector<uint8_t> rand_bytes(size_t n) {
    std::vector<uint8_t> v(n);
    for (auto &x : v) x = (uint8_t)rng();
    return v;
}

static int repacks() {
    const int64_t shapes[][2] = {{1, 256}, {16, 256}, {17, 512}, {37, 1024}, {300, 4096}, {5, 32}, {3, 320}};
    int done = 0;
    for (auto &s : shapes)
        for (int fmt : {NNQ_FMT_Q8_0, NNQ_FMT_Q4_K, NNQ_FMT_Q6_K})
            for (int lay : {NNQ_LAYOUT_GGUF, NNQ_LAYOUT_NN_GGUF}) {
                const int64_t n = s[0], k = s[1];
                if (k % (int64_t)blk_elems(fmt)) continue;
                auto b = rand_bytes((size_t)n * (k / blk_elems(fmt)) * blk_bytes(fmt));
                nnq_weight *w = nullptr;
                if (nnq_weight_create((nnq_format)fmt, (nnq_layout)lay, b.data(), b.size(), n, k, &w) == NNQ_OK) {
                    delete w;
                    done++;
                }
            }
    // MoE repack of both MXFP4 layouts
    for (int64_t E : {1, 3})
        for (int64_t K : {32, 96})
            for (int64_t N : {32, 160}) {
                auto packed = rand_bytes((size_t)E * K * N / 2), scales = rand_bytes((size_t)E * K * N / 32);
                std::vector<uint8_t> dc(packed.size()), ds(scales.size());
                nnq::moe_repack(packed.data(), scales.data(), E, K, N, dc.data(), ds.data(), true);
                auto blocks = rand_bytes((size_t)E * K * N / 32 * 17);
                nnq::ocp_split(blocks.data(), (size_t)E * K * N / 32, packed.data(), scales.data());
                nnq::moe_repack(packed.data(), scales.data(), E, K, N, dc.data(), ds.data(), false);
                done++;
            }
    std::printf("repack: %d weights\n", done);
    return 0;
}

static int encoders() {
    const float specials[] = {0.0f, -0.0f, 1e-45f, -1e-40f, 1e-30f, 3.4e38f, -3.4e38f, INFINITY, -INFINITY, NAN};
    for (size_t n : {(size_t)0, (size_t)1, (size_t)31, (size_t)256, (size_t)1000, (size_t)4096}) {
        std::normal_distribution<float> nd(0.0f, 1.0f);
        std::vector<float> v(n);
        for (auto &x : v) x = nd(rng) * std::pow(10.0f, (float)((int)(rng() % 60) - 30));
        for (int pass = 0; pass < 3; pass++) {
            if (pass == 1)
                for (size_t i = 0; i < n; i += 7) v[i] = specials[rng() % 10];
            if (pass == 2)
                for (auto &x : v) x = 0.0f;
            std::vector<uint8_t> o4((n + 255) / 256 * 144), om((n + 31) / 32 * 16), os((n + 31) / 32),
                oc((n + 31) / 32 * 17);
            nnq_quantize_q4_k(v.data(), n, o4.data());
            nnq_quantize_mxfp4(v.data(), n, om.data(), os.data());
            nnq_quantize_mxfp4_ocp(v.data(), n, oc.data());
            if (n % 32 == 0) {
                std::vector<uint8_t> o8(n / 32 * 34);
                nnq_quantize_q8_0(v.data(), n, o8.data());
            }
            if (n % 256 == 0) {
                std::vector<uint8_t> o6(n / 256 * 210);
                nnq_quantize_q6_k(v.data(), n, o6.data());
            }
        }
    }
    std::vector<float> g(1000);
    nnq_synth_normal(1, 2, g.size(), 0.5, g.data());
    std::printf("encoders: done\n");
    return 0;
}

static int oracle() {
    const size_t n = 8, k = 512, m = 3;
    std::vector<float> x(m * k), y(m * n), w(n * k);
    for (auto &v : x) v = (float)((int64_t)(rng() % 2001) - 1000) / 500.0f;
    auto b4 = rand_bytes(n * k / 256 * 144), b6 = rand_bytes(n * k / 256 * 210), b8 = rand_bytes(n * k / 32 * 34);
    for (size_t i = 0; i < b4.size(); i += 144) b4[i + 1] &= 0x3B, b4[i + 3] &= 0x3B;
    for (size_t i = 0; i < b6.size(); i += 210) b6[i + 209] &= 0x3B;
    for (size_t i = 0; i < b8.size(); i += 34) b8[i + 1] &= 0x3B;
    orc_q4k_linear(x.data(), m, k, b4.data(), n, y.data());
    orc_q6k_linear(x.data(), m, k, b6.data(), n, y.data());
    orc_q8_0_matmul(x.data(), m, k, b8.data(), n, y.data());
    orc_dequant_q4_k_legacy(b4.data(), b4.size(), n * k, w.data());
    orc_dequant_q4_k_gguf(b4.data(), b4.size() - 7, n * k, w.data());  // a short buffer decodes what it holds
    std::vector<uint8_t> q(n * k / 256 * 144);
    orc_quantize_q4_k(x.data(), 256, q.data());
    std::vector<uint8_t> oc(k / 32 * 17);
    orc_ocp_quantize_tensor(x.data(), k, oc.data());
    orc_ocp_dequantize_tensor(oc.data(), k, w.data());
    // MoE and sampling
    const size_t E = 4, H = 64, I = 32, T = 5, K = 2;
    auto gp = rand_bytes(E * H * 2 * I / 2), gs = rand_bytes(E * H * 2 * I / 32), dp = rand_bytes(E * I * H / 2),
         ds = rand_bytes(E * I * H / 32);
    for (auto &s : gs) s = 120 + s % 10;
    for (auto &s : ds) s = 120 + s % 10;
    std::vector<float> xe(T * H, 0.5f), lg(T * E), gb(E * 2 * I, 0.01f), db(E * H, 0.01f), out(T * H), tw(T * K);
    std::vector<uint32_t> ti(T * K);
    for (auto &v : lg) v = (float)(rng() % 100) / 25.0f;
    orc_moe_forward_mxfp4(xe.data(), T, H, lg.data(), E, K, gp.data(), gs.data(), gb.data(), dp.data(), ds.data(),
                          db.data(), I, 7.0f, 1, out.data(), ti.data(), tw.data());
    std::vector<float> logits(5000);
    for (auto &v : logits) v = (float)((int64_t)(rng() % 2001) - 1000) / 100.0f;
    logits[3] = INFINITY;
    logits[4] = NAN;
    const uint32_t past[] = {1, 1, 4999, 7000};
    uint32_t tok;
    for (int64_t topk : {-1, 0, 1, 50, 6000})
        orc_sample_token(logits.data(), logits.size(), past, 4, 0.8f, topk, 1, 0.9f, 1.3f, 0.2f, 42, &tok);
    std::printf("oracle: done\n");
    return 0;
}


// nnq_plan.cpp: array sizes, workspace regions, MoE token chunks and GEMM row chunks, as
// the ABI calls use them, over random and extreme shapes (UBSan checks the signed
// arithmetic; the properties below check the results)
static int plans() {
    auto bad = [](const char *what, long long a, long long b) {
        std::fprintf(stderr, "plan check failed: %s (%lld, %lld)\n", what, a, b);
        return 1;
    };
    const int64_t edge[] = {0, 1, 2, 3, 15, 16, 17, 255, 256, 4095, 4096, 12288, 65535, (int64_t)1 << 31,
                            ((int64_t)1 << 32) + 7, (int64_t)1 << 40, INT64_MAX / 2, INT64_MAX};
    std::uniform_int_distribution<int64_t> small(0, 1 << 20);
    for (int it = 0; it < 20000; it++) {
        const int64_t r = it < 400 ? edge[it % 18] : small(rng), c = it < 400 ? edge[(it / 18) % 18] : small(rng);
        const size_t el = (size_t)1 << (it % 4);
        size_t got = 0;
        const bool ok = nnq::array_bytes(r, c, el, &got);
        const unsigned __int128 exact = (unsigned __int128)(uint64_t)r * (uint64_t)c * el;
        if (ok != (exact <= SIZE_MAX)) return bad("array_bytes overflow flag", r, c);
        if (ok && got != (size_t)exact) return bad("array_bytes value", r, c);
        if (nnq::array_bytes(-1 - r, c, el, &got)) return bad("array_bytes negative", r, c);
    }
    std::uniform_int_distribution<int> nreg(1, 6);
    for (int it = 0; it < 20000; it++) {
        size_t sz[6], off[6], total = 0;
        const int n = nreg(rng);
        for (int i = 0; i < n; i++) {
            const int kind = (int)(rng() % 5);
            sz[i] = kind == 0 ? 0 : kind == 1 ? rng() % 512 : kind == 2 ? rng() % (1u << 30)
                  : kind == 3 ? (size_t)(rng() % 4096) * 256 : SIZE_MAX - rng() % 1024;
        }
        unsigned __int128 at = 0;
        bool fits = true;
        for (int i = 0; i < n; i++) {
            if (sz[i] == 0) continue;
            at = (at + sz[i] + 255) / 256 * 256;
            if (at > SIZE_MAX) fits = false;
        }
        const bool ok = nnq::plan_regions(sz, n, off, &total);
        if (ok != fits) return bad("plan_regions overflow flag", n, (long long)fits);
        if (!ok) continue;
        size_t end = 0;
        for (int i = 0; i < n; i++) {
            if (off[i] % 256) return bad("region alignment", i, (long long)off[i]);
            if (sz[i] == 0) continue;
            if (off[i] < end) return bad("regions overlap", i, (long long)off[i]);
            end = off[i] + sz[i];
            if (end > total) return bad("region past the total", i, (long long)end);
        }
    }
    for (int64_t T : {(int64_t)0, (int64_t)1, (int64_t)7, (int64_t)4095, (int64_t)4096, (int64_t)4097,
                      (int64_t)100000, (int64_t)1 << 40}) {
        for (int k : {1, 2, 3, 4, 8, 9, 16, 100, 4096, 16384, 16385, 1 << 20}) {
            const int64_t tc = nnq::moe_chunk_tokens(T, k);
            if (T == 0) {
                if (tc != 0) return bad("moe chunk of no tokens", T, k);
                continue;
            }
            if (tc < 1 || tc > T) return bad("moe chunk range", T, k);
            if (k <= nnq::kMoeChunkAssign && tc * k > nnq::kMoeChunkAssign) return bad("moe chunk assignments", T, k);
            int64_t covered = 0, launches = 0;
            for (int64_t t0 = 0; t0 < T && launches < 3; t0 += tc, launches++) covered = std::min(T, t0 + tc);
            if (launches < 3 && covered != T) return bad("moe chunks cover the batch", T, k);
        }
    }
    for (int64_t K : {(int64_t)32, (int64_t)256, (int64_t)4096, (int64_t)12288, (int64_t)32768, (int64_t)1 << 20,
                      (int64_t)1 << 26, (int64_t)1 << 30}) {
        for (int64_t m : {(int64_t)1, (int64_t)9, (int64_t)512, (int64_t)43690, (int64_t)43691, (int64_t)200000,
                          (int64_t)1 << 35}) {
            const int64_t mc = nnq::gemm_chunk_rows(m, K);
            if (mc < 1 || mc > m) return bad("gemm chunk range", m, K);
            if (4 * mc * K >= ((int64_t)1 << 31) && mc > 1) return bad("gemm chunk 32-bit offsets", m, K);
            if (mc < m && mc >= 256 && mc % 256) return bad("gemm chunk whole tiles", m, K);
        }
    }
    std::printf("plans: done\n");
    return 0;
}

int main(int argc, char **argv) {
    const int iters = argc > 1 ? std::atoi(argv[1]) : 3000;
    const char *dir = argc > 2 ? argv[2] : "/tmp";
    int rc = fuzz_gguf(iters, dir);
    if (!rc) rc = repacks();
    if (!rc) rc = encoders();
    if (!rc) rc = plans();
    if (!rc) rc = oracle();
    std::printf("%s\n", rc ? "FAILED" : "OK");
    return rc;
}
