// Sanitizer harness for the host-side C/C++: the package codec
// (csrc/codec/iqk_codec.cpp) and the C oracle (oracle/iqk_oracle.c), built
// with -fsanitize=address,undefined by tests/test_sanitize.py and run on the
// CPU.  It drives every quantizer and dequantizer over ordinary, degenerate
// and extreme rows (zeros, denormal-sized, huge, a zeroed imatrix span, no
// imatrix) and over random wire bytes, on several worker threads, and checks
// that the codec's dequantization equals the oracle's bit for bit.  Exit
// status 0 means every check passed and no sanitizer fired (sanitizer reports
// abort the run).
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "iqk_codec.h"

extern "C" {
int oracle_dequant_iq2_ks(const void *src, float *dst, int64_t rows, int64_t n);
int oracle_dequant_iq2_k(const void *src, float *dst, int64_t rows, int64_t n);
int oracle_dequant_iq1_s_r4(const void *src, float *dst, int64_t rows, int64_t n);
}

namespace {

struct Member {
    const char *name;
    size_t (*row_size)(int64_t);
    size_t (*quantize)(const float *, void *, int64_t, int64_t, const float *);
    int (*dequantize)(const void *, float *, int64_t, int64_t);
    int (*oracle)(const void *, float *, int64_t, int64_t);
    int width_unit;
};

const Member kMembers[] = {
    {"iq2_ks", iqk_row_size_iq2_ks, iqk_quantize_iq2_ks, iqk_dequantize_iq2_ks, oracle_dequant_iq2_ks, 256},
    {"iq2_k", iqk_row_size_iq2_k, iqk_quantize_iq2_k, iqk_dequantize_iq2_k, oracle_dequant_iq2_k, 256},
    {"iq1_s_r4", iqk_row_size_iq1_s_r4, iqk_quantize_iq1_s_r4, iqk_dequantize_iq1_s_r4, oracle_dequant_iq1_s_r4, 32},
};

int failures = 0;

void fail(const char *what, const Member &m, int64_t n, const char *kind) {
    std::fprintf(stderr, "FAIL %s: %s n=%lld rows=%s\n", what, m.name, (long long)n, kind);
    ++failures;
}

// Dequantize `wire` with the codec and the oracle; the floats must match bit
// for bit, except that any two NaNs match (the oracle decodes a NaN scale to
// the canonical NaN, the codec keeps its payload).
void compare(const Member &m, const std::vector<uint8_t> &wire, int64_t rows, int64_t n, const char *kind) {
    std::vector<float> a(static_cast<size_t>(rows * n)), b(static_cast<size_t>(rows * n));
    if (m.dequantize(wire.data(), a.data(), rows, n) != 0) return fail("codec dequantize refused", m, n, kind);
    if (m.oracle(wire.data(), b.data(), rows, n) != 0) return fail("oracle dequantize refused", m, n, kind);
    for (size_t i = 0; i < a.size(); ++i) {
        if (std::isnan(a[i]) && std::isnan(b[i])) continue;
        if (std::memcmp(&a[i], &b[i], sizeof(float)) != 0) return fail("codec != oracle", m, n, kind);
    }
}

void rows_of(const char *kind, std::mt19937 &rng, int64_t rows, int64_t n, std::vector<float> &w) {
    std::normal_distribution<float> normal(0.f, 0.02f);
    w.resize(size_t(rows * n));
    for (size_t i = 0; i < w.size(); ++i) {
        const float v = normal(rng);
        if (!std::strcmp(kind, "normal")) w[i] = v;
        else if (!std::strcmp(kind, "zeros")) w[i] = 0.f;
        else if (!std::strcmp(kind, "tiny")) w[i] = v * 1e-36f;      // scales underflow fp16
        else if (!std::strcmp(kind, "huge")) w[i] = v * 1e36f;       // block sums overflow float
        else if (!std::strcmp(kind, "large")) w[i] = v * 1e22f;      // squared distances overflow float
        else if (!std::strcmp(kind, "sparse")) w[i] = (i % 61) ? 0.f : v;  // mostly-zero blocks
        else w[i] = (i % 2) ? v : -v;                                // alternating signs
    }
}

}  // namespace

int main() {
    iqk_codec_set_threads(4);
    std::mt19937 rng(12345);
    const char *kinds[] = {"normal", "zeros", "tiny", "large", "huge", "sparse", "alternating"};
    for (const Member &m : kMembers) {
        for (int64_t n : {int64_t(m.width_unit), int64_t(2048)}) {
            const int64_t rows = 8;  // two IQ1_S_R4 four-row groups
            const size_t rb = m.row_size(n);
            if (rb == 0) { fail("row size refused", m, n, "-"); continue; }
            std::vector<float> imatrix(static_cast<size_t>(n));
            std::uniform_real_distribution<float> uni(0.1f, 1.0f);
            for (auto &v : imatrix) v = uni(rng);
            for (int64_t k = 0; k < std::min<int64_t>(n, 40); ++k) imatrix[size_t(k)] = 0.f;  // a zeroed span
            for (const char *kind : kinds) {
                std::vector<float> w;
                rows_of(kind, rng, rows, n, w);
                for (int with_imatrix = 0; with_imatrix < 2; ++with_imatrix) {
                    std::vector<uint8_t> wire(rb * size_t(rows));
                    const size_t wrote = m.quantize(w.data(), wire.data(), rows, n, with_imatrix ? imatrix.data() : nullptr);
                    // IQ1_S_R4 refuses rows whose block sums overflow float (its
                    // search finds no candidate), as the reference's quantizer
                    // does (vendor/ik_llama/iqk_iq1sr4.cpp:445, 548)
                    const bool may_refuse = m.width_unit == 32 && (!std::strcmp(kind, "huge") || !std::strcmp(kind, "large"));
                    if (wrote == 0 && may_refuse) continue;
                    if (wrote != wire.size()) { fail("quantize size", m, n, kind); continue; }
                    compare(m, wire, rows, n, kind);
                }
            }
            // random wire bytes: every field value, including non-finite scales
            std::vector<uint8_t> wire(rb * size_t(rows));
            std::uniform_int_distribution<int> byte(0, 255);
            for (auto &b : wire) b = uint8_t(byte(rng));
            compare(m, wire, rows, n, "random-wire");
        }
        // refused geometry: nothing written, nothing read
        if (m.row_size(m.width_unit + 1) != 0) fail("odd width accepted", m, m.width_unit + 1, "-");
    }
    if (iqk_quantize_iq1_s_r4(nullptr, nullptr, 3, 2048, nullptr) != 0) fail("3 IQ1 rows accepted", kMembers[2], 2048, "-");
    std::printf("sanitize harness: %d failure(s)\n", failures);
    return failures ? 1 : 0;
}
