// CPU codec for the routed IQ_K members (IQ2_KS, IQ2_K, IQ1_S_R4).
//
// The quantizers reproduce ik_llama's portable search bit for bit, so every
// float operation below is written in the order ik evaluates it: C evaluates
// `a * b * c` as `(a * b) * c` and `a + b + c` as `(a + b) + c`, and the bytes
// depend on that.  The build uses plain IEEE single precision (no fast-math,
// no FMA contraction: x86-64 without -mfma has no fused multiply-add).
//
// Algorithms restated (reference file:line):
//   row weights        vendor/ik_llama/iqk_iq2.cpp:105-135
//   make_qx_quants     vendor/ik_llama/iqk_iq2.cpp:154-196
//   IQ2_K quantizer    vendor/ik_llama/iqk_iq2.cpp:205-346
//   IQ2_KS quantizer   vendor/ik_llama/iqk_iq2.cpp:349-499
//   IQ2 dequantizers   vendor/ik_llama/iqk_iq2.cpp:502-562
//   IQ1_S tables       vendor/ik_llama/iqk_iq1sr4.cpp:248-342
//   IQ1_S block search vendor/ik_llama/iqk_iq1sr4.cpp:344-479
//   IQ1_S_R4 quantizer vendor/ik_llama/iqk_iq1sr4.cpp:490-577
//   IQ1_S_R4 dequant   vendor/ik_llama/iqk_iq1sr4.cpp:581-602

#include "iqk_codec.h"

#include <algorithm>
#include <atomic>
#include <cfloat>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <thread>
#include <utility>
#include <vector>

#include "../iq1s_grid.h"

namespace {

constexpr int kQK = 256;
constexpr int kIq2ksBlock = 70;  // extra u16, scales[4], qs[64]
constexpr int kIq2kBlock = 76;   // d f16, extra u16, scales[8], qs[64]
constexpr int kIq1Block = 24;    // qs[16], qh[4] u16 (four rows)
constexpr float kIq1Delta = 0.125f;

const int8_t kValues[8] = {-31, -13, 1, 17, -26, -8, 6, 22};

// ---------------------------------------------------------------- fp16 ----

float half_to_float(uint16_t h) {
    const uint32_t sign = uint32_t(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);
    } else if (exp != 0) {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    } else if (man == 0) {
        bits = sign;
    } else {  // subnormal: normalise
        int e = -1;
        do { man <<= 1; ++e; } while (!(man & 0x400u));
        bits = sign | (uint32_t(112 - e) << 23) | ((man & 0x3ffu) << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// Round-to-nearest-even float -> half, subnormals and overflow included.
uint16_t float_to_half(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint16_t sign = uint16_t((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {  // inf / nan
        return sign | 0x7c00u | (ax > 0x7f800000u ? uint16_t(0x200u | ((ax >> 13) & 0x3ffu)) : 0);
    }
    const int e = int(ax >> 23) - 127;
    const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    if (e >= -14) {
        if (e > 15) return sign | 0x7c00u;
        uint32_t h = (uint32_t(e + 15) << 10) | ((ax & 0x7fffffu) >> 13);
        const uint32_t rem = ax & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;  // may carry into inf
        return sign | uint16_t(h);
    }
    // subnormal half: value = m * 2^(e-23) = q * 2^-24 with q = m >> s
    const int s = -e - 1;
    if (s > 24) return sign;
    uint32_t q = m >> s;
    const uint32_t rem = m & ((1u << s) - 1u);
    const uint32_t halfway = 1u << (s - 1);
    if (rem > halfway || (rem == halfway && (q & 1u))) ++q;
    return sign | uint16_t(q);
}

uint16_t load_u16(const uint8_t *p) { return uint16_t(p[0] | (p[1] << 8)); }
void store_u16(uint8_t *p, uint16_t v) { p[0] = uint8_t(v); p[1] = uint8_t(v >> 8); }

// ------------------------------------------------------------- helpers ----

inline int nearest_int(float fval) {
    float val = fval + 12582912.f;
    int i;
    std::memcpy(&i, &val, sizeof(int));
    return (i & 0x007fffff) - 0x00400000;
}

// Per-row importance weights from a per-column imatrix: a block whose weight
// mass, value mass or cross term sits at the epsilon floor becomes uniform
// 1e-9 (the reference's degeneracy guard).
void row_weights(const float *imatrix, const float *x, int n, int block, float *out) {
    const float eps = 1e-9f;
    const float eps2 = eps * eps;
    for (int ib = 0; ib < n / block; ++ib) {
        const float *w_in = imatrix + ib * block;
        const float *xb = x + ib * block;
        float *wb = out + ib * block;
        float sw2 = 0, sx2 = 0, swx = 0;
        for (int j = 0; j < block; ++j) {
            wb[j] = w_in[j];
            sw2 += wb[j] * wb[j];
            sx2 += xb[j] * xb[j];
            swx += wb[j] * std::abs(xb[j]);
        }
        const float floor_ = block * eps2;
        if (sw2 > floor_ && sx2 > floor_ && swx > floor_) continue;
        for (int j = 0; j < block; ++j) wb[j] = eps;
    }
}

// Best symmetric integer scale for x with levels [-nmax, nmax-1]; writes the
// levels (offset by nmax) to L and returns the scale.
float best_int_scale(int n, int nmax, const float *x, int8_t *L, const float *w) {
    float max = 0, amax = 0;
    for (int i = 0; i < n; ++i) {
        const float ax = std::fabs(x[i]);
        if (ax > amax) { amax = ax; max = x[i]; }
    }
    if (!amax) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.f;
    }
    auto level = [nmax](float v) { return std::max(-nmax, std::min(nmax - 1, nearest_int(v))); };
    float iscale = -nmax / max;
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < n; ++i) {
        const int l = level(iscale * x[i]);
        L[i] = int8_t(l + nmax);
        sumlx += w[i] * x[i] * l;
        suml2 += w[i] * l * l;
    }
    float scale = suml2 ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    for (int step = -9; step <= 9; ++step) {
        if (step == 0) continue;
        iscale = -(nmax + 0.1f * step) / max;
        sumlx = suml2 = 0;
        for (int i = 0; i < n; ++i) {
            const int l = level(iscale * x[i]);
            sumlx += w[i] * x[i] * l;
            suml2 += w[i] * l * l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; ++i) L[i] = int8_t(nmax + level(iscale * x[i]));
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

inline int nearest_level(const int8_t *v, float x) {
    const int i = x < v[1] ? 0 : x > v[2] ? 2 : 1;
    return x - v[i] < v[i + 1] - x ? i : i + 1;
}

// Per-weight search weights of a sub-block.
inline void search_weights(const float *qw, const float *xb, int count, float sigma2, float *out) {
    if (qw) {
        for (int j = 0; j < count; ++j) out[j] = qw[j] * sqrtf(sigma2 + xb[j] * xb[j]);
    } else {
        for (int j = 0; j < count; ++j) out[j] = 0.25f * sigma2 + xb[j] * xb[j];
    }
}

// Exhaustive 3-boundary search over the sorted sub-block: every split of the
// sorted values into four runs, each run mapped to one alphabet entry, in
// both alphabets and both orientations.  Returns the best scale and sets
// `shifted`.  i1 < i1_end, i3 >= i3_min (IQ2_KS prunes, IQ2_K does not).
template <int B>
float alphabet_search(const float *xb, const float *weight, int i1_end, int i3_min, bool *shifted) {
    std::pair<float, int> order[B];
    for (int j = 0; j < B; ++j) order[j] = {xb[j], j};
    std::sort(order, order + B);
    float sx[B + 1], sw[B + 1];
    sx[0] = sw[0] = 0;
    for (int j = 0; j < B; ++j) {
        const int k = order[j].second;
        sw[j + 1] = sw[j] + weight[k];
        sx[j + 1] = sx[j] + weight[k] * xb[k];
    }
    const float a[4] = {float(kValues[0]), float(kValues[1]), float(kValues[2]), float(kValues[3])};
    const float s[4] = {float(kValues[4]), float(kValues[5]), float(kValues[6]), float(kValues[7])};
    float best = 0, d = 0;
    bool sh = false;
    auto consider = [&](const float *v, bool vshift, float x0, float x1, float x2, float x3,
                        float w0, float w1, float w2, float w3, int o0, int o1, int o2, int o3) {
        const float sumqx = x0 * v[o0] + x1 * v[o1] + x2 * v[o2] + x3 * v[o3];
        const float sumq2 = w0 * v[o0] * v[o0] + w1 * v[o1] * v[o1] + w2 * v[o2] * v[o2] +
                            w3 * v[o3] * v[o3];
        if (sumq2 > 0 && sumqx * sumqx > best * sumq2) {
            d = sumqx / sumq2;
            best = d * sumqx;
            sh = vshift;
        }
    };
    for (int i1 = 0; i1 < i1_end; ++i1) {
        for (int i2 = i1; i2 < B; ++i2) {
            for (int i3 = std::max(i2, i3_min); i3 < B; ++i3) {
                const float x0 = sx[i1] - sx[0], x1 = sx[i2] - sx[i1];
                const float x2 = sx[i3] - sx[i2], x3 = sx[B] - sx[i3];
                const float w0 = sw[i1] - sw[0], w1 = sw[i2] - sw[i1];
                const float w2 = sw[i3] - sw[i2], w3 = sw[B] - sw[i3];
                consider(a, false, x0, x1, x2, x3, w0, w1, w2, w3, 0, 1, 2, 3);
                consider(s, true, x0, x1, x2, x3, w0, w1, w2, w3, 0, 1, 2, 3);
                consider(a, false, x0, x1, x2, x3, w0, w1, w2, w3, 3, 2, 1, 0);
                consider(s, true, x0, x1, x2, x3, w0, w1, w2, w3, 3, 2, 1, 0);
            }
        }
    }
    *shifted = sh;
    return d;
}

float block_sigma2(const float *xbl) {
    float sumx2 = 0;
    for (int j = 0; j < kQK; ++j) sumx2 += xbl[j] * xbl[j];
    return 1.5f * sumx2 / kQK;
}

// ------------------------------------------------------------- IQ2_K -----

void quantize_row_iq2_k(const float *x, uint8_t *row, int n, const float *qw_row) {
    constexpr int B = 16;
    float scales[kQK / B], sw[kQK / B], weight[B];
    int8_t Ls[kQK / B];
    for (int ibl = 0; ibl < n / kQK; ++ibl) {
        uint8_t *blk = row + ibl * kIq2kBlock;
        std::memset(blk, 0, kIq2kBlock);  // d = +0, extra = 0
        const float *xbl = x + ibl * kQK;
        const float sigma2 = block_sigma2(xbl);
        uint16_t extra = 0;
        float max_abs_scale = 0;
        for (int ib = 0; ib < kQK / B; ++ib) {
            const float *xb = xbl + B * ib;
            const float *qw = qw_row ? qw_row + ibl * kQK + ib * B : nullptr;
            search_weights(qw, xb, B, sigma2, weight);
            sw[ib] = 0;
            float amax = 0;
            for (int j = 0; j < B; ++j) {
                sw[ib] += weight[j];
                amax = std::max(amax, std::abs(xb[j]));
            }
            if (amax < 1e-16f) { scales[ib] = 0; continue; }
            bool shifted;
            scales[ib] = alphabet_search<B>(xb, weight, B, 0, &shifted);
            if (shifted) extra |= uint16_t(1u << ib);
            max_abs_scale = std::max(max_abs_scale, std::fabs(scales[ib]));
        }
        if (!max_abs_scale) continue;
        const float d = best_int_scale(kQK / B, 8, scales, Ls, sw);
        if (!d) continue;
        store_u16(blk + 2, extra);
        uint8_t *scale_bytes = blk + 4;
        uint8_t *qs = blk + 12;
        const float id = 1 / d;
        float sumqx = 0, sumq2 = 0;
        for (int ib = 0; ib < kQK / B; ++ib) {
            int ls = std::max(-8, std::min(7, nearest_int(id * scales[ib])));
            scale_bytes[ib / 2] |= uint8_t((ls + 8) << 4 * (ib % 2));
            const float dl = d * ls;
            if (!dl) continue;
            const int8_t *vals = (extra >> ib) & 1 ? kValues + 4 : kValues;
            const float *xb = xbl + B * ib;
            const float *qw = qw_row ? qw_row + ibl * kQK + ib * B : nullptr;
            search_weights(qw, xb, B, sigma2, weight);
            const float idl = 1 / dl;
            const int ib32 = ib / 2;
            uint8_t *q = qs + 32 * (ib32 / 4) + 16 * (ib % 2);
            for (int j = 0; j < B; ++j) {
                const int best = nearest_level(vals, idl * xb[j]);
                q[j] |= uint8_t(best << 2 * (ib32 % 4));
                const float w = weight[j];
                const float v = float(vals[best] * ls);
                sumqx += w * v * xb[j];
                sumq2 += w * v * v;
            }
        }
        store_u16(blk, float_to_half(1.030f * (sumq2 > 0 ? sumqx / sumq2 : d)));
    }
}

// ------------------------------------------------------------ IQ2_KS -----

struct Iq2ksScratch {
    std::vector<float> scales, sw;
    std::vector<int8_t> Ls;
};

void quantize_row_iq2_ks(const float *x, uint8_t *row, int n, const float *qw_row, Iq2ksScratch &scr) {
    constexpr int B = 32;
    const int nblock = n / kQK;
    scr.scales.resize(nblock * 8);
    scr.sw.resize(nblock * 8);
    scr.Ls.resize(nblock * 8);
    float weight[B];
    store_u16(row, float_to_half(0.f));
    uint8_t *blocks = row + 2;
    for (int ibl = 0; ibl < nblock; ++ibl) {
        uint8_t *blk = blocks + ibl * kIq2ksBlock;
        std::memset(blk, 0, kIq2ksBlock);
        float *scales = scr.scales.data() + ibl * 8;
        float *sw = scr.sw.data() + ibl * 8;
        const float *xbl = x + ibl * kQK;
        const float sigma2 = block_sigma2(xbl);
        uint16_t extra = 0;
        for (int ib = 0; ib < kQK / B; ++ib) {
            const float *xb = xbl + B * ib;
            const float *qw = qw_row ? qw_row + ibl * kQK + ib * B : nullptr;
            search_weights(qw, xb, B, sigma2, weight);
            sw[ib] = 0;
            float amax = 0;
            for (int j = 0; j < B; ++j) {
                sw[ib] += weight[j];
                amax = std::max(amax, std::abs(xb[j]));
            }
            if (amax < 1e-16f) { scales[ib] = 0; continue; }
            bool shifted;
            scales[ib] = alphabet_search<B>(xb, weight, 3 * B / 4, B / 4, &shifted);
            if (shifted) extra |= uint16_t(1u << ib);
        }
        store_u16(blk, extra);
    }
    const float d = best_int_scale(nblock * 8, 16, scr.scales.data(), scr.Ls.data(), scr.sw.data());
    if (!d) return;
    float sumqx = 0, sumq2 = 0;
    for (int ibl = 0; ibl < nblock; ++ibl) {
        uint8_t *blk = blocks + ibl * kIq2ksBlock;
        uint16_t extra = load_u16(blk);
        uint8_t *scale_bytes = blk + 2;
        uint8_t *qs = blk + 6;
        const float *xbl = x + ibl * kQK;
        const float sigma2 = block_sigma2(xbl);
        const int8_t *Ls = scr.Ls.data() + ibl * 8;
        for (int ib = 0; ib < kQK / B; ++ib) {
            int ls = Ls[ib];
            scale_bytes[ib / 2] |= uint8_t((ls & 0xf) << 4 * (ib % 2));
            extra |= uint16_t((ls >> 4) << (8 + ib));
            ls -= 16;
            const float dl = d * ls;
            if (!dl) continue;
            const int8_t *vals = (extra >> ib) & 1 ? kValues + 4 : kValues;
            const float *xb = xbl + B * ib;
            const float *qw = qw_row ? qw_row + ibl * kQK + ib * B : nullptr;
            search_weights(qw, xb, B, sigma2, weight);
            const float idl = 1 / dl;
            uint8_t *q = qs + 32 * (ib / 4);
            for (int j = 0; j < B; ++j) {
                const int best = nearest_level(vals, idl * xb[j]);
                q[j] |= uint8_t(best << 2 * (ib % 4));
                const float w = weight[j];
                const float v = float(vals[best] * ls);
                sumqx += w * v * xb[j];
                sumq2 += w * v * v;
            }
        }
        store_u16(blk, extra);
    }
    store_u16(row, float_to_half(1.030f * (sumq2 > 0 ? sumqx / sumq2 : d)));
}

// ------------------------------------------------------ IQ2 dequantizers ----

void dequantize_row_iq2_k(const uint8_t *row, float *y, int n) {
    for (int ibl = 0; ibl < n / kQK; ++ibl) {
        const uint8_t *blk = row + ibl * kIq2kBlock;
        const float d = half_to_float(load_u16(blk));
        const uint16_t extra = load_u16(blk + 2);
        const uint8_t *scales = blk + 4, *qs = blk + 12;
        for (int w = 0; w < kQK; ++w) {
            const int sb = w / 16, ib32 = w / 32;
            const float dl = d * (((scales[sb / 2] >> 4 * (sb % 2)) & 0xf) - 8);
            const int8_t *vals = (extra >> sb) & 1 ? kValues + 4 : kValues;
            const int code = (qs[32 * (ib32 / 4) + 16 * ((w / 16) % 2) + w % 16] >> 2 * (ib32 % 4)) & 3;
            y[ibl * kQK + w] = dl * vals[code];
        }
    }
}

void dequantize_row_iq2_ks(const uint8_t *row, float *y, int n) {
    const float d = half_to_float(load_u16(row));
    for (int ibl = 0; ibl < n / kQK; ++ibl) {
        const uint8_t *blk = row + 2 + ibl * kIq2ksBlock;
        const uint16_t extra = load_u16(blk);
        const uint8_t *scales = blk + 2, *qs = blk + 6;
        for (int w = 0; w < kQK; ++w) {
            const int sb = w / 32;
            const int idx = (((scales[sb / 2] >> 4 * (sb % 2)) & 0xf) | (((extra >> (8 + sb)) & 1) << 4)) - 16;
            const float dl = d * idx;
            const int8_t *vals = (extra >> sb) & 1 ? kValues + 4 : kValues;
            const int code = (qs[32 * (w / 128) + w % 32] >> 2 * (sb % 4)) & 3;
            y[ibl * kQK + w] = dl * vals[code];
        }
    }
}

// ------------------------------------------------------ IQ1_S tables ----

// Quantizer-side grid tables: position bytes 2l+1, the code -> index map over
// every 8-position ternary word, and for every word off the grid the grid
// points in its three nearest distance shells (reference:
// vendor/ik_llama/iqk_iq1sr4.cpp:248-342).
struct Iq1Tables {
    std::vector<uint64_t> grid;      // bytes 2l+1
    std::vector<int> map;            // >= 0: grid index; < 0: -(offset+1) into neighbours
    std::vector<uint16_t> neighbours;
};

int worker_count();

template <typename F>
void parallel_for(int64_t count, int64_t grain, F &&fn);

const Iq1Tables &iq1_tables() {
    static Iq1Tables tables;
    static std::once_flag once;
    std::call_once(once, [] {
        const int G = IQK_IQ1S_GRID_SIZE;
        const int kmap = 43692;
        tables.grid.resize(G);
        for (int k = 0; k < G; ++k) {
            uint64_t v = 0;
            for (int i = 0; i < 8; ++i) {
                const uint64_t l = (iqk_iq1s_grid_codes[k] >> 2 * i) & 3;
                v |= (2 * l + 1) << 8 * i;
            }
            tables.grid[k] = v;
        }
        tables.map.assign(kmap, -1);
        for (int k = 0; k < G; ++k) tables.map[iqk_iq1s_grid_codes[k]] = k;
        std::vector<int> off;  // words not on the grid, in increasing order
        for (int i = 0; i < kmap; ++i) if (tables.map[i] < 0) off.push_back(i);
        std::vector<std::vector<uint16_t>> lists(off.size());
        parallel_for(int64_t(off.size()), 64, [&](int64_t lo, int64_t hi) {
            std::vector<std::pair<int, int>> dist(G);
            for (int64_t t = lo; t < hi; ++t) {
                const int word = off[t];
                int pos[8];
                for (int k = 0; k < 8; ++k) pos[k] = 2 * ((word >> 2 * k) & 3) + 1;
                for (int j = 0; j < G; ++j) {
                    int d2 = 0;
                    for (int k = 0; k < 8; ++k) {
                        const int g = int((tables.grid[j] >> 8 * k) & 0xff);
                        d2 += (g - pos[k]) * (g - pos[k]);
                    }
                    dist[j] = {d2, j};
                }
                std::sort(dist.begin(), dist.end());
                // every grid point in the first three distinct distance shells
                int shell = dist[0].first, shells = 1;
                std::vector<uint16_t> &out = lists[t];
                for (int j = 0; j < G; ++j) {
                    if (dist[j].first > shell) {
                        if (shells == 3) break;
                        shell = dist[j].first;
                        ++shells;
                    }
                    out.push_back(uint16_t(dist[j].second));
                }
            }
        });
        for (size_t t = 0; t < off.size(); ++t) {
            tables.map[off[t]] = -int(tables.neighbours.size() + 1);
            tables.neighbours.push_back(uint16_t(lists[t].size()));
            tables.neighbours.insert(tables.neighbours.end(), lists[t].begin(), lists[t].end());
        }
    });
    return tables;
}

inline int grid_pos(uint64_t g, int i) { return int((g >> 8 * i) & 0xff); }

// Nearest grid point (weighted squared error at `scale`) among a word's
// listed neighbours; writes that point's levels to L.
int best_neighbour(const uint16_t *nb, const uint64_t *grid, const float *xval, const float *weight,
                   float scale, const float *levels, int8_t *L) {
    const int count = nb[0];
    float best = FLT_MAX;
    int index = -1;
    for (int j = 1; j <= count; ++j) {
        const uint64_t g = grid[nb[j]];
        float d2 = 0;
        for (int i = 0; i < 8; ++i) {
            const float q = levels[(grid_pos(g, i) - 1) / 2];
            const float w = weight[i];
            const float diff = scale * q - xval[i];
            d2 += w * diff * diff;
        }
        if (d2 < best) { best = d2; index = nb[j]; }
    }
    // With finite inputs every listed distance is finite, so a neighbour is
    // always taken; a non-finite block falls through to a full-grid search.
    if (index < 0) {
        for (int k = 0; k < IQK_IQ1S_GRID_SIZE; ++k) {
            float d2 = 0;
            for (int i = 0; i < 8; ++i) {
                const float q = levels[(grid_pos(grid[k], i) - 1) / 2];
                const float diff = scale * q - xval[i];
                d2 += weight[i] * diff * diff;
            }
            if (d2 < best) { best = d2; index = k; }
        }
    }
    if (index < 0) return -1;
    for (int i = 0; i < 8; ++i) L[i] = int8_t((grid_pos(grid[index], i) - 1) / 2);
    return index;
}

// One 32-weight block: ternary levels by a 2-boundary search over the sorted
// values with shift +delta and -delta, snapped to the grid.
int iq1_block(const float *xb, const float *weight, float *out_scale, uint16_t *index, int *out_shift) {
    constexpr int B = 32;
    float max = std::fabs(xb[0]);
    for (int i = 1; i < B; ++i) max = fmaxf(max, std::fabs(xb[i]));
    if (max < 1e-12f) {
        *out_scale = 0;
        *out_shift = 1;
        for (int k = 0; k < B / 8; ++k) index[k] = 0;
        return 0;
    }
    const Iq1Tables &t = iq1_tables();
    const float xp[3] = {-1 + kIq1Delta, kIq1Delta, 1 + kIq1Delta};
    const float xm[3] = {-1 - kIq1Delta, -kIq1Delta, 1 - kIq1Delta};
    struct Rec { float v; int i; };
    Rec order[B];
    for (int j = 0; j < B; ++j) order[j] = {xb[j], j};
    // ordering by value only, equal values keeping their position (the
    // reference's qsort is glibc's stable merge sort for 32 records)
    std::stable_sort(order, order + B, [](const Rec &a, const Rec &b) { return a.v < b.v; });
    float sx[B + 1], sw[B + 1];
    sx[0] = sw[0] = 0;
    for (int j = 0; j < B; ++j) {
        const int i = order[j].i;
        sx[j + 1] = sx[j] + weight[i] * xb[i];
        sw[j + 1] = sw[j] + weight[i];
    }
    float best = -FLT_MIN, scale = max;
    int b1 = -1, b2 = -1, best_shift = 0;
    for (int i1 = 0; i1 <= B; ++i1) {
        for (int i2 = i1; i2 <= B; ++i2) {
            const float x0 = sx[i1] - sx[0], x1 = sx[i2] - sx[i1], x2 = sx[B] - sx[i2];
            const float w0 = sw[i1] - sw[0], w1 = sw[i2] - sw[i1], w2 = sw[B] - sw[i2];
            float sumqx = x0 * xp[0] + x1 * xp[1] + x2 * xp[2];
            float sumq2 = w0 * xp[0] * xp[0] + w1 * xp[1] * xp[1] + w2 * xp[2] * xp[2];
            if (sumq2 > 0 && sumqx * sumqx > best * sumq2) {
                scale = sumqx / sumq2; best = scale * sumqx;
                b1 = i1; b2 = i2; best_shift = 1;
            }
            sumqx = x0 * xm[0] + x1 * xm[1] + x2 * xm[2];
            sumq2 = w0 * xm[0] * xm[0] + w1 * xm[1] * xm[1] + w2 * xm[2] * xm[2];
            if (sumq2 > 0 && sumqx * sumqx > best * sumq2) {
                scale = sumqx / sumq2; best = scale * sumqx;
                b1 = i1; b2 = i2; best_shift = -1;
            }
        }
    }
    if (b1 < 0 || b2 < 0 || best_shift == 0) return 1;
    int8_t L[B];
    for (int j = 0; j < B; ++j) L[order[j].i] = int8_t(j < b1 ? 0 : j < b2 ? 1 : 2);
    if (scale < 0) {
        for (int j = 0; j < B; ++j) L[j] = int8_t(2 - L[j]);
        scale = -scale;
        best_shift = -best_shift;
    }
    const float *levels = best_shift == 1 ? xp : xm;
    bool on_grid = true;
    for (int k = 0; k < B / 8; ++k) {
        int word = 0;
        for (int j = 0; j < 8; ++j) word |= L[8 * k + j] << 2 * j;
        int gi = t.map[word];
        if (gi < 0) {
            on_grid = false;
            gi = best_neighbour(t.neighbours.data() - t.map[word] - 1, t.grid.data(), xb + 8 * k,
                                weight + 8 * k, scale, levels, L + 8 * k);
            if (gi < 0) return 1;
        }
        index[k] = uint16_t(gi);
    }
    if (!on_grid) {
        float sumqx = 0, sumq2 = 0;
        for (int k = 0; k < B / 8; ++k) {
            const uint64_t g = t.grid[index[k]];
            for (int j = 0; j < 8; ++j) {
                const float w = weight[8 * k + j];
                const float q = levels[(grid_pos(g, j) - 1) / 2];
                sumqx += w * q * xb[8 * k + j];
                sumq2 += w * q * q;
            }
        }
        if (sumqx > 0 && sumq2 > 0) scale = sumqx / sumq2;
    }
    *out_scale = scale;
    *out_shift = best_shift;
    return 0;
}

// One four-row group.  Returns false on an internal failure (the reference's
// zero-return paths).
bool quantize_group_iq1_s_r4(const float *src, uint8_t *dst, int n, const float *imatrix,
                             std::vector<float> &scales) {
    constexpr int B = 32;
    const int nblock = n / B;
    scales.resize(4 * nblock);
    float weight[B], max[4] = {0, 0, 0, 0};
    uint16_t index[4];
    int shift;
    uint8_t *blocks = dst + 8;
    for (int ibl = 0; ibl < nblock; ++ibl) {
        uint8_t *blk = blocks + ibl * kIq1Block;
        for (int k = 0; k < 4; ++k) {
            const float *xb = src + k * n + B * ibl;
            float sumx2 = 0;
            for (int j = 0; j < B; ++j) sumx2 += xb[j] * xb[j];
            if (sumx2 < 1e-14f) {
                const int ind = IQK_IQ1S_ZERO_INDEX;
                scales[4 * ibl + k] = 0;
                uint16_t h = 0;
                for (int i = 0; i < 4; ++i) {
                    blk[4 * i + k] = uint8_t(ind & 255);
                    h |= uint16_t((ind >> 8) << 3 * i);
                }
                store_u16(blk + 16 + 2 * k, h);
                continue;
            }
            const float sigma2 = 1.5f * sumx2 / B;
            bool use_imatrix = false;
            if (imatrix) {
                use_imatrix = true;
                float sumwx = 0;
                for (int j = 0; j < B; ++j) {
                    // the reference's unqualified sqrt is the double overload
                    weight[j] = float(double(imatrix[B * ibl + j]) * std::sqrt(double(sigma2 + xb[j] * xb[j])));
                    sumwx += weight[j] * std::abs(xb[j]);
                }
                if (sumwx < 1e-14f) {
                    std::printf("Found block with mismatching importance/model weights\n");
                    use_imatrix = false;
                }
            }
            if (!use_imatrix) {
                for (int j = 0; j < B; ++j) weight[j] = float(std::sqrt(double(sigma2 + xb[j] * xb[j])));
            }
            if (iq1_block(xb, weight, &scales[4 * ibl + k], index, &shift)) return false;
            if (scales[4 * ibl + k] < 0) return false;
            max[k] = std::max(max[k], scales[4 * ibl + k]);
            uint16_t h = 0;
            for (int i = 0; i < 4; ++i) {
                if (index[i] >= IQK_IQ1S_GRID_SIZE) return false;
                blk[4 * i + k] = uint8_t(index[i] & 255);
                h |= uint16_t((index[i] >> 8) << 3 * i);
            }
            if (shift < 0) h |= 0x8000u;
            store_u16(blk + 16 + 2 * k, h);
        }
    }
    float invd[4];
    for (int k = 0; k < 4; ++k) {
        store_u16(dst + 2 * k, float_to_half(1.0625f * max[k] / 15));
        invd[k] = max[k] ? 15 / max[k] : 0.f;
    }
    for (int ibl = 0; ibl < nblock; ++ibl) {
        uint8_t *blk = blocks + ibl * kIq1Block;
        for (int k = 0; k < 4; ++k) {
            int ls = nearest_int(0.5f * (scales[4 * ibl + k] * invd[k] - 1));
            ls = std::max(0, std::min(7, ls));
            store_u16(blk + 16 + 2 * k, uint16_t(load_u16(blk + 16 + 2 * k) | (ls << 12)));
        }
    }
    return true;
}

void dequantize_group_iq1_s_r4(const uint8_t *grp, float *y, int n) {
    float d[4];
    for (int k = 0; k < 4; ++k) d[k] = half_to_float(load_u16(grp + 2 * k));
    const uint8_t *blocks = grp + 8;
    for (int ib = 0; ib < n / 32; ++ib) {
        const uint8_t *blk = blocks + ib * kIq1Block;
        for (int k = 0; k < 4; ++k) {
            const uint16_t qh = load_u16(blk + 16 + 2 * k);
            const float shift = qh & 0x8000u ? -kIq1Delta : kIq1Delta;
            const float dl = d[k] * (2 * ((qh >> 12) & 7) + 1);
            for (int i = 0; i < 4; ++i) {
                const int idx = blk[4 * i + k] | (((qh >> 3 * i) & 7) << 8);
                const uint16_t code = iqk_iq1s_grid_codes[idx];
                for (int j = 0; j < 8; ++j) {
                    const int g = int((code >> 2 * j) & 3) - 1;
                    y[size_t(k) * n + 32 * ib + 8 * i + j] = dl * (g + shift);
                }
            }
        }
    }
}

// ------------------------------------------------------------ threading ----

std::atomic<int> g_threads{0};

int worker_count() {
    int t = g_threads.load();
    if (t > 0) return t;
    if (const char *env = std::getenv("IQK_CODEC_THREADS")) {
        const int v = std::atoi(env);
        if (v > 0) return v;
    }
    const unsigned hw = std::thread::hardware_concurrency();
    return hw ? int(hw) : 1;
}

// Split [0, count) into chunks of at least `grain` and run fn(lo, hi) on a
// pool of worker threads; the result must not depend on the split.
template <typename F>
void parallel_for(int64_t count, int64_t grain, F &&fn) {
    if (count <= 0) return;
    const int64_t chunks = (count + grain - 1) / grain;
    const int workers = int(std::min<int64_t>(worker_count(), chunks));
    if (workers <= 1) { fn(0, count); return; }
    std::atomic<int64_t> next{0};
    auto body = [&] {
        for (;;) {
            const int64_t c = next.fetch_add(1);
            if (c >= chunks) break;
            fn(c * grain, std::min(count, (c + 1) * grain));
        }
    };
    std::vector<std::thread> pool;
    for (int w = 1; w < workers; ++w) pool.emplace_back(body);
    body();
    for (auto &th : pool) th.join();
}

bool width_ok_256(int64_t n) { return n > 0 && n % kQK == 0 && n <= (int64_t(1) << 30); }
bool width_ok_32(int64_t n) { return n > 0 && n % 32 == 0 && n <= (int64_t(1) << 30); }

}  // namespace

extern "C" {

size_t iqk_row_size_iq2_k(int64_t n) { return width_ok_256(n) ? size_t(kIq2kBlock) * size_t(n / kQK) : 0; }
size_t iqk_row_size_iq2_ks(int64_t n) { return width_ok_256(n) ? 2 + size_t(kIq2ksBlock) * size_t(n / kQK) : 0; }
size_t iqk_row_size_iq1_s_r4(int64_t n) { return width_ok_32(n) ? 2 + 6 * size_t(n / 32) : 0; }

size_t iqk_block_size_iq2_k(void) { return kIq2kBlock; }
size_t iqk_block_size_iq2_ks(void) { return kIq2ksBlock; }
size_t iqk_block_size_iq1_s_r4(void) { return kIq1Block; }

void iqk_codec_set_threads(int threads) { g_threads.store(threads > 0 ? threads : 0); }
int iqk_codec_threads(void) { return worker_count(); }

size_t iqk_quantize_iq2_k(const float *src, void *dst, int64_t nrows, int64_t n, const float *imatrix) {
    const size_t rs = iqk_row_size_iq2_k(n);
    if (!rs || nrows <= 0) return 0;
    parallel_for(nrows, 8, [&](int64_t lo, int64_t hi) {
        std::vector<float> w(imatrix ? n : 0);
        for (int64_t r = lo; r < hi; ++r) {
            const float *x = src + r * n;
            if (imatrix) row_weights(imatrix, x, int(n), 16, w.data());
            quantize_row_iq2_k(x, static_cast<uint8_t *>(dst) + r * rs, int(n), imatrix ? w.data() : nullptr);
        }
    });
    return size_t(nrows) * rs;
}

size_t iqk_quantize_iq2_ks(const float *src, void *dst, int64_t nrows, int64_t n, const float *imatrix) {
    const size_t rs = iqk_row_size_iq2_ks(n);
    if (!rs || nrows <= 0) return 0;
    parallel_for(nrows, 8, [&](int64_t lo, int64_t hi) {
        std::vector<float> w(imatrix ? n : 0);
        Iq2ksScratch scr;
        for (int64_t r = lo; r < hi; ++r) {
            const float *x = src + r * n;
            if (imatrix) row_weights(imatrix, x, int(n), 32, w.data());
            quantize_row_iq2_ks(x, static_cast<uint8_t *>(dst) + r * rs, int(n), imatrix ? w.data() : nullptr, scr);
        }
    });
    return size_t(nrows) * rs;
}

size_t iqk_quantize_iq1_s_r4(const float *src, void *dst, int64_t nrows, int64_t n, const float *imatrix) {
    const size_t rs = iqk_row_size_iq1_s_r4(n);
    if (!rs || nrows <= 0 || nrows % 4) return 0;
    iq1_tables();  // build once, outside the workers
    std::atomic<bool> ok{true};
    parallel_for(nrows / 4, 2, [&](int64_t lo, int64_t hi) {
        std::vector<float> scales;
        for (int64_t g = lo; g < hi; ++g) {
            if (!quantize_group_iq1_s_r4(src + 4 * g * n, static_cast<uint8_t *>(dst) + 4 * g * rs, int(n),
                                         imatrix, scales))
                ok.store(false);
        }
    });
    return ok.load() ? size_t(nrows) * rs : 0;
}

int iqk_dequantize_iq2_k(const void *src, float *dst, int64_t nrows, int64_t n) {
    const size_t rs = iqk_row_size_iq2_k(n);
    if (!rs || nrows < 0) return 1;
    for (int64_t r = 0; r < nrows; ++r)
        dequantize_row_iq2_k(static_cast<const uint8_t *>(src) + r * rs, dst + r * n, int(n));
    return 0;
}

int iqk_dequantize_iq2_ks(const void *src, float *dst, int64_t nrows, int64_t n) {
    const size_t rs = iqk_row_size_iq2_ks(n);
    if (!rs || nrows < 0) return 1;
    for (int64_t r = 0; r < nrows; ++r)
        dequantize_row_iq2_ks(static_cast<const uint8_t *>(src) + r * rs, dst + r * n, int(n));
    return 0;
}

int iqk_dequantize_iq1_s_r4(const void *src, float *dst, int64_t nrows, int64_t n) {
    const size_t rs = iqk_row_size_iq1_s_r4(n);
    if (!rs || nrows <= 0 || nrows % 4) return 1;
    for (int64_t r = 0; r < nrows; r += 4)
        dequantize_group_iq1_s_r4(static_cast<const uint8_t *>(src) + r * rs, dst + r * n, int(n));
    return 0;
}

}  // extern "C"
