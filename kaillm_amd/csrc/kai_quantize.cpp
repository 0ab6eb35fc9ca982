// Host-side GGUF weight quantizers: float rows -> wire blocks of the six formats.
//
// Tooling, not the hot path: it plays the role of gguf-py's quants.quantize
// (runtime-source/gguf-reader/gguf/quants.py) for building synthetic weights.
// Q8_0 and Q4_0 follow gguf-py's closed forms (quants.py:382-394, :223-239) in
// float32. gguf-py has no K-quant or IQ3_S quantizer, so Q4_K/Q6_K/Q2_K use
// min/max or symmetric-max fits of our own and IQ3_S a nearest-grid search; any
// valid block is a valid input to the kernels, so the choice only affects how
// close the blocks are to the source floats.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/kai_quantize.h"
#include "kai_formats.h"
#include "kai_iq3s_grid.h"

namespace {

using namespace kai;

uint16_t f2h(float f) {
    // IEEE binary16, round to nearest even.
    uint32_t u;
    std::memcpy(&u, &f, 4);
    const uint16_t sign = static_cast<uint16_t>((u >> 16) & 0x8000u);
    const uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) return static_cast<uint16_t>(sign | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0u));
    const int e = static_cast<int>(a >> 23) - 127;
    if (e > 15) return static_cast<uint16_t>(sign | 0x7c00u);
    if (e >= -14) {
        const uint32_t mant = a & 0x7fffffu;
        uint32_t h = (static_cast<uint32_t>(e + 15) << 10) | (mant >> 13);
        const uint32_t rest = mant & 0x1fffu;
        if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h;
        return static_cast<uint16_t>(sign | h);
    }
    if (e < -25) return sign;
    const uint32_t mant = (a & 0x7fffffu) | 0x800000u;
    const int shift = -e - 1;
    uint32_t h = mant >> shift;
    const uint32_t rest = mant & ((1u << shift) - 1u);
    const uint32_t halfway = 1u << (shift - 1);
    if (rest > halfway || (rest == halfway && (h & 1u))) ++h;
    return static_cast<uint16_t>(sign | h);
}

float h2f(uint16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
    const int exp = (h >> 10) & 0x1f;
    const uint32_t mant = h & 0x3ffu;
    float f;
    if (exp == 0) {
        f = static_cast<float>(mant) * 5.9604644775390625e-08f;
        return sign ? -f : f;
    }
    const uint32_t u = exp == 31 ? (sign | 0x7f800000u | (mant << 13))
                                 : (sign | (static_cast<uint32_t>(exp - 15 + 127) << 23) | (mant << 13));
    std::memcpy(&f, &u, 4);
    return f;
}

void put16(uint8_t *p, uint16_t v) { std::memcpy(p, &v, 2); }
float roundf_away(float v) { return std::round(v); }  // half-way cases away from zero
int clampi(int v, int lo, int hi) { return std::min(std::max(v, lo), hi); }

void quant_q8_0(const float *x, uint8_t *b) {
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) amax = std::max(amax, std::fabs(x[i]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    put16(b, f2h(d));
    for (int i = 0; i < 32; ++i) b[2 + i] = static_cast<uint8_t>(static_cast<int8_t>(roundf_away(x[i] * id)));
}

void quant_q4_0(const float *x, uint8_t *b) {
    int imax = 0;
    for (int i = 1; i < 32; ++i)
        if (std::fabs(x[i]) > std::fabs(x[imax])) imax = i;
    const float d = x[imax] / -8.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    put16(b, f2h(d));
    uint8_t q[32];
    for (int i = 0; i < 32; ++i) {
        const float t = std::trunc(x[i] * id + 8.5f);
        q[i] = static_cast<uint8_t>(clampi(static_cast<int>(t), 0, 15));
    }
    for (int i = 0; i < 16; ++i) b[2 + i] = static_cast<uint8_t>(q[i] | (q[i + 16] << 4));
}

void quant_q4_k(const float *x, uint8_t *b) {
    float scale[8], minv[8];
    for (int i = 0; i < 8; ++i) {
        float lo = 0.0f, hi = 0.0f;
        for (int l = 0; l < 32; ++l) {
            lo = std::min(lo, x[32 * i + l]);
            hi = std::max(hi, x[32 * i + l]);
        }
        scale[i] = (hi - lo) / 15.0f;
        minv[i] = -lo;
    }
    const float smax = *std::max_element(scale, scale + 8), mmax = *std::max_element(minv, minv + 8);
    const uint16_t hd = f2h(smax / 63.0f), hm = f2h(mmax / 63.0f);
    const float d = h2f(hd), dmin = h2f(hm);
    int sc[8], mn[8];
    for (int i = 0; i < 8; ++i) {
        sc[i] = d > 0.0f ? clampi(static_cast<int>(roundf_away(scale[i] / d)), 0, 63) : 0;
        mn[i] = dmin > 0.0f ? clampi(static_cast<int>(roundf_away(minv[i] / dmin)), 0, 63) : 0;
    }
    put16(b, hd);
    put16(b + 2, hm);
    uint8_t *s = b + 4;
    for (int i = 0; i < 4; ++i) {
        s[i] = static_cast<uint8_t>((sc[i] & 63) | ((sc[i + 4] >> 4) << 6));
        s[4 + i] = static_cast<uint8_t>((mn[i] & 63) | ((mn[i + 4] >> 4) << 6));
        s[8 + i] = static_cast<uint8_t>((sc[i + 4] & 15) | ((mn[i + 4] & 15) << 4));
    }
    uint8_t q[256];
    for (int i = 0; i < 8; ++i) {
        const float ds = d * static_cast<float>(sc[i]), dm = dmin * static_cast<float>(mn[i]);
        for (int l = 0; l < 32; ++l) {
            const float v = ds > 0.0f ? (x[32 * i + l] + dm) / ds : 0.0f;
            q[32 * i + l] = static_cast<uint8_t>(clampi(static_cast<int>(roundf_away(v)), 0, 15));
        }
    }
    for (int j = 0; j < 4; ++j)
        for (int l = 0; l < 32; ++l) b[16 + 32 * j + l] = static_cast<uint8_t>(q[64 * j + l] | (q[64 * j + 32 + l] << 4));
}

void quant_q6_k(const float *x, uint8_t *b) {
    float sg[16];
    for (int g = 0; g < 16; ++g) {
        int imax = 0;
        for (int l = 1; l < 16; ++l)
            if (std::fabs(x[16 * g + l]) > std::fabs(x[16 * g + imax])) imax = l;
        sg[g] = x[16 * g + imax] / -32.0f;
    }
    float amax = 0.0f;
    for (int g = 0; g < 16; ++g) amax = std::max(amax, std::fabs(sg[g]));
    const uint16_t hd = f2h(amax / 127.0f);
    const float d = h2f(hd);
    int8_t sc[16];
    for (int g = 0; g < 16; ++g) sc[g] = static_cast<int8_t>(d > 0.0f ? clampi(static_cast<int>(roundf_away(sg[g] / d)), -127, 127) : 0);
    std::memset(b, 0, 210);
    for (int e = 0; e < 256; ++e) {
        const float ds = d * static_cast<float>(sc[e / 16]);
        const int code = ds != 0.0f ? clampi(static_cast<int>(roundf_away(x[e] / ds)), -32, 31) + 32 : 32;
        const int h = e / 128, s = (e % 128) / 32, l = e % 32;
        b[64 * h + 32 * (s % 2) + l] |= static_cast<uint8_t>((code & 15) << (4 * (s / 2)));
        b[128 + 32 * h + l] |= static_cast<uint8_t>((code >> 4) << (2 * s));
    }
    std::memcpy(b + 192, sc, 16);
    put16(b + 208, hd);
}

void quant_q2_k(const float *x, uint8_t *b) {
    float scale[16], minv[16];
    for (int g = 0; g < 16; ++g) {
        float lo = 0.0f, hi = 0.0f;
        for (int l = 0; l < 16; ++l) {
            lo = std::min(lo, x[16 * g + l]);
            hi = std::max(hi, x[16 * g + l]);
        }
        scale[g] = (hi - lo) / 3.0f;
        minv[g] = -lo;
    }
    const uint16_t hd = f2h(*std::max_element(scale, scale + 16) / 15.0f);
    const uint16_t hm = f2h(*std::max_element(minv, minv + 16) / 15.0f);
    const float d = h2f(hd), dmin = h2f(hm);
    std::memset(b, 0, 84);
    int sc[16], mn[16];
    for (int g = 0; g < 16; ++g) {
        sc[g] = d > 0.0f ? clampi(static_cast<int>(roundf_away(scale[g] / d)), 0, 15) : 0;
        mn[g] = dmin > 0.0f ? clampi(static_cast<int>(roundf_away(minv[g] / dmin)), 0, 15) : 0;
        b[g] = static_cast<uint8_t>(sc[g] | (mn[g] << 4));
    }
    for (int e = 0; e < 256; ++e) {
        const int g = e / 16;
        const float ds = d * static_cast<float>(sc[g]), dm = dmin * static_cast<float>(mn[g]);
        const int q = ds > 0.0f ? clampi(static_cast<int>(roundf_away((x[e] + dm) / ds)), 0, 3) : 0;
        const int h = e / 128, s = (e % 128) / 32, l = e % 32;
        b[16 + 32 * h + l] |= static_cast<uint8_t>(q << (2 * s));
    }
    put16(b + 80, hd);
    put16(b + 82, hm);
}

// IQ3_S nearest-grid lookup: for every tuple of 4 level indices (8^4 = 4096) the
// grid entry with the smallest squared level distance.
struct Iq3sLut {
    uint16_t nearest[4096];
    Iq3sLut() {
        static const uint32_t grid[512] = {KAI_IQ3S_GRID_VALUES};
        for (int t = 0; t < 4096; ++t) {
            int best = 0, best_err = 1 << 30;
            for (int e = 0; e < 512; ++e) {
                int err = 0;
                for (int j = 0; j < 4; ++j) {
                    const int want = 2 * ((t >> (3 * j)) & 7) + 1;
                    const int have = static_cast<int>((grid[e] >> (8 * j)) & 0xffu);
                    err += (want - have) * (want - have);
                }
                if (err < best_err) {
                    best_err = err;
                    best = e;
                }
            }
            nearest[t] = static_cast<uint16_t>(best);
        }
    }
};

const Iq3sLut &iq3s_lut() {
    static const Iq3sLut lut;  // built once, thread-safe initialisation
    return lut;
}

void quant_iq3_s(const float *x, uint8_t *b, const Iq3sLut &lut) {
    float db[8];
    for (int g = 0; g < 8; ++g) {
        float amax = 0.0f;
        for (int t = 0; t < 32; ++t) amax = std::max(amax, std::fabs(x[32 * g + t]));
        db[g] = amax / 15.0f;
    }
    const uint16_t hd = f2h(*std::max_element(db, db + 8) / 31.0f);
    const float d = h2f(hd);
    std::memset(b, 0, 110);
    put16(b, hd);
    for (int g = 0; g < 8; ++g) {
        const int sc = d > 0.0f ? clampi(static_cast<int>(roundf_away((db[g] / d - 1.0f) / 2.0f)), 0, 15) : 0;
        b[106 + g / 2] |= static_cast<uint8_t>(sc << (4 * (g % 2)));
        const float step = d * static_cast<float>(1 + 2 * sc);
        for (int i = 0; i < 8; ++i) {
            int key = 0;
            for (int j = 0; j < 4; ++j) {
                const float v = x[32 * g + 4 * i + j];
                const float level = step > 0.0f ? std::fabs(v) / step : 0.0f;  // nearest odd level 1..15
                const int li = clampi(static_cast<int>(std::floor(level / 2.0f)), 0, 7);
                key |= li << (3 * j);
                if (v < 0.0f) b[74 + 4 * g + (4 * i + j) / 8] |= static_cast<uint8_t>(1u << ((4 * i + j) % 8));
            }
            const int idx = lut.nearest[key];
            b[2 + 8 * g + i] = static_cast<uint8_t>(idx & 0xff);
            b[66 + g] |= static_cast<uint8_t>((idx >> 8) << i);
        }
    }
}

}  // namespace

extern "C" int kai_quantize_rows(int type, const float *src, int64_t n, int64_t k, void *dst, int threads) {
    const int qk = block_elems(type), bb = block_bytes(type);
    if (!src || !dst || n < 0 || k <= 0 || !weight_type_supported(type) || k % qk) return -1;
    const Iq3sLut *lut = type == IQ3_S ? &iq3s_lut() : nullptr;
    const int64_t blocks = k / qk;
    auto work = [&](int64_t r0, int64_t r1) {
        for (int64_t r = r0; r < r1; ++r) {
            for (int64_t blk = 0; blk < blocks; ++blk) {
                const float *x = src + r * k + blk * qk;
                uint8_t *b = static_cast<uint8_t *>(dst) + (r * blocks + blk) * bb;
                switch (type) {
                    case Q8_0: quant_q8_0(x, b); break;
                    case Q4_0: quant_q4_0(x, b); break;
                    case Q4_K: quant_q4_k(x, b); break;
                    case Q6_K: quant_q6_k(x, b); break;
                    case Q2_K: quant_q2_k(x, b); break;
                    case IQ3_S: quant_iq3_s(x, b, *lut); break;
                }
            }
        }
    };
    const int t = std::max(1, std::min<int>(threads > 0 ? threads : 1, static_cast<int>(std::max<int64_t>(n, 1))));
    if (t == 1) {
        work(0, n);
        return 0;
    }
    std::vector<std::thread> pool;
    const int64_t per = (n + t - 1) / t;
    for (int i = 0; i < t; ++i) {
        const int64_t r0 = i * per, r1 = std::min(n, r0 + per);
        if (r0 < r1) pool.emplace_back(work, r0, r1);
    }
    for (auto &th : pool) th.join();
    return 0;
}
