// synth.cpp — seeded synthetic checkpoints, binary16 conversions and the
// reference's Q4 quantizer (host code of the library).
#include "../../include/qtts_synth.h"

#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

namespace {

inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

// Box-Muller on the two 32-bit halves of one hash, in double.
inline double normal_from(uint64_t h) {
    const double u1 = ((double)(h >> 32) + 0.5) * 0x1p-32;
    const double u2 = ((double)(h & 0xFFFFFFFFULL) + 0.5) * 0x1p-32;
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}

// Runs body(lo, hi) over [0, count) on up to 16 threads; results depend only
// on the index, never on the split.
template <class F>
void parallel_for(int64_t count, F body) {
    int nt = (int)std::thread::hardware_concurrency();
    if (nt > 16) nt = 16;
    if (nt < 1) nt = 1;
    if (count < (int64_t)1 << 16) nt = 1;
    if (nt == 1) {
        body((int64_t)0, count);
        return;
    }
    std::vector<std::thread> th;
    const int64_t chunk = (count + nt - 1) / nt;
    for (int t = 0; t < nt; t++) {
        const int64_t lo = t * chunk, hi = std::min(count, lo + chunk);
        if (lo >= hi) break;
        th.emplace_back([=] { body(lo, hi); });
    }
    for (auto &x : th) x.join();
}

}  // namespace

extern "C" {

uint64_t qtts_synth_u64(uint64_t seed, uint64_t stream, uint64_t index) {
    return mix64(mix64(seed ^ (stream * 0x9E3779B97F4A7C15ULL)) + index * 0xD1B54A32D192ED03ULL);
}

uint16_t qtts_f32_to_f16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t a = x & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) {  // inf / nan (quiet the nan, keep payload bits)
        if (a == 0x7F800000u) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | 0x7E00u | ((a >> 13) & 0x3FFu));
    }
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);  // >= 65520 rounds to inf
    if (a >= 0x38800000u) {                                    // normal binary16 range
        uint32_t h = ((((a >> 23) - 112u) << 10) | ((a & 0x7FFFFFu) >> 13));
        const uint32_t rem = a & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    if (a < 0x33000000u) return (uint16_t)sign;  // < 2^-25 (ties to even 0)
    // subnormal result: round(mant * 2^(e-126)) with e the biased exponent
    const uint32_t e = a >> 23;
    const uint32_t mant = (a & 0x7FFFFFu) | 0x800000u;
    const uint32_t shift = 126u - e;  // 14..24
    uint32_t h = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float qtts_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t ex = (h >> 10) & 0x1Fu;
    const uint32_t man = h & 0x3FFu;
    uint32_t bits;
    float f;
    if (ex == 0) {
        f = (float)man * 0x1p-24f;
        std::memcpy(&bits, &f, 4);
        bits |= sign;
    } else if (ex == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((ex + 112u) << 23) | (man << 13);
    }
    std::memcpy(&f, &bits, 4);
    return f;
}

void qtts_synth_q4(uint64_t seed, uint64_t stream, int32_t k, int32_t n, float scale_std, uint8_t *packed,
                   uint16_t *scales) {
    const int64_t nbytes = (int64_t)k * (n / 2);
    const int64_t nwords = (nbytes + 7) / 8;
    parallel_for(nwords, [&](int64_t lo, int64_t hi) {
        for (int64_t w = lo; w < hi; w++) {
            const uint64_t h = qtts_synth_u64(seed, stream, (uint64_t)w);
            const int64_t b0 = w * 8;
            for (int b = 0; b < 8 && b0 + b < nbytes; b++) packed[b0 + b] = (uint8_t)(h >> (8 * b));
        }
    });
    const int64_t nscales = (int64_t)k * (n / 32);
    const uint64_t sstream = stream ^ 0x5CA1E5CA1E5CA1E5ULL;
    parallel_for(nscales, [&](int64_t lo, int64_t hi) {
        for (int64_t i = lo; i < hi; i++) {
            const float v = (float)std::fabs(normal_from(qtts_synth_u64(seed, sstream, (uint64_t)i)) * scale_std);
            scales[i] = qtts_f32_to_f16(v);
        }
    });
}

void qtts_synth_normal_f32(uint64_t seed, uint64_t stream, int64_t count, float mean, float std, float *out) {
    parallel_for(count, [&](int64_t lo, int64_t hi) {
        for (int64_t i = lo; i < hi; i++)
            out[i] = (float)(mean + std * normal_from(qtts_synth_u64(seed, stream, (uint64_t)i)));
    });
}

void qtts_synth_normal_f16(uint64_t seed, uint64_t stream, int64_t count, float mean, float std, uint16_t *out) {
    parallel_for(count, [&](int64_t lo, int64_t hi) {
        for (int64_t i = lo; i < hi; i++)
            out[i] = qtts_f32_to_f16((float)(mean + std * normal_from(qtts_synth_u64(seed, stream, (uint64_t)i))));
    });
}

// quantize_f32_to_q4, src/gemv.rs:92-130.
void qtts_quantize_f32_to_q4(const float *data, int32_t k, int32_t n, uint8_t *packed, uint16_t *scales) {
    const int32_t groups_per_row = n / 32;
    for (int32_t ki = 0; ki < k; ki++) {
        for (int32_t g = 0; g < groups_per_row; g++) {
            const int64_t gi = (int64_t)ki * groups_per_row + g;
            const float *v = data + (int64_t)ki * n + (int64_t)g * 32;
            float absmax = 0.0f;
            for (int j = 0; j < 32; j++) {
                const float a = std::fabs(v[j]);
                if (a > absmax) absmax = a;
            }
            const float scale = absmax / 7.0f;
            scales[gi] = qtts_f32_to_f16(scale);
            const float inv_scale = scale > 0.0f ? 1.0f / scale : 0.0f;
            for (int j = 0; j < 32; j += 2) {
                uint8_t q[2];
                for (int e = 0; e < 2; e++) {
                    const float r = std::round(v[j + e] * inv_scale);  // half away from zero
                    float c = r;
                    if (c != c) {
                        q[e] = 0;  // NaN as u8 == 0
                        continue;
                    }
                    c = c < -8.0f ? -8.0f : (c > 7.0f ? 7.0f : c);
                    q[e] = (uint8_t)(c + 8.0f);
                }
                packed[gi * 16 + j / 2] = (uint8_t)(q[0] | (q[1] << 4));
            }
        }
    }
}

}  // extern "C"
