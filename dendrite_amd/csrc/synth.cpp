// Seeded synthetic inputs for tests and benchmarks (no counterpart in the
// reference; built into libdendrite_testdata.so, not the backend library).  Normals: SplitMix64 counter hash + Box-Muller in double
// precision, so a value depends only on (seed, index) and any subset of a
// pool can be generated independently and in parallel.  FP8 encodings follow
// the OCP FP8 (E4M3 "FN") and OCP MX v1.0 (E8M0 scale) specifications.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <thread>
#include <vector>

#include <stdarg.h>
#include <stdio.h>

#include "dendrite_testdata.h"

namespace {

thread_local char g_error[256];

dh_status fail(dh_status s, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
dh_status fail(dh_status s, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof g_error, fmt, ap);
    va_end(ap);
    return s;
}

uint32_t kv_elem_bytes(uint32_t fmt) {
    switch (fmt) {
        case DH_KV_F16:
        case DH_KV_BF16: return 2;
        case DH_KV_F32: return 4;
        case DH_KV_FP8_E4M3:
        case DH_KV_MXFP8: return 1;
        default: return 0;
    }
}

uint64_t kv_scale_bytes(uint32_t fmt, uint32_t hkv, uint32_t d) {
    if (fmt == DH_KV_FP8_E4M3) return uint64_t(2) * hkv * 4;
    if (fmt == DH_KV_MXFP8) return uint64_t(2) * hkv * 16 * (d / 32);
    return 0;
}

inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;

inline double normal_at(uint64_t seed, uint64_t index) {
    const uint64_t key = mix64(seed + kGolden);
    const uint64_t pair = index >> 1;
    const uint64_t h1 = mix64(key + (2 * pair + 1) * kGolden);
    const uint64_t h2 = mix64(key + (2 * pair + 2) * kGolden);
    const double u1 = double((h1 >> 11) + 1) * 0x1.0p-53;   // (0, 1]
    const double u2 = double(h2 >> 11) * 0x1.0p-53;         // [0, 1)
    const double rad = sqrt(-2.0 * log(u1));
    const double th = 2.0 * M_PI * u2;
    return (index & 1) ? rad * sin(th) : rad * cos(th);
}

inline uint16_t f32_to_bf16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return uint16_t((u >> 16) | 0x40);   // quiet NaN
    u += 0x7FFFu + ((u >> 16) & 1u);
    return uint16_t(u >> 16);
}

inline uint16_t f32_to_f16_rne(float f) {
    _Float16 h = (_Float16)f;   // IEEE conversion, round to nearest even
    uint16_t u;
    memcpy(&u, &h, 2);
    return u;
}

// E4M3 (OCP FN) from float, round to nearest even, saturating to +-448.
inline uint8_t f32_to_e4m3(float x) {
    const uint8_t sign = std::signbit(x) ? 0x80 : 0x00;
    if (x != x) return 0x7F;
    float a = fabsf(x);
    if (a >= 448.0f) return sign | 0x7E;
    if (a < 0x1.0p-6f) {                        // subnormal range, step 2^-9
        const float m = nearbyintf(a * 512.0f);  // 0..8 (8 -> smallest normal)
        return sign | uint8_t(m);
    }
    int e;
    const float fr = frexpf(a, &e);              // a = fr * 2^e, fr in [0.5, 1)
    int exp = e - 1;                             // a = (2 fr) * 2^exp
    float q = nearbyintf((2.0f * fr - 1.0f) * 8.0f);
    if (q >= 8.0f) {
        q = 0.0f;
        exp += 1;
    }
    const int code = ((exp + 7) << 3) | int(q);
    return sign | uint8_t(code > 0x7E ? 0x7E : code);
}

template <typename F>
void parallel_for(uint64_t n, F&& f) {
    unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    if (n < 4096) nt = 1;
    if (nt == 1) {
        f(uint64_t(0), n);
        return;
    }
    std::vector<std::thread> th;
    for (unsigned t = 0; t < nt; ++t) {
        const uint64_t a = n * t / nt, b = n * (t + 1) / nt;
        th.emplace_back([=, &f] { f(a, b); });
    }
    for (auto& x : th) x.join();
}

}  // namespace

extern "C" {

const char* dh_testdata_last_error(void) { return g_error; }

double dh_synth_normal(uint64_t seed, uint64_t index) { return normal_at(seed, index); }

dh_status dh_synth_fill(void* out, uint32_t dtype, uint64_t seed, uint64_t first, uint64_t n) {
    if (!out && n) return fail(DH_EINVAL, "out is NULL");
    if (dtype > DH_DTYPE_F32) return fail(DH_EINVAL, "bad dtype %u", dtype);
    parallel_for(n, [&](uint64_t a, uint64_t b) {
        for (uint64_t i = a; i < b; ++i) {
            const float v = float(normal_at(seed, first + i));
            if (dtype == DH_DTYPE_F32) static_cast<float*>(out)[i] = v;
            else if (dtype == DH_DTYPE_BF16) static_cast<uint16_t*>(out)[i] = f32_to_bf16_rne(v);
            else static_cast<uint16_t*>(out)[i] = f32_to_f16_rne(v);
        }
    });
    return DH_OK;
}

dh_status dh_synth_pages(uint32_t fmt, uint32_t hkv, uint32_t d, uint64_t seed, const uint32_t* ids,
                         uint32_t n, double outlier, uint32_t outlier_every, void* data, void* scales) {
    const uint32_t eb = kv_elem_bytes(fmt);
    if (eb == 0) return fail(DH_EINVAL, "bad kv_format %u", fmt);
    if (n && (!ids || !data)) return fail(DH_EINVAL, "NULL argument");
    if ((fmt == DH_KV_FP8_E4M3 || fmt == DH_KV_MXFP8) && n && !scales)
        return fail(DH_EINVAL, "scales are required for this kv format");
    if (d % 32) return fail(DH_EINVAL, "head_dim must be a multiple of 32");
    const uint64_t block = uint64_t(16) * d;              // elements of one (plane, head) block
    const uint64_t elems = 2ull * hkv * block;            // elements per page
    const uint64_t page_bytes = elems * eb;
    const uint64_t scale_bytes = kv_scale_bytes(fmt, hkv, d);
    parallel_for(n, [&](uint64_t a, uint64_t b) {
        std::vector<float> x(block);
        for (uint64_t i = a; i < b; ++i) {
            const uint64_t pid = ids[i];
            uint8_t* dp = static_cast<uint8_t*>(data) + i * page_bytes;
            uint8_t* sp = scales ? static_cast<uint8_t*>(scales) + i * scale_bytes : nullptr;
            for (uint64_t blk = 0; blk < 2ull * hkv; ++blk) {   // (plane, head) blocks in layout order
                const uint64_t base = pid * elems + blk * block;
                for (uint64_t e = 0; e < block; ++e) {
                    float v = float(normal_at(seed, base + e));
                    if (outlier_every && (mix64(seed ^ 0x5DEECE66Dull ^ ((base + e) * kGolden)) % outlier_every) == 0)
                        v = float(v < 0 ? -outlier : outlier);
                    x[e] = v;
                }
                if (fmt == DH_KV_F32) {
                    memcpy(dp + blk * block * 4, x.data(), block * 4);
                } else if (fmt == DH_KV_BF16 || fmt == DH_KV_F16) {
                    uint16_t* o = reinterpret_cast<uint16_t*>(dp + blk * block * 2);
                    for (uint64_t e = 0; e < block; ++e)
                        o[e] = fmt == DH_KV_BF16 ? f32_to_bf16_rne(x[e]) : f32_to_f16_rne(x[e]);
                } else if (fmt == DH_KV_FP8_E4M3) {
                    float amax = 0.f;
                    for (uint64_t e = 0; e < block; ++e) amax = std::max(amax, fabsf(x[e]));
                    const float sc = amax > 0.f ? amax / 448.0f : 1.0f;
                    uint8_t* o = dp + blk * block;
                    for (uint64_t e = 0; e < block; ++e) o[e] = f32_to_e4m3(x[e] / sc);
                    memcpy(sp + blk * 4, &sc, 4);   // scale record [plane][head] == blk order
                } else {  // MXFP8: E8M0 per 32 consecutive elements along head_dim
                    uint8_t* o = dp + blk * block;
                    uint8_t* so = sp + blk * (block / 32);
                    for (uint64_t g0 = 0; g0 < block; g0 += 32) {
                        float amax = 0.f;
                        for (int k = 0; k < 32; ++k) amax = std::max(amax, fabsf(x[g0 + k]));
                        int sexp = -127;
                        if (amax > 0.f) {
                            int e;
                            frexpf(amax, &e);          // amax in [2^(e-1), 2^e)
                            sexp = (e - 1) - 8;        // floor(log2 amax) - emax(E4M3)
                        }
                        sexp = std::max(-127, std::min(127, sexp));
                        so[g0 / 32] = uint8_t(sexp + 127);
                        const float inv = ldexpf(1.0f, -sexp);
                        for (int k = 0; k < 32; ++k) o[g0 + k] = f32_to_e4m3(x[g0 + k] * inv);
                    }
                }
            }
        }
    });
    return DH_OK;
}

}  // extern "C"
