// Device-side page writes with quantise-on-write: the device half of
// ReferenceBackend::append_kv / store_kv (crates/dendrite-core/src/attention/
// backend.rs:285-301, 140-143) for K/V already resident in HBM.
//
// Also the plan patch kernel (dh_plan_update): a few words of a decode
// plan's device tables rewritten in stream order.
//
// A source page is [2][num_kv_heads][16][head_dim] elements (K plane, then
// V; tokens past a partial page's length are zero) of f32, bf16 or f16.  It
// becomes page page_ids[i] of the pool in the pool's format:
//   F32 / BF16 / F16: the element converted, round to nearest even;
//   FP8_E4M3: per (page, K|V, head) block scale = amax / 448 (1 if amax is
//     0), element = E4M3 "FN" of x / scale, round to nearest even, saturated
//     to +-448 (fp8.rs:39-52 states that range);
//   MXFP8: per 32 consecutive elements along head_dim (quantization/mod.rs:
//     96-97) scale = 2^(floor(log2 amax) - 8) stored as E8M0 (clamped to
//     2^-127 .. 2^127), element = E4M3 of x / scale, saturated.
//
// One wave per (page, plane, head) block of 16 x D elements: lane l holds
// elements [l E, (l + 1) E), E = D / 4 (whole MX groups at head_dim >= 128,
// half a group at 64).  HBM-bound: the source read and the page write,
// each block's loads and stores 16-byte vectors.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "dh_device.hpp"

namespace dh {
namespace {

typedef uint32_t w4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kSrcF16 = 0, kSrcBF16 = 1, kSrcF32 = 2;   // DH_DTYPE_*
constexpr uint32_t kF16 = 0, kBF16 = 1, kF32 = 2, kFP8 = 3, kMX = 4;   // DH_KV_*

struct WriteArgs {
    const uint32_t* ids;     // device, [n]; ids >= num_pages are skipped
    const void* src;         // device, [n][2][hkv][16][D] of the source dtype
    uint8_t* data;           // pool data
    uint8_t* scales;         // pool scale records (FP8, MXFP8)
    uint32_t n, hkv, num_pages;
};

template <uint32_t SRC, int E>
__device__ __forceinline__ void load_src(const void* src, uint64_t e0, float (&x)[E]) {
    if constexpr (SRC == kSrcF32) {
        const w4* p = reinterpret_cast<const w4*>(static_cast<const float*>(src) + e0);
        #pragma unroll
        for (int v = 0; v < E / 4; ++v) {
            const w4 w = p[v];
            #pragma unroll
            for (int k = 0; k < 4; ++k) x[4 * v + k] = __uint_as_float(w[k]);
        }
    } else {
        const w4* p = reinterpret_cast<const w4*>(static_cast<const uint16_t*>(src) + e0);
        #pragma unroll
        for (int v = 0; v < E / 8; ++v) {
            const w4 w = p[v];
            #pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t lo = w[k] & 0xFFFFu, hi = w[k] >> 16;
                if constexpr (SRC == kSrcBF16) {
                    x[8 * v + 2 * k] = __uint_as_float(lo << 16);
                    x[8 * v + 2 * k + 1] = __uint_as_float(hi << 16);
                } else {
                    x[8 * v + 2 * k] = float(__builtin_bit_cast(_Float16, uint16_t(lo)));
                    x[8 * v + 2 * k + 1] = float(__builtin_bit_cast(_Float16, uint16_t(hi)));
                }
            }
        }
    }
}

// Four E4M3 codes (x already divided by its scale): clamp to +-448, then the
// hardware conversion (round to nearest even), so out-of-range values
// saturate instead of becoming NaN.
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
    auto cl = [](float v) { return fminf(fmaxf(v, -448.f), 448.f); };
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(cl(a), cl(b), 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(cl(c), cl(d), w, true);
    return uint32_t(w);
}

template <int E>
__device__ __forceinline__ void store_e4m3(uint8_t* dst, const float (&y)[E]) {
    w4* p = reinterpret_cast<w4*>(dst);
    #pragma unroll
    for (int v = 0; v < E / 16; ++v) {
        w4 o;
        #pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int e = 16 * v + 4 * k;
            o[k] = e4m3x4(y[e], y[e + 1], y[e + 2], y[e + 3]);
        }
        p[v] = o;
    }
}

__device__ __forceinline__ float wave_max(float x) {
    #pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
    return x;
}

// E8M0 exponent of a group with max magnitude amax: floor(log2 amax) - 8
// (E4M3's largest exponent), clamped to the E8M0 range; -127 for amax = 0.
__device__ __forceinline__ int mx_exponent(float amax) {
    if (!(amax > 0.f)) return -127;
    const int e = __builtin_amdgcn_frexp_expf(amax);   // amax in [2^(e-1), 2^e)
    return min(127, max(-127, e - 1 - 8));
}

template <int D, uint32_t SRC, uint32_t FMT>
__global__ __launch_bounds__(256) void write_pages_kernel(WriteArgs w) {
    constexpr int E = D / 4;
    const int lane = threadIdx.x & 63;
    const uint32_t blk = blockIdx.x * 4 + (threadIdx.x >> 6);   // (page i, plane, head)
    const uint32_t per_page = 2 * w.hkv;
    if (blk >= w.n * per_page) return;
    const uint32_t i = blk / per_page, ph = blk - i * per_page;
    // The source block does not depend on the page id: both loads go out
    // together, so a block costs one memory round trip before its stores.
    float x[E];
    load_src<SRC, E>(w.src, uint64_t(blk) * 16 * D + uint64_t(lane) * E, x);
    const uint32_t pid = w.ids[i];
    if (pid >= w.num_pages) return;
    const uint64_t dblk = uint64_t(pid) * per_page + ph;   // destination block
    const uint64_t de = dblk * 16 * D + uint64_t(lane) * E;
    if constexpr (FMT == kF32) {
        w4* p = reinterpret_cast<w4*>(reinterpret_cast<float*>(w.data) + de);
        #pragma unroll
        for (int v = 0; v < E / 4; ++v)
            p[v] = w4{__float_as_uint(x[4 * v]), __float_as_uint(x[4 * v + 1]), __float_as_uint(x[4 * v + 2]),
                      __float_as_uint(x[4 * v + 3])};
    } else if constexpr (FMT == kBF16 || FMT == kF16) {
        w4* p = reinterpret_cast<w4*>(reinterpret_cast<uint16_t*>(w.data) + de);
        #pragma unroll
        for (int v = 0; v < E / 8; ++v) {
            w4 o;
            #pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float a = x[8 * v + 2 * k], b = x[8 * v + 2 * k + 1];
                if constexpr (FMT == kBF16) {
                    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
                    o[k] = __builtin_bit_cast(uint32_t, b2{(__bf16)a, (__bf16)b});
                } else {
                    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
                    o[k] = __builtin_bit_cast(uint32_t, h2{(_Float16)a, (_Float16)b});
                }
            }
            p[v] = o;
        }
    } else if constexpr (FMT == kFP8) {
        float amax = 0.f;
        #pragma unroll
        for (int e = 0; e < E; ++e) amax = fmaxf(amax, fabsf(x[e]));
        amax = wave_max(amax);
        const float sc = amax > 0.f ? amax / 448.0f : 1.0f;
        float y[E];
        #pragma unroll
        for (int e = 0; e < E; ++e) y[e] = x[e] / sc;
        store_e4m3<E>(w.data + de, y);
        if (lane == 0) reinterpret_cast<float*>(w.scales)[dblk] = sc;
    } else {   // MXFP8
        constexpr int G = E >= 32 ? E / 32 : 1;   // groups this lane scales
        float y[E];
        uint32_t codes = 0;
        #pragma unroll
        for (int gi = 0; gi < G; ++gi) {
            constexpr int GL = E >= 32 ? 32 : E;   // elements of the group in this lane
            float amax = 0.f;
            #pragma unroll
            for (int k = 0; k < GL; ++k) amax = fmaxf(amax, fabsf(x[gi * GL + k]));
            if constexpr (E < 32) amax = fmaxf(amax, __shfl_xor(amax, 1, 64));   // the group's other half
            const int se = mx_exponent(amax);
            const float inv = __builtin_amdgcn_ldexpf(1.0f, -se);
            #pragma unroll
            for (int k = 0; k < GL; ++k) y[gi * GL + k] = x[gi * GL + k] * inv;
            codes |= uint32_t(se + 127) << (8 * gi);
        }
        store_e4m3<E>(w.data + de, y);
        // Scale records [page][plane][head][16][D / 32]: this block's 16 D / 32
        // bytes, lane l's groups at l E / 32 (lane pairs share one at D = 64).
        uint8_t* so = w.scales + dblk * (16 * D / 32);
        if constexpr (E >= 32) {
            #pragma unroll
            for (int gi = 0; gi < G; ++gi) so[lane * G + gi] = uint8_t(codes >> (8 * gi));
        } else {
            if ((lane & 1) == 0) so[lane >> 1] = uint8_t(codes);
        }
    }
}

template <int D, uint32_t SRC>
hipError_t launch_write_d(const WriteArgs& w, uint32_t fmt, hipStream_t s) {
    dim3 grid((w.n * 2 * w.hkv + 3) / 4), block(256);
    switch (fmt) {
        case kF32: hipLaunchKernelGGL((write_pages_kernel<D, SRC, kF32>), grid, block, 0, s, w); break;
        case kBF16: hipLaunchKernelGGL((write_pages_kernel<D, SRC, kBF16>), grid, block, 0, s, w); break;
        case kF16: hipLaunchKernelGGL((write_pages_kernel<D, SRC, kF16>), grid, block, 0, s, w); break;
        case kFP8: hipLaunchKernelGGL((write_pages_kernel<D, SRC, kFP8>), grid, block, 0, s, w); break;
        case kMX: hipLaunchKernelGGL((write_pages_kernel<D, SRC, kMX>), grid, block, 0, s, w); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int D>
hipError_t launch_write_src(const WriteArgs& w, uint32_t src_dtype, uint32_t fmt, hipStream_t s) {
    switch (src_dtype) {
        case kSrcF32: return launch_write_d<D, kSrcF32>(w, fmt, s);
        case kSrcBF16: return launch_write_d<D, kSrcBF16>(w, fmt, s);
        case kSrcF16: return launch_write_d<D, kSrcF16>(w, fmt, s);
        default: return hipErrorInvalidValue;
    }
}

struct PatchArgs {
    uint32_t* words;
    uint32_t n;
    uint32_t idx[kPatchWords];
    uint32_t val[kPatchWords];
};

// One lane applies the patches in order (a later write to the same word
// wins); a handful of words per decode step.
__global__ __launch_bounds__(64) void plan_patch_kernel(PatchArgs a) {
    if (threadIdx.x != 0) return;
    for (uint32_t k = 0; k < a.n; ++k) a.words[a.idx[k]] = a.val[k];
}

}  // namespace

int launch_plan_patch(uint32_t* words, uint32_t n, const uint32_t* idx, const uint32_t* val, void* stream) {
    if (n == 0) return hipSuccess;
    if (n > kPatchWords) return hipErrorInvalidValue;
    PatchArgs a;
    a.words = words;
    a.n = n;
    for (uint32_t k = 0; k < n; ++k) {
        a.idx[k] = idx[k];
        a.val[k] = val[k];
    }
    hipLaunchKernelGGL(plan_patch_kernel, dim3(1), dim3(64), 0, reinterpret_cast<hipStream_t>(stream), a);
    return hipGetLastError();
}

int launch_write_pages(const uint32_t* ids, uint32_t n, const void* src, uint32_t src_dtype, uint8_t* data,
                       uint8_t* scales, uint32_t num_pages, uint32_t hkv, uint32_t d, uint32_t fmt,
                       void* stream) {
    if (n == 0) return hipSuccess;
    WriteArgs w{ids, src, data, scales, n, hkv, num_pages};
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    switch (d) {
        case 64: return launch_write_src<64>(w, src_dtype, fmt, s);
        case 128: return launch_write_src<128>(w, src_dtype, fmt, s);
        case 256: return launch_write_src<256>(w, src_dtype, fmt, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace dh
