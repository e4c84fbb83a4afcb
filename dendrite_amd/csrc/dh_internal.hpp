// Internal host-side definitions shared by the C-ABI implementation files.
#pragma once
#include <stdarg.h>
#include <stdint.h>
#include <string>

#include "dendrite_hip.h"

namespace dh {

// Records a failure for dh_last_error() and returns the status.
dh_status fail(dh_status s, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

inline uint32_t kv_elem_bytes(uint32_t fmt) {
    switch (fmt) {
        case DH_KV_F16:
        case DH_KV_BF16: return 2;
        case DH_KV_F32: return 4;
        case DH_KV_FP8_E4M3:
        case DH_KV_MXFP8: return 1;
        default: return 0;
    }
}

inline uint32_t dtype_bytes(uint32_t dt) {
    switch (dt) {
        case DH_DTYPE_F16:
        case DH_DTYPE_BF16: return 2;
        case DH_DTYPE_F32: return 4;
        default: return 0;
    }
}

// Scale record bytes of one page (both planes, all KV heads).
inline uint64_t kv_scale_bytes(uint32_t fmt, uint32_t hkv, uint32_t d) {
    if (fmt == DH_KV_FP8_E4M3) return uint64_t(2) * hkv * 4;
    if (fmt == DH_KV_MXFP8) return uint64_t(2) * hkv * 16 * (d / 32);
    return 0;
}

}  // namespace dh
