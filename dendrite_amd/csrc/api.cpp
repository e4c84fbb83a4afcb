// C-ABI implementation: backend, device page pool, decode plans and the
// decode launch.  Replaces crates/dendrite-ffi (cuda.rs device handling and
// the FlashInfer BatchDecodeKernel / CascadeAttention wrappers) and fills the
// FlashInferBackend slot of crates/dendrite-core/src/attention/flashinfer.rs.
#include <hip/hip_runtime_api.h>

#include <math.h>
#include <stddef.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "dh_device.hpp"
#include "dh_internal.hpp"
#include "planner.hpp"

namespace dh {

static thread_local std::string g_last_error;

dh_status fail(dh_status s, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return s;
}

void clear_error() { g_last_error.clear(); }

int launch_e4m3_debug(const uint32_t* codes, const uint8_t* e8m0, uint32_t n4, uint32_t* out,
                      void* stream);
int launch_scatter(uint8_t* dst, const uint8_t* src, const uint32_t* ids, uint32_t n,
                   uint64_t rec_bytes, void* stream);

}  // namespace dh

using dh::fail;

// A failed HIP call also leaves the runtime's per-thread last error set,
// where the caller's next hipGetLastError (torch checks it after every
// launch) would find it; the error is reported through dh_status instead.
#define DH_HIP(expr)                                                                      \
    do {                                                                                  \
        hipError_t e_ = (expr);                                                           \
        if (e_ != hipSuccess) {                                                           \
            (void)hipGetLastError();                                                      \
            return fail(DH_EHIP, "%s failed: %s", #expr, hipGetErrorString(e_));          \
        }                                                                                 \
    } while (0)

namespace dh {

// Makes `device` current for the scope and restores the caller's device.
class DeviceGuard {
public:
    explicit DeviceGuard(int device) {
        if (hipGetDevice(&prev_) != hipSuccess) prev_ = -1;
        err_ = (prev_ == device) ? hipSuccess : hipSetDevice(device);
        if (err_ != hipSuccess) (void)hipGetLastError();
        set_ = (err_ == hipSuccess && prev_ >= 0 && prev_ != device);
    }
    ~DeviceGuard() {
        if (set_) (void)hipSetDevice(prev_);
    }
    hipError_t error() const { return err_; }
    DeviceGuard(const DeviceGuard&) = delete;
    DeviceGuard& operator=(const DeviceGuard&) = delete;

private:
    int prev_ = -1;
    hipError_t err_ = hipSuccess;
    bool set_ = false;
};

}  // namespace dh

#define DH_DEVICE(dev)                                                                    \
    dh::DeviceGuard device_guard_(dev);                                                   \
    if (device_guard_.error() != hipSuccess)                                              \
    return fail(DH_EHIP, "hipSetDevice(%d) failed: %s", int(dev), hipGetErrorString(device_guard_.error()))

// Pools and plans keep their backend alive: a handle may be destroyed in any
// order relative to the objects made from it.
struct dh_backend {
    int device;
    std::atomic<int> refs;
    // Device address of the GPU's static scratch array (dh_decode_batch_static),
    // looked up once at dh_create with the device current.
    void* scratch;
};

static dh_backend* retain(dh_backend* be) {
    be->refs.fetch_add(1, std::memory_order_relaxed);
    return be;
}

static void release(dh_backend* be) {
    if (be && be->refs.fetch_sub(1, std::memory_order_acq_rel) == 1) delete be;
}

struct dh_pool {
    dh_backend* be;
    uint32_t num_pages, hkv, d, fmt, eb;
    uint64_t page_bytes, scale_bytes;
    uint8_t* data;
    uint8_t* scales;
    // Staging memory of host page uploads (dh_pool_write_pages), kept from
    // call to call and grown when a call needs more; the mutex serialises
    // uploads that would share it.
    std::mutex stage_mu;
    uint8_t* stage = nullptr;
    uint64_t stage_bytes = 0;
};

struct dh_plan {
    dh_backend* be;
    dh_attn_config cfg;
    uint32_t batch;
    uint32_t pool_pages;
    uint32_t n_items;
    uint32_t n_tasks;
    uint32_t n_group_items;
    uint32_t n_wave_items;
    uint32_t n_slots;
    uint8_t* dev;
    dh::Item* items;
    uint32_t* pages;
    dh::SeqSlot* seqslots;
    uint32_t* slot_ptr;
    // Prefill plans: tokens each query sees, item token ranges.
    bool prefill;
    uint32_t* row_len;
    dh::ItemLim* item_lim;
    dh_plan_stats stats;
    size_t ws_bytes;
    size_t ws_lse_off;
    // Decode plans: host copies of the last-chunk tables (HostPlan::tail_*)
    // for dh_plan_update, and where items and pages start in dev (words).
    std::vector<uint32_t> tail_off, tail_n, tail_cap, tail_item_ptr, tail_items;
    size_t items_word, pages_word;
    // Prefill plans with one partial state per row, and direct decode plans
    // (each workgroup merges its own rows): the attention kernel writes out
    // and there is no merge launch.
    bool direct;
    uint32_t max_slots;      // most partial states of one sequence
    uint32_t uniform_slots;  // every sequence's count of partial states when they are all equal, else 0
};

extern "C" {

const char* dh_last_error(void) { return dh::g_last_error.c_str(); }
const char* dh_version(void) { return "dendrite-hip 0.1.0 (gfx950)"; }

/* ------------------------------------------------------------------ config */

dh_status dh_attn_config_init(dh_attn_config* cfg, uint32_t num_heads, uint32_t num_kv_heads,
                              uint32_t head_dim) {
    if (!cfg) return fail(DH_EINVAL, "cfg is NULL");
    memset(cfg, 0, sizeof *cfg);
    cfg->num_heads = num_heads;
    cfg->num_kv_heads = num_kv_heads;
    cfg->head_dim = head_dim;
    // backend.rs:37: 1.0 / (head_dim as f32).sqrt(), in f32.
    cfg->scale = 1.0f / sqrtf(float(head_dim));
    cfg->sliding_window = 0;
    cfg->gqa_mapping = DH_GQA_TILED;
    cfg->q_dtype = DH_DTYPE_BF16;
    cfg->kv_format = DH_KV_BF16;
    return DH_OK;
}

uint32_t dh_attn_config_num_queries_per_kv(const dh_attn_config* cfg) {
    if (!cfg || cfg->num_kv_heads == 0) return 0;
    return cfg->num_heads / cfg->num_kv_heads;
}

static dh_status validate_config(const dh_attn_config* cfg) {
    if (!cfg) return fail(DH_EINVAL, "config is NULL");
    if (cfg->num_heads == 0 || cfg->num_kv_heads == 0)
        return fail(DH_EINVAL, "num_heads and num_kv_heads must be positive");
    // batch_decode.rs:41-45
    if (cfg->num_heads % cfg->num_kv_heads != 0)
        return fail(DH_EINVAL, "num_qo_heads must be divisible by num_kv_heads");
    // batch_decode.rs:33-39, flashinfer/mod.rs:20
    if (cfg->head_dim != 64 && cfg->head_dim != 128 && cfg->head_dim != 256)
        return fail(DH_EINVAL, "unsupported head_dim: %u, supported: [64, 128, 256]", cfg->head_dim);
    // sliding_window is ignored, as ReferenceBackend::decode ignores it
    // (attention/backend.rs:206-265 never reads the field).
    if (cfg->gqa_mapping > DH_GQA_INTERLEAVED) return fail(DH_EINVAL, "bad gqa_mapping %u", cfg->gqa_mapping);
    if (cfg->q_dtype > DH_DTYPE_F32) return fail(DH_EINVAL, "bad q_dtype %u", cfg->q_dtype);
    if (cfg->kv_format > DH_KV_MXFP8) return fail(DH_EINVAL, "bad kv_format %u", cfg->kv_format);
    if (!(cfg->scale == cfg->scale) || isinf(cfg->scale)) return fail(DH_EINVAL, "scale must be finite");
    if (!dh::attend_supported(cfg->q_dtype, cfg->kv_format, cfg->head_dim))
        return fail(DH_EUNSUPPORTED, "q dtype %u with kv format %u is not supported", cfg->q_dtype,
                    cfg->kv_format);
    return DH_OK;
}

/* ----------------------------------------------------------------- backend */

int dh_is_available(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n > 0;
}

dh_status dh_device_count(int* count) {
    if (!count) return fail(DH_EINVAL, "count is NULL");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e == hipErrorNoDevice) n = 0;
    else if (e != hipSuccess) return fail(DH_EHIP, "hipGetDeviceCount: %s", hipGetErrorString(e));
    *count = n;
    return DH_OK;
}

dh_status dh_create(int device, dh_backend** out) {
    if (!out) return fail(DH_EINVAL, "out is NULL");
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0)
        return fail(DH_EUNSUPPORTED, "no HIP device available");
    if (device < 0 || device >= n) return fail(DH_EINVAL, "device %d out of range (%d devices)", device, n);
    hipDeviceProp_t prop;
    DH_HIP(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(DH_EUNSUPPORTED, "device %d is %s; this library is built for gfx950", device,
                    prop.gcnArchName);
    void* scratch = nullptr;
    {
        DH_DEVICE(device);
        const hipError_t e = hipError_t(dh::static_scratch_address(&scratch));
        if (e != hipSuccess || !scratch)
            return fail(DH_EHIP, "static scratch of device %d: %s", device, hipGetErrorString(e));
    }
    dh_backend* be = new (std::nothrow) dh_backend;
    if (!be) return fail(DH_ENOMEM, "out of host memory");
    be->device = device;
    be->refs.store(1, std::memory_order_relaxed);
    be->scratch = scratch;
    *out = be;
    return DH_OK;
}

dh_status dh_destroy(dh_backend* be) {
    release(be);
    return DH_OK;
}

dh_status dh_memory_info(dh_backend* be, size_t* free_b, size_t* total_b) {
    if (!be || !free_b || !total_b) return fail(DH_EINVAL, "NULL argument");
    DH_DEVICE(be->device);
    DH_HIP(hipMemGetInfo(free_b, total_b));
    return DH_OK;
}

dh_status dh_synchronize(dh_backend* be) {
    if (!be) return fail(DH_EINVAL, "backend is NULL");
    DH_DEVICE(be->device);
    DH_HIP(hipDeviceSynchronize());
    return DH_OK;
}

/* -------------------------------------------------------------------- pool */

dh_status dh_pool_create(dh_backend* be, uint32_t num_pages, uint32_t hkv, uint32_t d,
                         uint32_t page_size, uint32_t fmt, dh_pool** out) {
    if (!be || !out) return fail(DH_EINVAL, "NULL argument");
    *out = nullptr;
    if (page_size != DH_PAGE_SIZE) return fail(DH_EINVAL, "page_size must be %u", DH_PAGE_SIZE);
    if (num_pages == 0 || hkv == 0) return fail(DH_EINVAL, "num_pages and num_kv_heads must be positive");
    if (d != 64 && d != 128 && d != 256) return fail(DH_EINVAL, "unsupported head_dim: %u", d);
    const uint32_t eb = dh::kv_elem_bytes(fmt);
    if (eb == 0) return fail(DH_EINVAL, "bad kv_format %u", fmt);
    DH_DEVICE(be->device);
    dh_pool* p = new (std::nothrow) dh_pool;
    if (!p) return fail(DH_ENOMEM, "out of host memory");
    p->be = be;
    p->num_pages = num_pages;
    p->hkv = hkv;
    p->d = d;
    p->fmt = fmt;
    p->eb = eb;
    p->page_bytes = uint64_t(2) * hkv * DH_PAGE_SIZE * d * eb;
    p->scale_bytes = dh::kv_scale_bytes(fmt, hkv, d);
    p->data = nullptr;
    p->scales = nullptr;
    const unsigned long long data_bytes = (unsigned long long)(p->page_bytes * num_pages);
    hipError_t e = hipMalloc(&p->data, data_bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        delete p;
        return fail(DH_ENOMEM, "pool allocation of %llu bytes failed: %s", data_bytes, hipGetErrorString(e));
    }
    e = hipMemset(p->data, 0, p->page_bytes * num_pages);
    if (e == hipSuccess && p->scale_bytes) {
        e = hipMalloc(&p->scales, p->scale_bytes * num_pages);
        if (e == hipSuccess) e = hipMemset(p->scales, 0, p->scale_bytes * num_pages);
    }
    if (e != hipSuccess) {
        (void)hipGetLastError();
        (void)hipFree(p->data);
        if (p->scales) (void)hipFree(p->scales);
        delete p;
        return fail(DH_ENOMEM, "pool initialisation failed: %s", hipGetErrorString(e));
    }
    retain(be);
    *out = p;
    return DH_OK;
}

dh_status dh_pool_destroy(dh_pool* p) {
    if (!p) return DH_OK;
    {
        dh::DeviceGuard g(p->be->device);
        (void)hipDeviceSynchronize();
        (void)hipFree(p->data);
        if (p->scales) (void)hipFree(p->scales);
        if (p->stage) (void)hipFree(p->stage);
        (void)hipGetLastError();
    }
    release(p->be);
    delete p;
    return DH_OK;
}

size_t dh_pool_page_bytes(const dh_pool* p) { return p ? size_t(p->page_bytes) : 0; }
size_t dh_pool_scale_bytes(const dh_pool* p) { return p ? size_t(p->scale_bytes) : 0; }
uint32_t dh_pool_num_pages(const dh_pool* p) { return p ? p->num_pages : 0; }
void* dh_pool_data(dh_pool* p) { return p ? p->data : nullptr; }
void* dh_pool_scales(dh_pool* p) { return p ? p->scales : nullptr; }

// FP8 E4M3 block scales must be finite and positive: the kernels order a
// page's scaled scores by its raw ones, and a masked -inf times 0 is NaN.
// The quantiser never makes another (amax / 448, or 1 for an all-zero block).
static bool fp8_scales_ok(const void* scales, uint64_t n) {
    const uint8_t* b = static_cast<const uint8_t*>(scales);
    for (uint64_t i = 0; i < n; ++i) {
        float x;
        memcpy(&x, b + 4 * i, 4);
        if (!(x > 0.f) || isinf(x)) return false;
    }
    return true;
}

dh_status dh_pool_write_tokens(dh_pool* p, uint32_t page_id, uint32_t tok_offset, uint32_t n_tok,
                               const void* k, const void* v, const void* k_scale,
                               const void* v_scale, void* stream) {
    if (!p || !k || !v) return fail(DH_EINVAL, "NULL argument");
    if (page_id >= p->num_pages) return fail(DH_EINVAL, "page id %u outside the pool", page_id);
    if (n_tok == 0 || tok_offset + n_tok > DH_PAGE_SIZE)
        return fail(DH_EINVAL, "tokens [%u, %u) do not fit a %u-token page", tok_offset,
                    tok_offset + n_tok, DH_PAGE_SIZE);
    if ((p->fmt == DH_KV_FP8_E4M3 || p->fmt == DH_KV_MXFP8) && (!k_scale || !v_scale))
        return fail(DH_EINVAL, "scales are required for this kv format");
    if (p->fmt == DH_KV_FP8_E4M3 && (!fp8_scales_ok(k_scale, p->hkv) || !fp8_scales_ok(v_scale, p->hkv)))
        return fail(DH_EINVAL, "FP8 block scales must be finite and positive");
    DH_DEVICE(p->be->device);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const uint64_t row = uint64_t(p->d) * p->eb;
    for (uint32_t plane = 0; plane < 2; ++plane) {
        const uint8_t* src = static_cast<const uint8_t*>(plane ? v : k);
        for (uint32_t h = 0; h < p->hkv; ++h) {
            uint8_t* dst = p->data + dh::plane_offset(page_id, plane, h, p->hkv, p->d, p->eb) +
                           uint64_t(tok_offset) * row;
            DH_HIP(hipMemcpyAsync(dst, src + uint64_t(h) * n_tok * row, n_tok * row,
                                  hipMemcpyHostToDevice, s));
        }
    }
    if (p->fmt == DH_KV_FP8_E4M3) {
        for (uint32_t plane = 0; plane < 2; ++plane) {
            uint8_t* dst = p->scales + (uint64_t(page_id) * 2 + plane) * p->hkv * 4;
            DH_HIP(hipMemcpyAsync(dst, plane ? v_scale : k_scale, p->hkv * 4, hipMemcpyHostToDevice, s));
        }
    } else if (p->fmt == DH_KV_MXFP8) {
        const uint64_t G = p->d / 32;
        for (uint32_t plane = 0; plane < 2; ++plane) {
            const uint8_t* src = static_cast<const uint8_t*>(plane ? v_scale : k_scale);
            for (uint32_t h = 0; h < p->hkv; ++h) {
                uint8_t* dst = p->scales + ((uint64_t(page_id) * 2 + plane) * p->hkv + h) * DH_PAGE_SIZE * G +
                               uint64_t(tok_offset) * G;
                DH_HIP(hipMemcpyAsync(dst, src + uint64_t(h) * n_tok * G, n_tok * G,
                                      hipMemcpyHostToDevice, s));
            }
        }
    }
    return DH_OK;
}

// Staging memory dh_pool_write_pages keeps between calls (larger uploads
// allocate, use and free their own).
constexpr uint64_t kKeepStage = 16ull << 20;

dh_status dh_pool_write_pages(dh_pool* p, const uint32_t* ids, uint32_t n, const void* data,
                              const void* scales, void* stream) {
    if (!p || (n && (!ids || !data))) return fail(DH_EINVAL, "NULL argument");
    if (p->scale_bytes && n && !scales) return fail(DH_EINVAL, "scales are required for this kv format");
    for (uint32_t i = 0; i < n; ++i)
        if (ids[i] >= p->num_pages) return fail(DH_EINVAL, "page id %u outside the pool", ids[i]);
    if (n == 0) return DH_OK;
    if (p->fmt == DH_KV_FP8_E4M3 && !fp8_scales_ok(scales, uint64_t(n) * p->scale_bytes / 4))
        return fail(DH_EINVAL, "FP8 block scales must be finite and positive");
    DH_DEVICE(p->be->device);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const uint32_t batch = std::min<uint32_t>(n, std::max<uint64_t>(1, (256ull << 20) / p->page_bytes));
    std::lock_guard<std::mutex> lock(p->stage_mu);
    // page data, scale records, page ids: one staging allocation
    const uint64_t ids_off = (uint64_t(batch) * (p->page_bytes + p->scale_bytes) + 255) & ~uint64_t(255);
    const uint64_t need = ids_off + uint64_t(batch) * sizeof(uint32_t);
    if (p->stage_bytes < need) {
        if (p->stage) (void)hipFree(p->stage);
        p->stage = nullptr;
        p->stage_bytes = 0;
        DH_HIP(hipMalloc(&p->stage, need));
        p->stage_bytes = need;
    }
    uint8_t* stage = p->stage;
    uint32_t* dids = reinterpret_cast<uint32_t*>(stage + ids_off);
    hipError_t e = hipSuccess;
    dh_status st = DH_OK;
    for (uint32_t i0 = 0; e == hipSuccess && i0 < n; i0 += batch) {
        const uint32_t m = std::min(batch, n - i0);
        e = hipMemcpyAsync(dids, ids + i0, m * sizeof(uint32_t), hipMemcpyHostToDevice, s);
        if (e == hipSuccess)
            e = hipMemcpyAsync(stage, static_cast<const uint8_t*>(data) + uint64_t(i0) * p->page_bytes,
                               uint64_t(m) * p->page_bytes, hipMemcpyHostToDevice, s);
        if (e == hipSuccess)
            e = hipError_t(dh::launch_scatter(p->data, stage, dids, m, p->page_bytes, s));
        if (e == hipSuccess && p->scale_bytes) {
            uint8_t* sst = stage + uint64_t(batch) * p->page_bytes;
            e = hipMemcpyAsync(sst, static_cast<const uint8_t*>(scales) + uint64_t(i0) * p->scale_bytes,
                               uint64_t(m) * p->scale_bytes, hipMemcpyHostToDevice, s);
            if (e == hipSuccess) e = hipError_t(dh::launch_scatter(p->scales, sst, dids, m, p->scale_bytes, s));
        }
        if (e == hipSuccess) e = hipStreamSynchronize(s);
    }
    if (e != hipSuccess) {
        st = fail(DH_EHIP, "page upload failed: %s", hipGetErrorString(e));
        (void)hipStreamSynchronize(s);   // nothing queued may still use the staging memory
        (void)hipGetLastError();
    }
    // The staging memory is kept for the next call only up to kKeepStage
    // bytes: an engine that sizes its pool to fill the device does not lose
    // the memory of one large upload for the pool's lifetime.  Every copy
    // that read it has completed (the stream was synchronised above).
    if (p->stage_bytes > kKeepStage) {
        (void)hipFree(p->stage);
        p->stage = nullptr;
        p->stage_bytes = 0;
    }
    return st;
}

dh_status dh_pool_write_pages_device(dh_pool* p, const uint32_t* ids, uint32_t n, const void* src,
                                     uint32_t src_dtype, void* stream) {
    if (!p) return fail(DH_EINVAL, "pool is NULL");
    if (n == 0) return DH_OK;
    if (!ids || !src) return fail(DH_EINVAL, "NULL argument");
    if (src_dtype > DH_DTYPE_F32) return fail(DH_EINVAL, "bad source dtype %u", src_dtype);
    if (reinterpret_cast<uintptr_t>(src) & 15) return fail(DH_EINVAL, "src must be 16-byte aligned");
    if (p->d != 64 && p->d != 128 && p->d != 256)
        return fail(DH_EUNSUPPORTED, "head_dim %u: device page writes take 64, 128 or 256", p->d);
    DH_DEVICE(p->be->device);
    const hipError_t e = hipError_t(dh::launch_write_pages(ids, n, src, src_dtype, p->data, p->scales,
                                                           p->num_pages, p->hkv, p->d, p->fmt, stream));
    if (e != hipSuccess) return fail(DH_EHIP, "page write launch failed: %s", hipGetErrorString(e));
    return DH_OK;
}

dh_status dh_pool_copy_page(dh_pool* p, uint32_t src, uint32_t dst, void* stream) {
    if (!p) return fail(DH_EINVAL, "pool is NULL");
    if (src >= p->num_pages || dst >= p->num_pages)
        return fail(DH_EINVAL, "page id outside the pool (src %u, dst %u)", src, dst);
    if (src == dst) return DH_OK;
    DH_DEVICE(p->be->device);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    DH_HIP(hipMemcpyAsync(p->data + uint64_t(dst) * p->page_bytes, p->data + uint64_t(src) * p->page_bytes,
                          p->page_bytes, hipMemcpyDeviceToDevice, s));
    if (p->scale_bytes)
        DH_HIP(hipMemcpyAsync(p->scales + uint64_t(dst) * p->scale_bytes,
                              p->scales + uint64_t(src) * p->scale_bytes, p->scale_bytes,
                              hipMemcpyDeviceToDevice, s));
    return DH_OK;
}

dh_status dh_pool_read_page(dh_pool* p, uint32_t page_id, void* data_out, void* scales_out) {
    if (!p || !data_out) return fail(DH_EINVAL, "NULL argument");
    if (page_id >= p->num_pages) return fail(DH_EINVAL, "page id %u outside the pool", page_id);
    DH_DEVICE(p->be->device);
    DH_HIP(hipDeviceSynchronize());
    DH_HIP(hipMemcpy(data_out, p->data + uint64_t(page_id) * p->page_bytes, p->page_bytes,
                     hipMemcpyDeviceToHost));
    if (p->scale_bytes && scales_out)
        DH_HIP(hipMemcpy(scales_out, p->scales + uint64_t(page_id) * p->scale_bytes, p->scale_bytes,
                         hipMemcpyDeviceToHost));
    return DH_OK;
}

/* -------------------------------------------------------------------- plan */

static size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Validates the planning inputs and runs the host planner.
static dh_status host_plan(const dh_attn_config* cfg, uint32_t num_pool_pages, const uint32_t* indptr,
                           const uint32_t* indices, uint32_t batch, uint32_t flags,
                           const dh_plan_options* opt, dh::HostPlan& hp) {
    dh_status st = validate_config(cfg);
    if (st != DH_OK) return st;
    if (batch && !indptr) return fail(DH_EINVAL, "indptr is NULL");
    if (batch && indptr[batch] > indptr[0] && !indices) return fail(DH_EINVAL, "indices is NULL");
    if (flags & ~DH_PLAN_CASCADE) return fail(DH_EINVAL, "unknown plan flags 0x%x", flags);
    dh::PlanInput in;
    in.batch = batch;
    static const uint32_t zero_ptr[1] = {0};
    in.indptr = batch ? indptr : zero_ptr;
    in.indices = indices;
    in.num_pool_pages = num_pool_pages;
    in.hq = cfg->num_heads;
    in.hkv = cfg->num_kv_heads;
    in.wave_items_only = cfg->q_dtype == DH_DTYPE_F32;
    in.group_rows = uint32_t(dh::group_rows(cfg->kv_format == DH_KV_FP8_E4M3 || cfg->kv_format == DH_KV_MXFP8,
                                            int(cfg->head_dim)));
    in.cascade = (flags & DH_PLAN_CASCADE) != 0;
    if (opt) {
        in.shared_chunk_pages = opt->shared_chunk_pages;
        in.private_chunk_pages = opt->private_chunk_pages;
        in.target_items = opt->target_items;
        if (opt->direct > DH_DIRECT_OFF) return fail(DH_EINVAL, "unknown direct option %u", opt->direct);
        in.direct_ok = opt->direct != DH_DIRECT_OFF;
    }
    std::string err;
    const int rc = dh::build_plan(in, hp, err);
    if (rc != DH_OK) return fail(dh_status(rc), "%s", err.c_str());
    return DH_OK;
}

static void fill_stats(const dh::HostPlan& hp, uint32_t batch, dh_plan_stats* s) {
    memset(s, 0, sizeof *s);
    s->batch_size = batch;
    s->num_segments = hp.num_segments;
    s->num_shared_segments = hp.num_shared_segments;
    s->num_items = uint32_t(hp.items.size());
    s->num_tasks = uint32_t(hp.tasks.size());
    s->num_group_items = hp.num_group_items;
    s->num_partials = hp.num_slots;
    s->direct = hp.direct ? 1u : 0u;
    s->unique_pages = hp.unique_pages;
    s->page_reads = hp.page_reads;
    s->total_pages = hp.total_pages;
}

dh_status dh_plan_inspect(const dh_attn_config* cfg, uint32_t num_pool_pages, const uint32_t* indptr,
                          const uint32_t* indices, uint32_t batch, uint32_t flags,
                          const dh_plan_options* opt, dh_plan_stats* stats, dh_plan_item* items,
                          uint32_t* n_items, uint32_t* pages, uint32_t* n_pages, uint32_t* seqslots,
                          uint32_t* n_seqslots) {
    if (!n_items || !n_pages || !n_seqslots) return fail(DH_EINVAL, "NULL size argument");
    dh::HostPlan hp;
    dh_status st = host_plan(cfg, num_pool_pages, indptr, indices, batch, flags, opt, hp);
    if (st != DH_OK) return st;
    if (stats) fill_stats(hp, batch, stats);
    static_assert(sizeof(dh_plan_item) == sizeof(dh::Item), "item layout");
    static_assert(sizeof(dh::SeqSlot) == 2 * sizeof(uint32_t), "seqslot layout");
    if (items) {
        if (*n_items < hp.items.size()) return fail(DH_EINVAL, "items array too small");
        memcpy(items, hp.items.data(), hp.items.size() * sizeof(dh::Item));
    }
    if (pages) {
        if (*n_pages < hp.pages.size()) return fail(DH_EINVAL, "pages array too small");
        memcpy(pages, hp.pages.data(), hp.pages.size() * sizeof(uint32_t));
    }
    if (seqslots) {
        if (*n_seqslots < hp.seqslots.size()) return fail(DH_EINVAL, "seqslots array too small");
        memcpy(seqslots, hp.seqslots.data(), hp.seqslots.size() * sizeof(dh::SeqSlot));
    }
    *n_items = uint32_t(hp.items.size());
    *n_pages = uint32_t(hp.pages.size());
    *n_seqslots = uint32_t(hp.seqslots.size());
    return DH_OK;
}

// Uploads a host plan: items, pages, seqslots, slot_ptr (and, for prefill,
// per-query token counts and item token ranges) in one device blob.
static dh_status upload_plan(dh_backend* be, const dh_attn_config* cfg, const dh_pool* pool,
                             const dh::HostPlan& hp, uint32_t batch, bool prefill, dh_plan** out) {
    dh_plan* pl = new (std::nothrow) dh_plan();
    if (!pl) return fail(DH_ENOMEM, "out of host memory");
    pl->be = be;
    pl->cfg = *cfg;
    pl->batch = batch;
    pl->pool_pages = pool->num_pages;
    pl->n_items = uint32_t(hp.items.size());
    pl->n_tasks = uint32_t(hp.tasks.size());
    pl->n_group_items = hp.num_group_items;
    pl->n_wave_items = hp.num_wave_items;
    pl->n_slots = hp.num_slots;
    pl->prefill = prefill;
    const size_t o_items = 0;
    const size_t o_pages = align_up(o_items + hp.items.size() * sizeof(dh::Item), 256);
    const size_t o_ss = align_up(o_pages + hp.pages.size() * sizeof(uint32_t), 256);
    const size_t o_sp = align_up(o_ss + hp.seqslots.size() * sizeof(dh::SeqSlot), 256);
    const size_t o_rl = align_up(o_sp + hp.slot_ptr.size() * sizeof(uint32_t), 256);
    const size_t o_il = align_up(o_rl + hp.row_len.size() * sizeof(uint32_t), 256);
    const size_t total = align_up(o_il + hp.item_lim.size() * sizeof(dh::ItemLim), 256);
    std::vector<uint8_t> blob(total, 0);
    memcpy(blob.data() + o_items, hp.items.data(), hp.items.size() * sizeof(dh::Item));
    memcpy(blob.data() + o_pages, hp.pages.data(), hp.pages.size() * sizeof(uint32_t));
    memcpy(blob.data() + o_ss, hp.seqslots.data(), hp.seqslots.size() * sizeof(dh::SeqSlot));
    memcpy(blob.data() + o_sp, hp.slot_ptr.data(), hp.slot_ptr.size() * sizeof(uint32_t));
    if (!hp.row_len.empty()) memcpy(blob.data() + o_rl, hp.row_len.data(), hp.row_len.size() * sizeof(uint32_t));
    if (!hp.item_lim.empty())
        memcpy(blob.data() + o_il, hp.item_lim.data(), hp.item_lim.size() * sizeof(dh::ItemLim));
    dh::DeviceGuard guard(be->device);
    hipError_t e = guard.error();
    if (e == hipSuccess) e = hipMalloc(&pl->dev, total);
    if (e == hipSuccess) e = hipMemcpy(pl->dev, blob.data(), total, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        if (pl->dev) (void)hipFree(pl->dev);
        delete pl;
        return fail(DH_EHIP, "plan upload failed: %s", hipGetErrorString(e));
    }
    pl->items = reinterpret_cast<dh::Item*>(pl->dev + o_items);
    pl->pages = reinterpret_cast<uint32_t*>(pl->dev + o_pages);
    pl->seqslots = reinterpret_cast<dh::SeqSlot*>(pl->dev + o_ss);
    pl->slot_ptr = reinterpret_cast<uint32_t*>(pl->dev + o_sp);
    pl->row_len = prefill ? reinterpret_cast<uint32_t*>(pl->dev + o_rl) : nullptr;
    pl->item_lim = prefill ? reinterpret_cast<dh::ItemLim*>(pl->dev + o_il) : nullptr;
    const size_t rows = size_t(hp.num_slots) * cfg->num_heads;
    // Partial O: fp32 for f32 q, else f16 scaled per row (dh::PartialLse).
    const size_t o_bytes = cfg->q_dtype == DH_DTYPE_F32 ? sizeof(float) : sizeof(uint16_t);
    pl->ws_lse_off = align_up(rows * cfg->head_dim * o_bytes, 256);
    pl->ws_bytes = align_up(pl->ws_lse_off + rows * sizeof(dh::PartialLse), 256);
    fill_stats(hp, batch, &pl->stats);
    if (!prefill) {
        pl->tail_off = hp.tail_off;
        pl->tail_n = hp.tail_n;
        pl->tail_cap = hp.tail_cap;
        pl->tail_item_ptr = hp.tail_item_ptr;
        pl->tail_items = hp.tail_items;
    }
    pl->direct = prefill || hp.direct;
    pl->max_slots = 0;
    for (uint32_t v = 0; v < batch; ++v) pl->max_slots = std::max(pl->max_slots, hp.slot_ptr[v + 1] - hp.slot_ptr[v]);
    pl->uniform_slots = batch ? pl->max_slots : 0;
    for (uint32_t v = 0; v < batch; ++v)
        if (hp.slot_ptr[v + 1] - hp.slot_ptr[v] != pl->max_slots) pl->uniform_slots = 0;
    for (uint32_t v = 0; prefill && v < batch; ++v)
        if (hp.slot_ptr[v + 1] - hp.slot_ptr[v] != 1) pl->direct = false;
    pl->items_word = o_items / sizeof(uint32_t);
    pl->pages_word = o_pages / sizeof(uint32_t);
    retain(be);
    *out = pl;
    return DH_OK;
}

static dh_status check_pool_matches(const dh_attn_config* cfg, const dh_pool* pool) {
    if (pool->hkv != cfg->num_kv_heads || pool->d != cfg->head_dim || pool->fmt != cfg->kv_format)
        return fail(DH_EINVAL, "pool (kv heads %u, head_dim %u, format %u) does not match the config "
                    "(%u, %u, %u)", pool->hkv, pool->d, pool->fmt, cfg->num_kv_heads, cfg->head_dim,
                    cfg->kv_format);
    return DH_OK;
}

dh_status dh_plan_create(dh_backend* be, const dh_attn_config* cfg, const dh_pool* pool,
                         const uint32_t* indptr, const uint32_t* indices, uint32_t batch,
                         uint32_t flags, const dh_plan_options* opt, dh_plan** out) {
    if (!be || !pool || !out || !cfg) return fail(DH_EINVAL, "NULL argument");
    *out = nullptr;
    dh_status st = check_pool_matches(cfg, pool);
    if (st != DH_OK) return st;
    dh::HostPlan hp;
    st = host_plan(cfg, pool->num_pages, indptr, indices, batch, flags, opt, hp);
    if (st != DH_OK) return st;
    return upload_plan(be, cfg, pool, hp, batch, false, out);
}

dh_status dh_plan_create_tree(dh_backend* be, const dh_attn_config* cfg, const dh_pool* pool,
                              const dh_tree* tree, const uint64_t* nodes, uint32_t n, uint32_t flags,
                              const dh_plan_options* opt, dh_plan** out) {
    if (!tree || !out || (n && !nodes)) return fail(DH_EINVAL, "NULL argument");
    *out = nullptr;
    if (dh_tree_tokens_per_block(tree) != DH_PAGE_SIZE)
        return fail(DH_EUNSUPPORTED, "the tree has %u-token blocks; decode pages hold %u tokens",
                    dh_tree_tokens_per_block(tree), DH_PAGE_SIZE);
    std::vector<uint32_t> indptr(1, 0), indices;
    for (uint32_t i = 0; i < n; ++i) {
        uint32_t cnt = 0, got = 0;
        dh_status st = dh_tree_get_block_table(tree, nodes[i], nullptr, 0, &cnt);
        if (st != DH_OK) return st;
        const size_t o = indices.size();
        indices.resize(o + cnt);
        st = dh_tree_get_block_table(tree, nodes[i], indices.data() + o, cnt, &got);
        if (st != DH_OK) return st;
        if (got != cnt) return fail(DH_EINVAL, "node %llu changed while it was read", (unsigned long long)nodes[i]);
        indptr.push_back(uint32_t(indices.size()));
    }
    return dh_plan_create(be, cfg, pool, indptr.data(), indices.empty() ? nullptr : indices.data(), n, flags,
                          opt, out);
}

dh_status dh_tree_last_page_len(const dh_tree* tree, const uint64_t* nodes, uint32_t n, int32_t* out) {
    if (!tree || (n && (!nodes || !out))) return fail(DH_EINVAL, "NULL argument");
    if (dh_tree_tokens_per_block(tree) != DH_PAGE_SIZE)
        return fail(DH_EUNSUPPORTED, "the tree has %u-token blocks; decode pages hold %u tokens",
                    dh_tree_tokens_per_block(tree), DH_PAGE_SIZE);
    for (uint32_t i = 0; i < n; ++i) {
        dh_node_info info;
        const dh_status st = dh_tree_get_node(tree, nodes[i], &info);
        if (st != DH_OK) return st;
        out[i] = int32_t(info.num_tokens % DH_PAGE_SIZE);
    }
    return DH_OK;
}

dh_status dh_plan_create_prefill(dh_backend* be, const dh_attn_config* cfg, const dh_pool* pool,
                                 const uint32_t* indptr, const uint32_t* indices, const uint32_t* kv_len,
                                 const uint32_t* q_len, uint32_t batch, uint32_t causal, uint32_t chunk_pages,
                                 dh_plan** out) {
    if (!be || !pool || !out || !cfg) return fail(DH_EINVAL, "NULL argument");
    *out = nullptr;
    dh_status st = validate_config(cfg);
    if (st != DH_OK) return st;
    st = check_pool_matches(cfg, pool);
    if (st != DH_OK) return st;
    const bool fp8 = cfg->kv_format == DH_KV_FP8_E4M3 || cfg->kv_format == DH_KV_MXFP8;
    if (cfg->q_dtype == DH_DTYPE_F32 || (fp8 && cfg->head_dim == 64))
        return fail(DH_EUNSUPPORTED, "prefill takes bf16 / f16 queries over 16-bit KV, and over FP8 / MXFP8 KV "
                    "at head_dim 128 or 256");
    if (batch && (!indptr || !kv_len || !q_len)) return fail(DH_EINVAL, "NULL argument");
    if (batch && indptr[batch] > indptr[0] && !indices) return fail(DH_EINVAL, "indices is NULL");
    dh::PrefillInput in;
    in.batch = batch;
    static const uint32_t zero_ptr[1] = {0};
    in.indptr = batch ? indptr : zero_ptr;
    in.indices = indices;
    in.kv_len = kv_len;
    in.q_len = q_len;
    in.num_pool_pages = pool->num_pages;
    in.hq = cfg->num_heads;
    in.hkv = cfg->num_kv_heads;
    in.group_rows = uint32_t(dh::group_rows(false, int(cfg->head_dim)));
    in.causal = causal != 0;
    in.chunk_pages = chunk_pages;
    dh::HostPlan hp;
    std::string err;
    const int rc = dh::build_prefill_plan(in, hp, err);
    if (rc != DH_OK) return fail(dh_status(rc), "%s", err.c_str());
    return upload_plan(be, cfg, pool, hp, uint32_t(hp.row_len.size()), true, out);
}

dh_status dh_plan_update(dh_plan* pl, uint32_t n, const uint32_t* seqs, const uint32_t* ops,
                         const uint32_t* page_ids, void* stream, uint32_t* patched) {
    static_assert(sizeof(dh::Item) == 8 * sizeof(uint32_t) && offsetof(dh::Item, npages) == sizeof(uint32_t),
                  "Item.npages is word 1 of 8");
    if (!pl || !patched) return fail(DH_EINVAL, "NULL argument");
    *patched = 0;
    if (pl->prefill) return fail(DH_EUNSUPPORTED, "prefill plans are not updated in place");
    if (n && (!seqs || !ops || !page_ids)) return fail(DH_EINVAL, "NULL argument");
    // Validate every event and check that all fit before changing anything.
    std::vector<std::pair<uint32_t, uint32_t>> count;   // (sequence, pages in its last chunk)
    auto find = [&](uint32_t b) -> uint32_t& {
        for (auto& c : count)
            if (c.first == b) return c.second;
        count.emplace_back(b, pl->tail_n[b]);
        return count.back().second;
    };
    bool fits = true;
    uint32_t appended = 0;
    for (uint32_t k = 0; k < n; ++k) {
        if (seqs[k] >= pl->batch)
            return fail(DH_EINVAL, "event %u: sequence %u outside the plan's batch of %u", k, seqs[k], pl->batch);
        if (ops[k] != DH_PLAN_APPEND && ops[k] != DH_PLAN_REPLACE_LAST)
            return fail(DH_EINVAL, "event %u: unknown op %u", k, ops[k]);
        if (page_ids[k] >= pl->pool_pages)
            return fail(DH_EINVAL, "event %u: page id %u outside the pool of %u pages", k, page_ids[k],
                        pl->pool_pages);
        uint32_t& c = find(seqs[k]);
        if (c == 0) fits = false;                       // no pages: no chunk to patch
        else if (ops[k] == DH_PLAN_APPEND) {
            if (c == pl->tail_cap[seqs[k]]) fits = false;
            else ++c, ++appended;
        }
    }
    if (!fits) return DH_OK;
    // The words to write: page ids in event order, then each changed chunk's
    // page count in every item of it.
    std::vector<uint32_t> idx, val;
    for (auto& c : count) c.second = pl->tail_n[c.first];
    for (uint32_t k = 0; k < n; ++k) {
        const uint32_t b = seqs[k];
        uint32_t& c = find(b);
        if (ops[k] == DH_PLAN_APPEND) ++c;
        idx.push_back(uint32_t(pl->pages_word + pl->tail_off[b] + c - 1));
        val.push_back(page_ids[k]);
    }
    for (const auto& c : count) {
        if (c.second == pl->tail_n[c.first]) continue;
        for (uint32_t t = pl->tail_item_ptr[c.first]; t < pl->tail_item_ptr[c.first + 1]; ++t) {
            idx.push_back(uint32_t(pl->items_word + size_t(pl->tail_items[t]) * 8 + 1));
            val.push_back(c.second);
        }
    }
    {
        dh::DeviceGuard guard(pl->be->device);
        hipError_t e = guard.error();
        for (size_t o = 0; e == hipSuccess && o < idx.size(); o += dh::kPatchWords) {
            const uint32_t m = uint32_t(std::min<size_t>(dh::kPatchWords, idx.size() - o));
            e = hipError_t(dh::launch_plan_patch(reinterpret_cast<uint32_t*>(pl->dev), m, idx.data() + o,
                                                 val.data() + o, stream));
        }
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return fail(DH_EHIP, "plan update failed: %s", hipGetErrorString(e));
        }
    }
    for (const auto& c : count) pl->tail_n[c.first] = c.second;
    pl->stats.total_pages += appended;
    pl->stats.page_reads += appended;
    pl->stats.unique_pages += appended;   // a new block is read by its sequence alone
    *patched = 1;
    return DH_OK;
}

dh_status dh_plan_destroy(dh_plan* pl) {
    if (!pl) return DH_OK;
    {
        dh::DeviceGuard g(pl->be->device);
        (void)hipDeviceSynchronize();
        (void)hipFree(pl->dev);
        (void)hipGetLastError();
    }
    release(pl->be);
    delete pl;
    return DH_OK;
}

size_t dh_plan_workspace_size(const dh_plan* pl) { return pl ? pl->ws_bytes : 0; }

dh_status dh_plan_get_stats(const dh_plan* pl, dh_plan_stats* st) {
    if (!pl || !st) return fail(DH_EINVAL, "NULL argument");
    *st = pl->stats;
    return DH_OK;
}

/* ------------------------------------------------------------------ decode */

// The decode kernels dereference q, out, the workspace and last_page_len on
// the device; a pageable host pointer there would fault the GPU, so each is
// checked against the runtime's allocation records.  Each thread remembers
// the address ranges of the last few allocations it accepted, so a pointer
// inside one of them costs no runtime query.  Such a range is not dropped
// when its allocation is freed: device allocations come from the runtime's
// own reserved address range, which host mappings do not reuse, and a freed
// range that is reallocated is device memory again.
static dh_status check_device_ptr(const void* p, const char* what) {
    struct Range {
        uintptr_t lo = 0, hi = 0;
    };
    thread_local Range seen[8];
    thread_local unsigned next = 0;
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    for (const Range& r : seen)
        if (a >= r.lo && a < r.hi) return DH_OK;
    hipPointerAttribute_t attr;
    hipError_t e = hipPointerGetAttributes(&attr, p);
    if (e != hipSuccess || attr.type == hipMemoryTypeUnregistered) {
        (void)hipGetLastError();
        return fail(DH_EINVAL, "%s is not GPU-accessible memory (copy a host array to the device first)", what);
    }
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    e = hipMemGetAddressRange(&base, &size, const_cast<void*>(p));
    Range r;
    if (e == hipSuccess && base && size) {
        r.lo = reinterpret_cast<uintptr_t>(base);
        r.hi = r.lo + size;
    } else {   // accepted, but only this address is remembered
        (void)hipGetLastError();
        r.lo = a;
        r.hi = a + 1;
    }
    seen[next++ % 8] = r;
    return DH_OK;
}

// ws_static: ws is the backend's static scratch (device memory by
// construction; the runtime does not track module globals as allocations).
// host_lens: last-page lengths in host memory (dh_decode_batch_host_lens),
// packed into the kernel arguments; last_page_len is then null.
static dh_status decode_impl(dh_backend* be, const dh_pool* pool, const dh_plan* pl, const void* q,
                             const int32_t* last_page_len, void* out, void* ws, size_t ws_bytes, uint32_t mask,
                             void* stream, bool ws_static, const int32_t* host_lens = nullptr) {
    if (!be || !pool || !pl) return fail(DH_EINVAL, "NULL argument");
    if (pl->be != be || pool->be != be) return fail(DH_EINVAL, "plan/pool belong to another backend");
    if (pool->num_pages != pl->pool_pages || pool->hkv != pl->cfg.num_kv_heads ||
        pool->d != pl->cfg.head_dim || pool->fmt != pl->cfg.kv_format)
        return fail(DH_EINVAL, "pool does not match the plan");
    if (pl->batch == 0) return DH_OK;
    if (!q || !out) return fail(DH_EINVAL, "q and out must be device pointers");
    if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(out)) & 15)
        return fail(DH_EINVAL, "q and out must be 16-byte aligned");
    if (ws_bytes < pl->ws_bytes || (pl->ws_bytes && !ws))
        return fail(DH_EINVAL, "workspace of %zu bytes is smaller than the %zu bytes the plan needs",
                    ws_bytes, pl->ws_bytes);
    if (reinterpret_cast<uintptr_t>(ws) & 255) return fail(DH_EINVAL, "workspace must be 256-byte aligned");
    DH_DEVICE(be->device);
    for (const auto& [ptr, what] : {std::pair<const void*, const char*>{q, "q"}, {out, "out"},
                                    {pl->ws_bytes && !ws_static ? ws : nullptr, "workspace"},
                                    {last_page_len, "last_page_len"}}) {
        if (!ptr) continue;
        const dh_status st = check_device_ptr(ptr, what);
        if (st != DH_OK) return st;
    }
    const dh_attn_config& c = pl->cfg;
    // Group items address query rows by 32-bit byte offsets into q.
    if (uint64_t(pl->batch) * c.num_heads * c.head_dim * (c.q_dtype == DH_DTYPE_F32 ? 4u : 2u) > 0xFFFFFFFFull)
        return fail(DH_EUNSUPPORTED, "q of %u x %u x %u exceeds 4 GiB", pl->batch, c.num_heads, c.head_dim);
    void* ws_o = ws;
    dh::PartialLse* ws_lse = reinterpret_cast<dh::PartialLse*>(static_cast<uint8_t*>(ws) + pl->ws_lse_off);
    if (mask & 1u) {
        dh::AttendArgs a{};
        a.items = pl->items;
        a.pages = pl->pages;
        a.seqslots = pl->seqslots;
        a.q = q;
        a.kv = pool->data;
        a.scales = pool->scales;
        a.last_page_len = last_page_len;
        if (host_lens) {
            // 4 bits a sequence; 16 and every value outside 1..15 pack as
            // 0, which the kernels read as a full page (as they read the
            // device array's out-of-range values).
            a.lpl_inline = 1u;
            for (uint32_t b = 0; b < pl->batch; ++b) {
                const int32_t v = host_lens[b];
                const uint32_t nib = v >= 1 && v < int32_t(DH_PAGE_SIZE) ? uint32_t(v) : 0u;
                a.lpl_nib[b >> 3] |= nib << (4 * (b & 7));
            }
        }
        a.ws_o = ws_o;
        a.ws_lse = ws_lse;
        a.hq = c.num_heads;
        a.hkv = c.num_kv_heads;
        a.r = c.num_heads / c.num_kv_heads;
        a.gqa_tiled = c.gqa_mapping == DH_GQA_TILED ? 1u : 0u;
        // A negative scale goes into the query's sign; zero becomes 2^-60
        // (scores * 2^-60 round to 0 in exp2, and a masked -inf stays -inf).
        const float sl = c.scale * 1.4426950408889634f;
        a.scale_log2 = std::max(fabsf(sl), 0x1p-60f);
        a.q_sign = sl < 0.f ? (c.q_dtype == DH_DTYPE_F32 ? 0x80000000u : 0x80008000u) : 0u;
        a.n_group_items = pl->n_group_items;
        a.n_wave_items = pl->n_wave_items;
        a.row_len = pl->row_len;
        a.item_lim = pl->item_lim;
        a.out_direct = pl->direct && pl->prefill ? out : nullptr;
        a.page_limit = pool->num_pages;
        if (pl->direct && !pl->prefill) {   // direct decode plan: wave tasks merge their own rows
            a.wave_direct = 1u;
            a.slot_ptr = pl->slot_ptr;
            a.out = out;
        }
        hipError_t e = hipError_t(dh::launch_attend(a, pl->n_tasks, c.q_dtype, c.kv_format, c.head_dim,
                                                    pl->prefill, stream));
        if (e != hipSuccess) return fail(DH_EHIP, "attention launch failed: %s", hipGetErrorString(e));
    }
    if ((mask & 2u) && !pl->direct) {
        dh::MergeArgs m{};
        m.slot_ptr = pl->slot_ptr;
        m.ws_o = ws_o;
        m.ws_lse = ws_lse;
        m.out = out;
        m.batch = pl->batch;
        m.hq = c.num_heads;
        m.max_states = pl->max_slots;
        m.uniform_slots = pl->uniform_slots;
        hipError_t e = hipError_t(dh::launch_merge(m, c.q_dtype, c.head_dim, stream));
        if (e != hipSuccess) return fail(DH_EHIP, "merge launch failed: %s", hipGetErrorString(e));
    }
    return DH_OK;
}

dh_status dh_decode_stages(dh_backend* be, const dh_pool* pool, const dh_plan* pl, const void* q,
                           const int32_t* last_page_len, void* out, void* ws, size_t ws_bytes,
                           uint32_t mask, void* stream) {
    return decode_impl(be, pool, pl, q, last_page_len, out, ws, ws_bytes, mask, stream, false);
}

dh_status dh_decode_batch(dh_backend* be, const dh_pool* pool, const dh_plan* pl, const void* q,
                          const int32_t* last_page_len, void* out, void* ws, size_t ws_bytes,
                          void* stream) {
    return decode_impl(be, pool, pl, q, last_page_len, out, ws, ws_bytes, 3u, stream, false);
}

dh_status dh_decode_batch_host_lens(dh_backend* be, const dh_pool* pool, const dh_plan* pl, const void* q,
                                    const int32_t* last_page_len_host, void* out, void* ws, size_t ws_bytes,
                                    void* stream) {
    if (!pl) return fail(DH_EINVAL, "NULL argument");
    if (pl->batch > DH_HOST_LENS_MAX_BATCH)
        return fail(DH_EUNSUPPORTED, "%u sequences: host last-page lengths take at most %u (use dh_decode_batch)",
                    pl->batch, DH_HOST_LENS_MAX_BATCH);
    return decode_impl(be, pool, pl, q, nullptr, out, ws, ws_bytes, 3u, stream, false, last_page_len_host);
}

dh_status dh_decode_batch_static(dh_backend* be, const dh_pool* pool, const dh_plan* pl, const void* q,
                                 const int32_t* last_page_len, void* out, void* stream) {
    if (!be || !pl) return fail(DH_EINVAL, "NULL argument");
    if (pl->ws_bytes > DH_STATIC_WORKSPACE_BYTES)
        return fail(DH_ENOMEM, "the plan needs %zu bytes of partial states; the static scratch holds %zu "
                    "(use dh_decode_batch with a workspace)", pl->ws_bytes, size_t(DH_STATIC_WORKSPACE_BYTES));
    return decode_impl(be, pool, pl, q, last_page_len, out, be->scratch, DH_STATIC_WORKSPACE_BYTES, 3u, stream,
                       true);
}

/* ------------------------------------------------- decode from device CSR */

namespace {

// Whether a CSR call looks for shared prefixes (group items need 16-bit
// queries; the common-prefix pass keeps one LDS entry per sequence).
bool csr_cascade(const dh_attn_config& c, uint32_t batch) {
    return c.q_dtype != DH_DTYPE_F32 && batch >= 2 && batch <= dh::kCsrCascadeMaxBatch;
}

uint32_t csr_group_rows(const dh_attn_config& c) {
    const bool fp8 = c.kv_format == DH_KV_FP8_E4M3 || c.kv_format == DH_KV_MXFP8;
    return uint32_t(dh::group_rows(fp8, int(c.head_dim)));
}

// Group items a CSR call may emit: the planning kernel keeps them near 256
// (one per CU) by its chunk choice, up to 32 chunks of 256 pages per group
// and KV head (DH_MAX_SEQ_LEN); bounded by kCsrMaxGroupItems.
uint32_t csr_group_cap(const dh_attn_config& c, uint32_t batch) {
    if (!csr_cascade(c, batch)) return 0;
    const uint64_t r = c.num_heads / c.num_kv_heads, gr = csr_group_rows(c);
    const uint64_t cap = 256 + 32ull * c.num_kv_heads * ((uint64_t(batch) * r + gr - 1) / gr);
    return uint32_t(std::min<uint64_t>(cap, dh::kCsrMaxGroupItems));
}

// Workspace of dh_decode_csr for `slots` partial-state slots, each section
// 256-byte aligned: header, slot_ptr[B+1], seq_bad[B], seqslots[slots],
// partial O [slots][Hq][D] (fp32 for f32 queries, else f16), log-sum-exps;
// with a cascade also the common-prefix slices [B][kCsrLcpSlices], the skip
// words [B] and the group items [gcap].
struct CsrLayout {
    size_t hdr, slot_ptr, seq_bad, seqslots, ws_o, ws_lse, lcp, skip, gitems, total;
};

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

CsrLayout csr_layout(const dh_attn_config& c, uint32_t batch, uint64_t slots) {
    CsrLayout l;
    const size_t eb = c.q_dtype == DH_DTYPE_F32 ? 4 : 2;
    const bool casc = csr_cascade(c, batch);
    l.hdr = 0;
    l.slot_ptr = align256(sizeof(dh::CsrHeader));
    l.seq_bad = l.slot_ptr + align256(size_t(batch + 1) * 4);
    l.seqslots = l.seq_bad + align256(size_t(batch) * 4);
    l.ws_o = l.seqslots + align256(slots * sizeof(dh::SeqSlot));
    l.ws_lse = l.ws_o + align256(slots * c.num_heads * c.head_dim * eb);
    l.lcp = l.ws_lse + align256(slots * c.num_heads * sizeof(dh::PartialLse));
    l.skip = l.lcp + (casc ? align256(size_t(batch) * dh::kCsrLcpSlices * 4) : 0);
    l.gitems = l.skip + (casc ? align256(size_t(batch) * 4) : 0);
    l.total = l.gitems + align256(size_t(csr_group_cap(c, batch)) * sizeof(dh::Item));
    return l;
}

uint32_t csr_row_blocks(const dh_attn_config& c) {
    const uint32_t r = c.num_heads / c.num_kv_heads;
    return (r + dh::kWaveRows - 1) / dh::kWaveRows;
}

// Slots beyond the batch's own that a call uses at most (its grid covers
// them; a larger workspace is not used past this).
constexpr uint64_t kCsrMaxExtraSlots = 4096, kCsrMaxCascadeSlots = 8192;
constexpr uint32_t kCsrMaxBatch = 65536;

}  // namespace

size_t dh_csr_workspace_size(const dh_attn_config* cfg, uint32_t batch, uint32_t max_total_pages) {
    if (!cfg || cfg->num_kv_heads == 0 || cfg->num_heads == 0 || batch == 0) return 0;
    const uint64_t per = uint64_t(cfg->num_kv_heads) * csr_row_blocks(*cfg);
    const uint64_t t = max_total_pages;
    // Room for chunks that give up to two waves per wave slot, and for the
    // largest chunks whatever the batch.
    const uint64_t need = (t + dh::kCsrMaxChunk - 1) / dh::kCsrMaxChunk;
    const uint64_t par = std::min((t + dh::kCsrMinChunk - 1) / dh::kCsrMinChunk,
                                  (2 * uint64_t(dh::kCsrWaveSlots) + per - 1) / per);
    uint64_t extra = std::min(kCsrMaxExtraSlots, std::max<uint64_t>(1, std::max(need, par)));
    // A cascade's group chunks take one slot per member: at most one per 8
    // shared pages of each sequence, plus one per sequence for rounding.
    if (csr_cascade(*cfg, batch)) extra += std::min(kCsrMaxCascadeSlots, (t + 7) / 8 + batch);
    return csr_layout(*cfg, batch, uint64_t(batch) + extra).total;
}

dh_status dh_decode_csr(dh_backend* be, const dh_pool* pool, const dh_attn_config* cfg, uint32_t batch,
                        const void* q, const int32_t* indices, const int32_t* indptr,
                        const int32_t* last_page_len, void* out, void* ws, size_t ws_bytes, int32_t* status,
                        void* stream) {
    if (!be || !pool || !cfg) return fail(DH_EINVAL, "NULL argument");
    dh_status st = validate_config(cfg);
    if (st != DH_OK) return st;
    st = check_pool_matches(cfg, pool);
    if (st != DH_OK) return st;
    if (batch == 0) return DH_OK;
    if (batch > kCsrMaxBatch) return fail(DH_EINVAL, "batch_size %u exceeds %u", batch, kCsrMaxBatch);
    if (!q || !out || !indptr || !indices || !ws)
        return fail(DH_EINVAL, "q, out, indices, indptr and workspace must be device pointers");
    if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(out)) & 15)
        return fail(DH_EINVAL, "q and out must be 16-byte aligned");
    if (reinterpret_cast<uintptr_t>(ws) & 255) return fail(DH_EINVAL, "workspace must be 256-byte aligned");
    if ((reinterpret_cast<uintptr_t>(indptr) | reinterpret_cast<uintptr_t>(indices) |
         reinterpret_cast<uintptr_t>(last_page_len) | reinterpret_cast<uintptr_t>(status)) & 3)
        return fail(DH_EINVAL, "indices, indptr, last_page_len and status must be 4-byte aligned");
    const dh_attn_config& c = *cfg;
    if (uint64_t(batch) * c.num_heads * c.head_dim * (c.q_dtype == DH_DTYPE_F32 ? 4u : 2u) > 0xFFFFFFFFull)
        return fail(DH_EUNSUPPORTED, "q of %u x %u x %u exceeds 4 GiB", batch, c.num_heads, c.head_dim);
    // Slots the workspace holds (at most kCsrMaxExtraSlots past the batch).
    const CsrLayout one = csr_layout(c, batch, 1);
    const size_t per_slot = sizeof(dh::SeqSlot) + size_t(c.num_heads) * sizeof(dh::PartialLse) +
                            size_t(c.num_heads) * c.head_dim * (c.q_dtype == DH_DTYPE_F32 ? 4 : 2);
    uint64_t slots = ws_bytes > one.total ? 1 + (ws_bytes - one.total) / per_slot : 0;
    const uint64_t cap = uint64_t(batch) + kCsrMaxExtraSlots + (csr_cascade(c, batch) ? kCsrMaxCascadeSlots : 0);
    slots = std::min(slots, cap);
    // The estimate ignores the sections' alignment: settle on the exact count.
    while (slots < cap && csr_layout(c, batch, slots + 1).total <= ws_bytes) ++slots;
    while (slots > 0 && csr_layout(c, batch, slots).total > ws_bytes) --slots;
    if (slots <= batch)
        return fail(DH_EINVAL, "workspace of %zu bytes holds %llu chunk slots; a batch of %u needs more than %u "
                    "(dh_csr_workspace_size)", ws_bytes, (unsigned long long)slots, batch, batch);
    DH_DEVICE(be->device);
    for (const auto& [ptr, what] : {std::pair<const void*, const char*>{q, "q"}, {out, "out"}, {ws, "workspace"},
                                    {indptr, "indptr"}, {indices, "indices"}, {last_page_len, "last_page_len"},
                                    {status, "status"}}) {
        if (!ptr) continue;
        st = check_device_ptr(ptr, what);
        if (st != DH_OK) return st;
    }
    const CsrLayout l = csr_layout(c, batch, slots);
    uint8_t* w = static_cast<uint8_t*>(ws);
    auto* hdr = reinterpret_cast<dh::CsrHeader*>(w + l.hdr);
    auto* slot_ptr = reinterpret_cast<uint32_t*>(w + l.slot_ptr);
    auto* seq_bad = reinterpret_cast<uint32_t*>(w + l.seq_bad);
    auto* seqslots = reinterpret_cast<dh::SeqSlot*>(w + l.seqslots);
    auto* ws_lse = reinterpret_cast<dh::PartialLse*>(w + l.ws_lse);
    const uint32_t nrb = csr_row_blocks(c);
    const uint32_t per_chunk = c.num_kv_heads * nrb;

    const bool casc = csr_cascade(c, batch);
    const uint32_t gcap = csr_group_cap(c, batch);
    auto* lcp = reinterpret_cast<uint32_t*>(w + l.lcp);
    auto* skip = reinterpret_cast<uint32_t*>(w + l.skip);
    auto* gitems = reinterpret_cast<dh::Item*>(w + l.gitems);
    hipError_t e = hipSuccess;
    if (casc) {
        e = hipError_t(dh::launch_csr_lcp(indptr, indices, batch, pool->num_pages, lcp, stream));
        if (e != hipSuccess) return fail(DH_EHIP, "CSR common-prefix launch failed: %s", hipGetErrorString(e));
    }
    dh::CsrPlanArgs p{};
    p.indptr = indptr;
    p.batch = batch;
    p.per_chunk = per_chunk;
    p.slot_cap = uint32_t(slots);
    p.hdr = hdr;
    p.slot_ptr = slot_ptr;
    p.seq_bad = seq_bad;
    p.seqslots = seqslots;
    p.lcp = casc ? lcp : nullptr;
    p.skip = skip;
    p.gitems = gitems;
    p.gcap = gcap;
    p.hkv = c.num_kv_heads;
    p.r = c.num_heads / c.num_kv_heads;
    p.group_rows = csr_group_rows(c);
    e = hipError_t(dh::launch_csr_plan(p, stream));
    if (e != hipSuccess) return fail(DH_EHIP, "CSR planning launch failed: %s", hipGetErrorString(e));

    dh::AttendArgs a{};
    a.items = gitems;
    a.csr_skip = casc ? skip : nullptr;
    a.pages = reinterpret_cast<const uint32_t*>(indices);
    a.seqslots = seqslots;
    a.q = q;
    a.kv = pool->data;
    a.scales = pool->scales;
    a.last_page_len = last_page_len;
    a.ws_o = w + l.ws_o;
    a.ws_lse = ws_lse;
    a.hq = c.num_heads;
    a.hkv = c.num_kv_heads;
    a.r = c.num_heads / c.num_kv_heads;
    a.gqa_tiled = c.gqa_mapping == DH_GQA_TILED ? 1u : 0u;
    const float sl = c.scale * 1.4426950408889634f;
    a.scale_log2 = std::max(fabsf(sl), 0x1p-60f);
    a.q_sign = sl < 0.f ? (c.q_dtype == DH_DTYPE_F32 ? 0x80000000u : 0x80008000u) : 0u;
    a.page_limit = pool->num_pages;
    a.csr_indptr = indptr;
    a.csr_slot_ptr = slot_ptr;
    a.csr_hdr = reinterpret_cast<const uint32_t*>(hdr);
    a.seq_bad = seq_bad;
    a.csr_nrb = nrb;
    // The group items the planning kernel writes (at most gcap) take the
    // first workgroups; then one wave per wave item, four per workgroup,
    // over every slot the workspace holds.  Workgroups past the call's
    // items exit at once.
    const uint64_t waves = slots * per_chunk;
    e = hipError_t(dh::launch_attend(a, uint32_t(gcap + (waves + dh::kWaves - 1) / dh::kWaves), c.q_dtype,
                                     c.kv_format, c.head_dim, false, stream));
    if (e != hipSuccess) return fail(DH_EHIP, "attention launch failed: %s", hipGetErrorString(e));

    dh::MergeArgs m{};
    m.slot_ptr = slot_ptr;
    m.ws_o = w + l.ws_o;
    m.ws_lse = ws_lse;
    m.out = out;
    m.batch = batch;
    m.hq = c.num_heads;
    m.seq_bad = seq_bad;
    m.csr_hdr = hdr;
    m.status = status;
    m.max_states = 0;   // chunks per sequence are chosen on the device
    e = hipError_t(dh::launch_merge(m, c.q_dtype, c.head_dim, stream));
    if (e != hipSuccess) return fail(DH_EHIP, "merge launch failed: %s", hipGetErrorString(e));
    return DH_OK;
}

/* ------------------------------------------------------------------- merge */

dh_status dh_merge_states(const float* o_a, const float* lse_a, const float* o_b, const float* lse_b,
                          float* o_out, float* lse_out, uint32_t n_rows, uint32_t d, void* stream) {
    if (n_rows == 0) return DH_OK;
    if (!o_a || !lse_a || !o_b || !lse_b || !o_out || !lse_out) return fail(DH_EINVAL, "NULL argument");
    if (d == 0 || d > 1024) return fail(DH_EINVAL, "head_dim %u out of range", d);
    hipError_t e = hipError_t(dh::launch_merge_states(o_a, lse_a, o_b, lse_b, o_out, lse_out, n_rows, d, stream));
    if (e != hipSuccess) return fail(DH_EHIP, "merge launch failed: %s", hipGetErrorString(e));
    return DH_OK;
}

/* ------------------------------------------------------------------ gather */

dh_status dh_gather_debug(const dh_pool* pool, const uint32_t* ids, uint32_t n, uint32_t kv_head,
                          void* out, uint32_t* n_out, void* stream) {
    if (!pool || !out || !n_out || (n && !ids)) return fail(DH_EINVAL, "NULL argument");
    if (kv_head >= pool->hkv) return fail(DH_EINVAL, "kv head %u out of range", kv_head);
    std::vector<uint32_t> sel;
    sel.reserve(n);
    for (uint32_t i = 0; i < n; ++i) {
        if (ids[i] == DH_INVALID_PAGE) continue;
        if (ids[i] >= pool->num_pages) return fail(DH_EINVAL, "page id %u outside the pool", ids[i]);
        sel.push_back(ids[i]);
    }
    *n_out = uint32_t(sel.size());
    if (sel.empty()) return DH_OK;
    DH_DEVICE(pool->be->device);
    uint32_t* d_ids = nullptr;
    DH_HIP(hipMalloc(&d_ids, sel.size() * sizeof(uint32_t)));
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    hipError_t e = hipMemcpyAsync(d_ids, sel.data(), sel.size() * sizeof(uint32_t), hipMemcpyHostToDevice, s);
    if (e == hipSuccess)
        e = hipError_t(dh::launch_gather(pool->data, d_ids, uint32_t(sel.size()), kv_head, pool->hkv, pool->d,
                                         pool->eb, static_cast<uint8_t*>(out), s));
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    (void)hipFree(d_ids);
    if (e != hipSuccess) return fail(DH_EHIP, "gather failed: %s", hipGetErrorString(e));
    return DH_OK;
}

dh_status dh_debug_e4m3_to_bf16(int device, const uint8_t* codes, const uint8_t* e8m0, uint32_t n,
                                uint16_t* out) {
    if (n % 4) return fail(DH_EINVAL, "n must be a multiple of 4");
    if (n == 0) return DH_OK;
    if (!codes || !e8m0 || !out) return fail(DH_EINVAL, "NULL argument");
    DH_DEVICE(device);
    uint8_t* buf = nullptr;
    const size_t nb = size_t(n) + n / 4 + size_t(n) * 2;
    DH_HIP(hipMalloc(&buf, nb));
    hipError_t e = hipMemcpy(buf, codes, n, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(buf + n, e8m0, n / 4, hipMemcpyHostToDevice);
    uint32_t* dout = reinterpret_cast<uint32_t*>(buf + ((size_t(n) + n / 4 + 3) / 4) * 4);
    if (e == hipSuccess)
        e = hipError_t(dh::launch_e4m3_debug(reinterpret_cast<const uint32_t*>(buf), buf + n, n / 4, dout, nullptr));
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(out, dout, size_t(n) * 2, hipMemcpyDeviceToHost);
    (void)hipFree(buf);
    if (e != hipSuccess) return fail(DH_EHIP, "debug conversion failed: %s", hipGetErrorString(e));
    return DH_OK;
}

}  // extern "C"
