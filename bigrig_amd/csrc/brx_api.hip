// The C-ABI of libbrx: validation, the HBM slot pool, the workspace and kernel dispatch.
// Host-side state only; the kernels live in k_*.hip.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <string>

#include "brx_internal.h"

using namespace brx;

namespace {

thread_local std::string g_err;
int g_device = -1;

struct Workspace {
    void* ptr = nullptr;
    size_t bytes = 0;
    int device = -1;
};
Workspace g_ws;
std::mutex g_ws_mu;

// Scratch of brx_moe_block_forward_noalloc: a file-scope device array (one copy per GPU, held
// until the process ends). Host code never uses the array's name as an address: brx_init looks
// up each device's copy with hipGetSymbolAddress and keeps that pointer.
constexpr int kMaxDevices = 64;
static __device__ __align__(256) uint8_t scratch[BRX_NOALLOC_SCRATCH_BYTES];
void* g_scratch_ptr[kMaxDevices] = {};

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(BRX_EHIP, "%s: %s", what, hipGetErrorString(e));
}

#define HIP_TRY(expr)                                   \
    do {                                                \
        hipError_t _e = (expr);                         \
        if (_e != hipSuccess) return hip_fail(_e, #expr); \
    } while (0)

int check_desc(const brx_layer_desc* d) {
    if (!d) return fail(BRX_EINVAL, "layer descriptor is NULL");
    if (d->hidden <= 0 || d->hidden % 64)
        return fail(BRX_EINVAL, "hidden %d must be a positive multiple of 64", d->hidden);
    if (d->inter <= 0 || d->inter % 64)
        return fail(BRX_EINVAL, "inter %d must be a positive multiple of 64", d->inter);
    // the decode kernels stage 8 token rows of x (and h rows) in LDS and split a weight row over
    // at most 256 lanes x 4 units; the router loops over any width (its LDS token tiles serve
    // widths up to 5120, wider layers take its register path)
    if (d->hidden > kMaxWidth || d->inter > kMaxWidth || d->shared_inter > kMaxWidth)
        return fail(BRX_EINVAL, "hidden %d, inter %d and shared_inter %d must be at most %d", d->hidden,
                    d->inter, d->shared_inter, kMaxWidth);
    if (d->n_experts < 1 || d->n_experts > 512)
        return fail(BRX_EINVAL, "n_experts %d outside [1, 512]", d->n_experts);
    if (d->top_k < 1 || d->top_k > d->n_experts || d->top_k > 64)
        return fail(BRX_EINVAL, "top_k %d outside [1, min(n_experts, 64)]", d->top_k);
    if (d->quant_mode == BRX_QUANT_AFFINE) {
        // the reference's per-layer precision candidates (bigrig_engine/precision.py:58): 2, 3 and
        // 4 bits in groups of 64 or 128, 6 and 8 bits in groups of 64 (MLX also writes 6- and 8-bit
        // g128, which the kernels take as well)
        if (kernel_mode(BRX_QUANT_AFFINE, d->bits) < 0 || (d->group_size != 64 && d->group_size != 128))
            return fail(BRX_EINVAL, "affine kernels take 2-, 3-, 4-, 6- or 8-bit weights in groups of 64 or 128 "
                        "(got %d-bit g%d)", d->bits, d->group_size);
        if (d->hidden % d->group_size || d->inter % d->group_size || d->shared_inter % d->group_size)
            return fail(BRX_EINVAL, "hidden %d, inter %d and shared_inter %d must be multiples of the group size %d",
                        d->hidden, d->inter, d->shared_inter, d->group_size);
        if (d->scale_dtype != BRX_SCALE_BF16 && d->scale_dtype != BRX_SCALE_F16)
            return fail(BRX_EINVAL, "scale_dtype %d unknown", d->scale_dtype);
    } else if (d->quant_mode == BRX_QUANT_MXFP4) {
        if (d->bits != 4 || d->group_size != 32)
            return fail(BRX_EINVAL, "mxfp4 is 4-bit in groups of 32 (got %d-bit g%d)", d->bits,
                        d->group_size);
    } else if (d->quant_mode == BRX_QUANT_NONE) {
        // unquantized experts: bf16 weights with no scales (the mx.gather_mm branch,
        // bigrig_engine/stream.py:1626-1628)
        if (d->bits != 16 || d->group_size != 0)
            return fail(BRX_EINVAL, "unquantized experts are bf16: bits 16, group_size 0 (got %d-bit g%d)",
                        d->bits, d->group_size);
    } else {
        return fail(BRX_EINVAL, "quant_mode %d unknown", d->quant_mode);
    }
    if (d->act != BRX_ACT_SWIGLU && d->act != BRX_ACT_SWIGLU_CLAMPED && d->act != BRX_ACT_SILU_MLP)
        return fail(BRX_EINVAL, "act %d unknown", d->act);
    if (d->route_mode < 0 || d->route_mode > BRX_ROUTE_SIGMOID_TOPK_RENORM)
        return fail(BRX_EINVAL, "route_mode %d unknown", d->route_mode);
    if (d->n_group < 0 || d->n_group > 64)
        return fail(BRX_EINVAL, "n_group %d outside [0, 64]", d->n_group);
    if (d->n_group > 1) {
        if (d->n_experts % d->n_group)
            return fail(BRX_EINVAL, "n_group %d does not divide n_experts %d", d->n_group, d->n_experts);
        if (d->topk_group < 1 || d->topk_group > d->n_group)
            return fail(BRX_EINVAL, "topk_group %d outside [1, n_group %d]", d->topk_group, d->n_group);
        if (d->top_k > d->topk_group * (d->n_experts / d->n_group))
            return fail(BRX_EINVAL, "top_k %d exceeds the %d experts of topk_group %d groups", d->top_k,
                        d->topk_group * (d->n_experts / d->n_group), d->topk_group);
    }
    if (!(d->route_scale >= 0.0f) || d->route_scale > 1e30f)
        return fail(BRX_EINVAL, "route_scale must be finite and >= 0 (0 means 1)");
    if (d->router_dtype != BRX_DT_F32 && d->router_dtype != BRX_DT_BF16)
        return fail(BRX_EINVAL, "router_dtype %d unknown", d->router_dtype);
    if (d->shared_inter < 0 || d->shared_inter % 64)
        return fail(BRX_EINVAL, "shared_inter %d must be 0 or a multiple of 64", d->shared_inter);
    return BRX_OK;
}

int ensure_device() {
    if (g_device < 0) return fail(BRX_ESTATE, "brx_init() has not been called");
    return BRX_OK;
}

int ws_reserve(size_t bytes, hipStream_t s, void** out) {
    std::lock_guard<std::mutex> lk(g_ws_mu);
    if (g_ws.ptr && g_ws.bytes >= bytes) { *out = g_ws.ptr; return BRX_OK; }
    // growing: work queued on the old buffer must finish before it is released
    HIP_TRY(hipDeviceSynchronize());
    if (g_ws.ptr) { HIP_TRY(hipFree(g_ws.ptr)); g_ws.ptr = nullptr; g_ws.bytes = 0; }
    size_t want = bytes + bytes / 4 + (1 << 20);
    hipError_t e = hipMalloc(&g_ws.ptr, want);
    if (e != hipSuccess) { g_ws.ptr = nullptr; return fail(BRX_ENOMEM, "workspace of %zu bytes: %s", want, hipGetErrorString(e)); }
    g_ws.bytes = want;
    (void)s;
    *out = g_ws.ptr;
    return BRX_OK;
}

}  // namespace

struct brx_pool {
    brx_layer_desc d;
    Layout lay;
    int capacity;
    int64_t stride;
    uint8_t* slots;
    int32_t* g2s_dev;
    int32_t* g2s_pinned;
    int32_t* err_dev;           // {flag, expert}: a forward met an expert that was not resident
    int resident;               // table entries >= 0 as last uploaded (pools without host backing)
    hipEvent_t last_read;
    hipEvent_t refill_done;
    hipEvent_t g2s_uploaded;
    const uint8_t* host;        // host backing (device-visible pinned memory), slot stride apart, or null
    bool read_recorded;
    bool refill_recorded;
    bool refill_pending;
    bool g2s_recorded;
};

extern "C" {

int brx_abi_version(void) { return BRX_ABI_VERSION; }

const char* brx_last_error(void) { return g_err.c_str(); }

int brx_init(int device) {
    int n = 0;
    HIP_TRY(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) return fail(BRX_EINVAL, "device %d outside [0, %d)", device, n);
    HIP_TRY(hipSetDevice(device));
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(BRX_EINVAL, "device %d is %s; libbrx is built for gfx950 only", device, prop.gcnArchName);
    if (device >= kMaxDevices) return fail(BRX_EINVAL, "device %d outside [0, %d)", device, kMaxDevices);
    if (!g_scratch_ptr[device]) {
        // this device's copy of the no-alloc scratch, looked up with the device current
        void* sp = nullptr;
        HIP_TRY(hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch)));
        if (!sp || ((uintptr_t)sp & 255)) return fail(BRX_EHIP, "no-alloc scratch resolved to %p", sp);
        g_scratch_ptr[device] = sp;
    }
    g_device = device;
    return BRX_OK;
}

int brx_expert_layout_get(const brx_layer_desc* d, int shared, brx_expert_layout* out) {
    int rc = check_desc(d);
    if (rc) return rc;
    if (!out) return fail(BRX_EINVAL, "out is NULL");
    if (shared && !d->shared_inter) return fail(BRX_EINVAL, "layer has no shared expert");
    Layout L = make_layout(*d, shared ? d->shared_inter : d->inter);
    for (int p = 0; p < 3; ++p) {
        out->weight[p] = L.p[p].w;
        out->scales[p] = L.p[p].s;
        out->biases[p] = L.p[p].b;
        out->bias[p] = L.p[p].bias;
    }
    out->bytes_per_expert = L.bytes;
    return BRX_OK;
}

int brx_pool_create(const brx_layer_desc* d, int capacity, brx_pool** out) {
    int rc = check_desc(d);
    if (rc) return rc;
    if ((rc = ensure_device())) return rc;
    if (!out) return fail(BRX_EINVAL, "out is NULL");
    if (capacity < 1 || capacity > d->n_experts)
        return fail(BRX_EINVAL, "capacity must be in [1, %d], got %d", d->n_experts, capacity);
    brx_pool* p = new brx_pool{};
    p->d = *d;
    p->lay = make_layout(*d, d->inter);
    p->capacity = capacity;
    p->stride = (p->lay.bytes + 255) & ~(int64_t)255;
    hipError_t e = hipMalloc(&p->slots, (size_t)p->stride * capacity);
    if (e != hipSuccess) {
        delete p;
        return fail(BRX_ENOMEM, "%d slots of %lld bytes: %s", capacity, (long long)p->stride, hipGetErrorString(e));
    }
    e = hipMalloc(&p->g2s_dev, sizeof(int32_t) * d->n_experts);
    // every expert starts absent (-1)
    if (e == hipSuccess) e = hipMemset(p->g2s_dev, 0xFF, sizeof(int32_t) * d->n_experts);
    if (e == hipSuccess) e = hipMalloc(&p->err_dev, 2 * sizeof(int32_t));
    if (e == hipSuccess) e = hipMemset(p->err_dev, 0, 2 * sizeof(int32_t));
    if (e == hipSuccess) e = hipHostMalloc(&p->g2s_pinned, sizeof(int32_t) * d->n_experts, hipHostMallocDefault);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&p->last_read, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&p->refill_done, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&p->g2s_uploaded, hipEventDisableTiming);
    if (e != hipSuccess) {
        brx_pool_destroy(p);
        return fail(BRX_ENOMEM, "pool tables: %s", hipGetErrorString(e));
    }
    *out = p;
    return BRX_OK;
}

int brx_pool_destroy(brx_pool* p) {
    if (!p) return BRX_OK;
    (void)hipDeviceSynchronize();
    if (p->slots) (void)hipFree(p->slots);
    if (p->g2s_dev) (void)hipFree(p->g2s_dev);
    if (p->err_dev) (void)hipFree(p->err_dev);
    if (p->g2s_pinned) (void)hipHostFree(p->g2s_pinned);
    if (p->last_read) (void)hipEventDestroy(p->last_read);
    if (p->refill_done) (void)hipEventDestroy(p->refill_done);
    if (p->g2s_uploaded) (void)hipEventDestroy(p->g2s_uploaded);
    delete p;
    return BRX_OK;
}

int brx_pool_capacity(const brx_pool* p) { return p ? p->capacity : fail(BRX_EINVAL, "pool is NULL"); }

int brx_pool_slot_ptr(brx_pool* p, int slot, void** out) {
    if (!p || !out) return fail(BRX_EINVAL, "pool or out is NULL");
    if (slot < 0 || slot >= p->capacity) return fail(BRX_ERANGE, "slot %d outside [0, %d)", slot, p->capacity);
    *out = p->slots + (int64_t)slot * p->stride;
    return BRX_OK;
}

int brx_pool_g2s_ptr(brx_pool* p, int32_t** out) {
    if (!p || !out) return fail(BRX_EINVAL, "pool or out is NULL");
    *out = p->g2s_dev;
    return BRX_OK;
}

static int refill(brx_pool* p, int slot, const void* src, size_t nbytes, void* copy_stream,
                  hipMemcpyKind kind) {
    if (!p || !src) return fail(BRX_EINVAL, "pool or source is NULL");
    if (slot < 0 || slot >= p->capacity) return fail(BRX_ERANGE, "slot %d outside [0, %d)", slot, p->capacity);
    if ((int64_t)nbytes != p->lay.bytes)
        return fail(BRX_EINVAL, "the layout accounts for %lld bytes but the region supplied %zu. "
                    "Refusing to write a partially-filled slot.", (long long)p->lay.bytes, nbytes);
    hipStream_t cs = (hipStream_t)copy_stream;
    if (p->read_recorded) HIP_TRY(hipStreamWaitEvent(cs, p->last_read, 0));
    HIP_TRY(hipMemcpyAsync(p->slots + (int64_t)slot * p->stride, src, nbytes, kind, cs));
    HIP_TRY(hipEventRecord(p->refill_done, cs));
    p->refill_pending = true;
    p->refill_recorded = true;
    return BRX_OK;
}

int brx_pool_refill_async(brx_pool* p, int slot, const void* host_src, size_t nbytes, void* copy_stream) {
    return refill(p, slot, host_src, nbytes, copy_stream, hipMemcpyHostToDevice);
}

int brx_pool_refill_range_async(brx_pool* p, int slot0, int n, const void* host_src, int64_t host_stride,
                                size_t nbytes, void* copy_stream) {
    if (!p || !host_src) return fail(BRX_EINVAL, "pool or source is NULL");
    if (n < 1 || slot0 < 0 || slot0 + n > p->capacity)
        return fail(BRX_ERANGE, "slots [%d, %d) outside [0, %d)", slot0, slot0 + n, p->capacity);
    if ((int64_t)nbytes != p->lay.bytes)
        return fail(BRX_EINVAL, "the layout accounts for %lld bytes but the region supplied %zu. "
                    "Refusing to write a partially-filled slot.", (long long)p->lay.bytes, nbytes);
    if (host_stride < (int64_t)nbytes) return fail(BRX_EINVAL, "host stride %lld is below the expert size", (long long)host_stride);
    hipStream_t cs = (hipStream_t)copy_stream;
    if (p->read_recorded) HIP_TRY(hipStreamWaitEvent(cs, p->last_read, 0));
    uint8_t* dst = p->slots + (int64_t)slot0 * p->stride;
    const uint8_t* src = (const uint8_t*)host_src;
    if (host_stride == p->stride && p->stride == p->lay.bytes) {
        // the experts are back to back on both sides: one transfer (a single DMA stream moves
        // ~40% more per second than one copy per expert)
        HIP_TRY(hipMemcpyAsync(dst, src, (size_t)n * nbytes, hipMemcpyHostToDevice, cs));
    } else {
        for (int i = 0; i < n; ++i)
            HIP_TRY(hipMemcpyAsync(dst + (int64_t)i * p->stride, src + (int64_t)i * host_stride, nbytes,
                                   hipMemcpyHostToDevice, cs));
    }
    HIP_TRY(hipEventRecord(p->refill_done, cs));
    p->refill_pending = true;
    p->refill_recorded = true;
    return BRX_OK;
}

int brx_pool_refill_from_device_async(brx_pool* p, int slot, const void* dev_src, size_t nbytes,
                                      void* copy_stream) {
    return refill(p, slot, dev_src, nbytes, copy_stream, hipMemcpyDeviceToDevice);
}

int brx_pool_set_g2s(brx_pool* p, const int32_t* g2s_host, int n, void* stream) {
    if (!p || !g2s_host) return fail(BRX_EINVAL, "pool or table is NULL");
    if (n != p->d.n_experts) return fail(BRX_EINVAL, "table has %d entries, layer has %d experts", n, p->d.n_experts);
    for (int e = 0; e < n; ++e)
        if (g2s_host[e] >= p->capacity)
            return fail(BRX_ERANGE, "expert %d maps to slot %d outside [0, %d)", e, g2s_host[e], p->capacity);
    hipStream_t s = (hipStream_t)stream;
    // the staging copy of the previous upload must have been consumed before it is rewritten
    if (p->g2s_recorded) HIP_TRY(hipEventSynchronize(p->g2s_uploaded));
    // -1 stays -1 (absent): with host backing the kernels read the expert from host memory,
    // without it a forward that routes to it records the error and writes NaN rows
    int resident = 0;
    for (int e = 0; e < n; ++e) {
        p->g2s_pinned[e] = g2s_host[e] >= 0 ? g2s_host[e] : -1;
        resident += g2s_host[e] >= 0 ? 1 : 0;
    }
    p->resident = resident;
    HIP_TRY(hipMemcpyAsync(p->g2s_dev, p->g2s_pinned, sizeof(int32_t) * n, hipMemcpyHostToDevice, s));
    HIP_TRY(hipEventRecord(p->g2s_uploaded, s));
    p->g2s_recorded = true;
    return BRX_OK;
}

int brx_pool_set_host_backing(brx_pool* p, const void* host_base, int64_t host_stride, size_t host_bytes) {
    if (!p || !host_base) return fail(BRX_EINVAL, "pool or host_base is NULL");
    if (p->host) return fail(BRX_EINVAL, "the pool already has host backing");
    if (p->refill_recorded || p->g2s_recorded || p->read_recorded)
        return fail(BRX_EINVAL, "host backing is set on a fresh pool, before any refill, table upload or forward");
    const int E = p->d.n_experts;
    // the kernels address a host expert exactly as a slot: same stride, same alignment
    if (host_stride != p->stride)
        return fail(BRX_EINVAL, "host stride %lld must equal the slot stride %lld (bytes per expert rounded "
                    "up to 256)", (long long)host_stride, (long long)p->stride);
    if ((uintptr_t)host_base & 255) return fail(BRX_EINVAL, "host_base must be a multiple of 256 bytes");
    const size_t need = (size_t)(E - 1) * (size_t)host_stride + (size_t)p->lay.bytes;
    if (host_bytes < need)
        return fail(BRX_EINVAL, "%d experts at stride %lld need %zu bytes, the region has %zu", E,
                    (long long)host_stride, need, host_bytes);
    // both ends of the range must be pinned host memory the device sees at the same address
    const uint8_t* ends[2] = {(const uint8_t*)host_base, (const uint8_t*)host_base + need - 1};
    for (const uint8_t* q : ends) {
        hipPointerAttribute_t at{};
        hipError_t e = hipPointerGetAttributes(&at, q);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return fail(BRX_EINVAL, "host backing %p is not memory the runtime knows (%s): allocate it pinned",
                        (const void*)q, hipGetErrorString(e));
        }
        // the kernels are given host_base itself: the device must see it at that address
        if (at.type != hipMemoryTypeHost || (q == ends[0] && at.devicePointer != (void*)q))
            return fail(BRX_EINVAL, "host backing %p is not pinned host memory mapped at the same device "
                        "address (type %d, device pointer %p)", (const void*)q, (int)at.type, at.devicePointer);
    }
    // nothing is resident yet: every entry starts as -1, "read from host"
    p->host = (const uint8_t*)host_base;
    for (int e = 0; e < E; ++e) p->g2s_pinned[e] = -1;
    HIP_TRY(hipMemcpy(p->g2s_dev, p->g2s_pinned, sizeof(int32_t) * E, hipMemcpyHostToDevice));
    return BRX_OK;
}

int brx_pool_publish_async(brx_pool* p, int n, const int32_t* experts, const int32_t* slots, void* stream) {
    if (!p || (n > 0 && (!experts || !slots))) return fail(BRX_EINVAL, "pool, experts or slots is NULL");
    if (!p->host) return fail(BRX_EINVAL, "table entries are published only on a pool with host backing");
    if (n < 0) return fail(BRX_EINVAL, "n %d < 0", n);
    for (int i = 0; i < n; ++i) {
        if (experts[i] < 0 || experts[i] >= p->d.n_experts)
            return fail(BRX_ERANGE, "expert %d outside [0, %d)", experts[i], p->d.n_experts);
        if (slots[i] < -1 || slots[i] >= p->capacity)
            return fail(BRX_ERANGE, "slot %d outside [-1, %d)", slots[i], p->capacity);
        for (int j = 0; j < i; ++j)
            if (experts[j] == experts[i]) return fail(BRX_EINVAL, "expert %d appears twice", experts[i]);
    }
    for (int i0 = 0; i0 < n; i0 += kMaxTableEdits) {
        TableEdits ed{};
        ed.n = n - i0 < kMaxTableEdits ? n - i0 : kMaxTableEdits;
        for (int i = 0; i < ed.n; ++i) {
            ed.e[i] = experts[i0 + i];
            ed.v[i] = slots[i0 + i];
        }
        hipError_t e = launch_table_set(p->g2s_dev, ed, (hipStream_t)stream);
        if (e != hipSuccess) return hip_fail(e, "table update");
    }
    return BRX_OK;
}

int brx_pool_admit_async(brx_pool* p, int expert, int slot, const void* host_src, size_t nbytes,
                         void* copy_stream) {
    if (!p) return fail(BRX_EINVAL, "pool is NULL");
    if (!p->host) return fail(BRX_EINVAL, "brx_pool_admit_async needs a pool with host backing");
    if (expert < 0 || expert >= p->d.n_experts)
        return fail(BRX_ERANGE, "expert %d outside [0, %d)", expert, p->d.n_experts);
    if (slot < 0 || slot >= p->capacity) return fail(BRX_ERANGE, "slot %d outside [0, %d)", slot, p->capacity);
    if (!host_src) return fail(BRX_EINVAL, "source is NULL");
    if ((int64_t)nbytes != p->lay.bytes)
        return fail(BRX_EINVAL, "the layout accounts for %lld bytes but the region supplied %zu. "
                    "Refusing to write a partially-filled slot.", (long long)p->lay.bytes, nbytes);
    hipStream_t cs = (hipStream_t)copy_stream;
    // write-after-read: every forward issued so far may still read the slot's old expert
    if (p->read_recorded) HIP_TRY(hipStreamWaitEvent(cs, p->last_read, 0));
    HIP_TRY(hipMemcpyAsync(p->slots + (int64_t)slot * p->stride, host_src, nbytes, hipMemcpyHostToDevice, cs));
    TableEdits ed{};
    ed.n = 1;
    ed.e[0] = expert;
    ed.v[0] = slot;
    hipError_t e = launch_table_set(p->g2s_dev, ed, cs);
    if (e != hipSuccess) return hip_fail(e, "table update");
    // forwards do not wait for this copy: until the table entry lands they read the expert
    // from host backing, after it from the slot (the same bytes)
    HIP_TRY(hipEventRecord(p->refill_done, cs));
    p->refill_recorded = true;
    return BRX_OK;
}

int brx_pool_sync(brx_pool* p) {
    if (!p) return fail(BRX_EINVAL, "pool is NULL");
    if (p->refill_recorded) HIP_TRY(hipEventSynchronize(p->refill_done));
    if (p->read_recorded) HIP_TRY(hipEventSynchronize(p->last_read));
    if (p->g2s_recorded) HIP_TRY(hipEventSynchronize(p->g2s_uploaded));
    return BRX_OK;
}

int brx_pool_check(brx_pool* p) {
    if (!p) return fail(BRX_EINVAL, "pool is NULL");
    int rc = brx_pool_sync(p);
    if (rc) return rc;
    int32_t h[2] = {0, 0};
    HIP_TRY(hipMemcpy(h, p->err_dev, sizeof h, hipMemcpyDeviceToHost));
    if (h[0]) {
        HIP_TRY(hipMemset(p->err_dev, 0, sizeof h));
        return fail(BRX_ERANGE, "a forward routed to expert %d, which is neither in a slot nor host-backed; "
                    "the rows it touched were written as NaN", h[1]);
    }
    return BRX_OK;
}

int brx_router_topk(const brx_layer_desc* d, const void* x, const void* w_router, const float* bias,
                    const void* shared_gate_w, int T, int32_t* out_idx, float* out_w,
                    float* out_shared_gate, void* stream) {
    int rc = check_desc(d);
    if (rc) return rc;
    if ((rc = ensure_device())) return rc;
    if (T < 0) return fail(BRX_EINVAL, "T %d < 0", T);
    if (T == 0) return BRX_OK;
    if (!x || !w_router || !out_idx || !out_w) return fail(BRX_EINVAL, "x, w_router, out_idx and out_w are required");
    if (((uintptr_t)x | (uintptr_t)w_router) & 15) return fail(BRX_EINVAL, "x and w_router must be 16-byte aligned");
    if (shared_gate_w && ((uintptr_t)shared_gate_w & 15)) return fail(BRX_EINVAL, "shared_gate_w must be 16-byte aligned");
    if (shared_gate_w && !out_shared_gate) return fail(BRX_EINVAL, "shared_gate_w given without out_shared_gate");
    void* ws = nullptr;
    size_t need = router_workspace_bytes(*d, T);
    if (need && (rc = ws_reserve(need, (hipStream_t)stream, &ws))) return rc;
    hipError_t e = launch_router(*d, x, w_router, bias, shared_gate_w, T, out_idx, out_w, out_shared_gate,
                                 (float*)ws, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "router launch");
    return BRX_OK;
}

static FwdArgs make_args(const brx_layer_desc* d, brx_pool* p, const void* x, int T, int P,
                         const int32_t* pexp, const int32_t* ptok, const int32_t* prow, int yrows,
                         const float* w, const void* shared_expert, const float* shared_gate,
                         void* out, void* y_rows) {
    const bool token_mode = ptok == nullptr;
    FwdArgs a{};
    a.x = (const uint16_t*)x;
    a.P = P;
    a.pexp = pexp;
    a.ptok = ptok;
    a.prow = prow;
    a.w = w;
    a.sgate = shared_gate;
    a.slots = p->slots;
    a.slot_stride = p->stride;
    a.g2s = p->g2s_dev;
    a.capacity = p->capacity;
    a.host = p->host;
    a.shared = (const uint8_t*)shared_expert;
    a.auto_shared = (token_mode && shared_expert) ? 1 : 0;
    a.lay = p->lay;
    a.lay_sh = d->shared_inter ? make_layout(*d, d->shared_inter) : p->lay;
    a.T = T; a.H = d->hidden; a.I = d->inter; a.I_sh = shared_expert ? d->shared_inter : 0;
    a.E = d->n_experts; a.k = d->top_k;
    a.quant_mode = kernel_mode(d->quant_mode, d->bits);
    a.gshift = d->quant_mode == BRX_QUANT_AFFINE && d->group_size == 128 ? 1 : 0;
    a.scale_f16 = d->scale_dtype == BRX_SCALE_F16; a.has_bias = d->has_bias;
    a.act = d->act; a.alpha = d->alpha; a.limit = d->limit;
    a.out = (uint16_t*)out;
    a.yun = (uint16_t*)y_rows;
    a.yrows = yrows;
    const RouteRule rr = route_rule(*d, nullptr);
    a.route_mode = rr.mode;
    a.n_group = rr.n_group;
    a.topk_group = rr.topk_group;
    a.route_scale = rr.scale;
    a.err = p->err_dev;
    return a;
}

// Queue the expert kernels of one forward on `s` over workspace `ws` (decode or grouped GEMM),
// ordered after the pool's pending refills, and mark the pool read.
static int run_forward(brx_pool* p, const FwdArgs& a, bool decode, int phases, void* ws,
                       size_t ws_bytes, hipStream_t s) {
    if (p->refill_pending) {
        // forwards of one pool are issued on one stream: once it has waited, later ones follow
        HIP_TRY(hipStreamWaitEvent(s, p->refill_done, 0));
        p->refill_pending = false;
    }
    hipError_t e = decode ? launch_decode(a, ws, phases, s) : launch_prefill(a, ws, ws_bytes, phases, s);
    if (e != hipSuccess) return hip_fail(e, decode ? "decode launch" : "prefill launch");
    HIP_TRY(hipEventRecord(p->last_read, s));
    p->read_recorded = true;
    return BRX_OK;
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

static int forward_impl(const brx_layer_desc* d, brx_pool* p, const void* x, int T, int P,
                        const int32_t* pexp, const int32_t* ptok, const int32_t* prow, int yrows,
                        const float* w, const void* shared_expert, const float* shared_gate,
                        void* out, void* y_rows, unsigned flags, void* stream) {
    const bool force_dec = flags & BRX_FWD_FORCE_DECODE, force_pf = flags & BRX_FWD_FORCE_PREFILL;
    if (force_dec && force_pf) return fail(BRX_EINVAL, "FORCE_DECODE and FORCE_PREFILL are exclusive");
    const bool token_mode = ptok == nullptr;
    // the decode kernels stage every token row of x and plan at most 64 pairs
    bool decode = force_dec || (!force_pf && T <= 8 && P <= (token_mode ? 64 : 8));
    if (decode && (T > 8 || P > 64))
        return fail(BRX_EINVAL, "the decode path takes at most 8 token rows and 64 pairs (T=%d, P=%d)", T, P);
    FwdArgs a = make_args(d, p, x, T, P, pexp, ptok, prow, yrows, w, shared_expert, shared_gate, out, y_rows);
    hipStream_t s = (hipStream_t)stream;
    size_t need = decode ? decode_workspace_bytes(a) : prefill_workspace_bytes(a);
    void* ws = nullptr;
    int rc = ws_reserve(need, s, &ws);
    if (rc) return rc;
    int phases = (flags & (BRX_FWD_PHASE_A | BRX_FWD_PHASE_B)) >> 2;
    if (phases == 0) phases = 3;
    return run_forward(p, a, decode, phases, ws, g_ws.bytes, s);
}

static int check_forward_common(const brx_layer_desc* d, brx_pool* p, const void* x) {
    int rc = check_desc(d);
    if (rc) return rc;
    if ((rc = ensure_device())) return rc;
    if (!p) return fail(BRX_EINVAL, "pool is NULL");
    if (memcmp(&p->d, d, sizeof(brx_layer_desc)) != 0)
        return fail(BRX_EINVAL, "descriptor differs from the one the pool was built with");
    if (!x) return fail(BRX_EINVAL, "x is required");
    if ((uintptr_t)x & 15) return fail(BRX_EINVAL, "x must be 16-byte aligned");
    return BRX_OK;
}

int brx_moe_forward(const brx_layer_desc* d, brx_pool* p, const void* x, const int32_t* idx, const float* w,
                    const void* shared_expert, const float* shared_gate, int T, void* out, void* y_unreduced,
                    unsigned flags, void* stream) {
    int rc = check_forward_common(d, p, x);
    if (rc) return rc;
    if (T < 0) return fail(BRX_EINVAL, "T %d < 0", T);
    if (T == 0) return BRX_OK;
    if (!idx) return fail(BRX_EINVAL, "idx is required");
    if (out && !w) return fail(BRX_EINVAL, "a combined output needs routing weights w");
    if (!out && !y_unreduced) return fail(BRX_EINVAL, "nothing to write: out and y_unreduced are both NULL");
    if (((uintptr_t)out & 3) || ((uintptr_t)y_unreduced & 3))
        return fail(BRX_EINVAL, "out and y_unreduced must be 4-byte aligned");
    if (shared_expert && !d->shared_inter) return fail(BRX_EINVAL, "layer descriptor has no shared expert");
    if (shared_expert && out && !shared_gate) return fail(BRX_EINVAL, "shared expert given without its gate values");
    if (shared_expert && ((uintptr_t)shared_expert & 15)) return fail(BRX_EINVAL, "shared expert must be 16-byte aligned");
    return forward_impl(d, p, x, T, T * d->top_k, idx, nullptr, nullptr, T * d->top_k, w, shared_expert, shared_gate, out,
                        y_unreduced, flags, stream);
}

int brx_moe_forward_pairs(const brx_layer_desc* d, brx_pool* p, const void* x, int T,
                          const int32_t* pair_token, const int32_t* pair_expert, const int32_t* pair_row,
                          int n_pairs, int n_rows, const void* shared_expert, void* y_rows, unsigned flags,
                          void* stream) {
    int rc = check_forward_common(d, p, x);
    if (rc) return rc;
    if (n_pairs < 0 || T < 0) return fail(BRX_EINVAL, "negative size (T=%d, n_pairs=%d)", T, n_pairs);
    if (n_pairs == 0) return BRX_OK;
    if (T == 0) return fail(BRX_EINVAL, "pairs given but x has no rows");
    if (!pair_token || !pair_expert || !y_rows) return fail(BRX_EINVAL, "pair_token, pair_expert and y_rows are required");
    if ((uintptr_t)y_rows & 3) return fail(BRX_EINVAL, "y_rows must be 4-byte aligned");
    if (pair_row ? n_rows < 1 : n_rows < n_pairs)
        return fail(BRX_EINVAL, "y_rows has %d rows for %d pairs", n_rows, n_pairs);
    if (shared_expert && !d->shared_inter) return fail(BRX_EINVAL, "layer descriptor has no shared expert");
    if (shared_expert && ((uintptr_t)shared_expert & 15)) return fail(BRX_EINVAL, "shared expert must be 16-byte aligned");
    return forward_impl(d, p, x, T, n_pairs, pair_expert, pair_token, pair_row, n_rows, nullptr, shared_expert, nullptr,
                        nullptr, y_rows, flags, stream);
}

// The whole block over either the library workspace (scratch == nullptr: grown on demand) or
// the caller-free static scratch of `scratch_bytes` (nothing allocated; too small -> EINVAL).
static int block_forward_impl(const brx_layer_desc* d, brx_pool* p, const void* x, const void* w_router,
                              const float* router_bias, const void* shared_gate_w, const void* shared_expert,
                              int T, void* out, int32_t* out_idx, float* out_w, unsigned flags, void* stream,
                              void* scratch_ws, size_t scratch_bytes) {
    int rc = check_forward_common(d, p, x);
    if (rc) return rc;
    if (T < 0) return fail(BRX_EINVAL, "T %d < 0", T);
    if (T == 0) return BRX_OK;
    if (!w_router || !out) return fail(BRX_EINVAL, "w_router and out are required");
    if ((uintptr_t)w_router & 15) return fail(BRX_EINVAL, "w_router must be 16-byte aligned");
    if ((uintptr_t)out & 3) return fail(BRX_EINVAL, "out must be 4-byte aligned");
    if (!shared_gate_w != !shared_expert)
        return fail(BRX_EINVAL, "shared_gate_w and shared_expert go together");
    if (shared_expert && !d->shared_inter) return fail(BRX_EINVAL, "layer descriptor has no shared expert");
    if (shared_expert && (((uintptr_t)shared_expert | (uintptr_t)shared_gate_w) & 15))
        return fail(BRX_EINVAL, "shared expert and shared_gate_w must be 16-byte aligned");
    const bool force_dec = flags & BRX_FWD_FORCE_DECODE, force_pf = flags & BRX_FWD_FORCE_PREFILL;
    if (force_dec && force_pf) return fail(BRX_EINVAL, "FORCE_DECODE and FORCE_PREFILL are exclusive");
    const unsigned phase_bits = flags & (BRX_FWD_PHASE_R | BRX_FWD_PHASE_A | BRX_FWD_PHASE_B);
    const bool do_route = !phase_bits || (flags & BRX_FWD_PHASE_R);
    int phases = phase_bits ? (int)((flags & (BRX_FWD_PHASE_A | BRX_FWD_PHASE_B)) >> 2) : 3;
    const int k = d->top_k, P = T * k;
    // the decode kernels rank and plan at most 64 (token, expert) pairs in one wave
    const bool decode = force_dec || (!force_pf && T <= 8 && P <= 64);
    if (decode && (T > 8 || P > 64))
        return fail(BRX_EINVAL, "the decode path takes at most 8 tokens and 64 pairs (T=%d, top_k=%d)", T, k);
    // the block reads the table for every expert the router may pick: all must be resident, or
    // served from host backing (the reference raises KeyError for a non-resident expert,
    // stream.py:608-615)
    if (!p->host && p->resident < d->n_experts)
        return fail(BRX_ESTATE, "brx_moe_block_forward needs every expert resident or a host-backed pool "
                    "(%d of %d experts resident)", p->resident, d->n_experts);
    hipStream_t s = (hipStream_t)stream;

    // one workspace for the whole block: routing first, then the expert kernels' scratch
    const size_t logits_b = align256(sizeof(float) * (size_t)T * (d->n_experts + 1));
    const size_t idx_b = out_idx ? 0 : align256(sizeof(int32_t) * P);
    const size_t w_b = out_w ? 0 : align256(sizeof(float) * P);
    const size_t sg_b = shared_expert ? align256(sizeof(float) * T) : 0;
    const size_t route_b = logits_b + idx_b + w_b + sg_b;
    FwdArgs a = make_args(d, p, x, T, P, nullptr, nullptr, nullptr, P, nullptr, shared_expert, nullptr, out,
                          nullptr);
    const size_t fwd_b = decode ? decode_workspace_bytes(a) : prefill_workspace_bytes(a);
    void* ws = nullptr;
    size_t ws_bytes = 0;
    if (scratch_ws) {
        if (route_b + fwd_b > scratch_bytes)
            return fail(BRX_EINVAL, "this call needs %zu bytes of scratch, the no-alloc scratch holds %zu "
                        "(T=%d); use brx_moe_block_forward", route_b + fwd_b, scratch_bytes, T);
        ws = scratch_ws;
        ws_bytes = scratch_bytes;
    } else {
        if ((rc = ws_reserve(route_b + fwd_b, s, &ws))) return rc;
        ws_bytes = g_ws.bytes;
    }
    char* base = (char*)ws;
    float* logits = (float*)base;
    int32_t* ridx = out_idx ? out_idx : (int32_t*)(base + logits_b);
    float* rw = out_w ? out_w : (float*)(base + logits_b + idx_b);
    float* rsg = shared_expert ? (float*)(base + logits_b + idx_b + w_b) : nullptr;
    void* fws = base + route_b;
    a.pexp = ridx;
    a.w = rw;
    a.sgate = rsg;
    hipError_t e = hipSuccess;
    if (decode) {
        a.logits = logits;
        a.route_bias = route_rule(*d, router_bias).bias;
        a.route_idx = ridx;
        a.route_w = rw;
        a.route_sg = rsg;
        if (do_route) e = launch_router_logits(*d, x, w_router, router_bias, shared_gate_w, T, logits, s);
    } else if (do_route) {
        e = launch_router(*d, x, w_router, router_bias, shared_gate_w, T, ridx, rw, rsg, logits, s);
    }
    if (e != hipSuccess) return hip_fail(e, "router launch");
    if (!phases) return BRX_OK;
    return run_forward(p, a, decode, phases, fws, ws_bytes - route_b, s);
}

int brx_moe_block_forward(const brx_layer_desc* d, brx_pool* p, const void* x, const void* w_router,
                          const float* router_bias, const void* shared_gate_w, const void* shared_expert,
                          int T, void* out, int32_t* out_idx, float* out_w, unsigned flags, void* stream) {
    return block_forward_impl(d, p, x, w_router, router_bias, shared_gate_w, shared_expert, T, out, out_idx,
                              out_w, flags, stream, nullptr, 0);
}

int brx_moe_block_forward_noalloc(const brx_layer_desc* d, brx_pool* p, const void* x, const void* w_router,
                                  const float* router_bias, const void* shared_gate_w,
                                  const void* shared_expert, int T, void* out, int32_t* out_idx, float* out_w,
                                  unsigned flags, void* stream) {
    int rc = ensure_device();
    if (rc) return rc;
    void* sp = g_scratch_ptr[g_device];
    if (!sp) return fail(BRX_ESTATE, "no-alloc scratch of device %d is not set up", g_device);
    return block_forward_impl(d, p, x, w_router, router_bias, shared_gate_w, shared_expert, T, out, out_idx,
                              out_w, flags, stream, sp, BRX_NOALLOC_SCRATCH_BYTES);
}

int brx_combine(const brx_layer_desc* d, const void* y_routed, const float* w, const void* y_shared,
                const float* shared_gate, int T, void* out, void* stream) {
    int rc = check_desc(d);
    if (rc) return rc;
    if ((rc = ensure_device())) return rc;
    if (T < 0) return fail(BRX_EINVAL, "T %d < 0", T);
    if (T == 0) return BRX_OK;
    if (!y_routed || !w || !out) return fail(BRX_EINVAL, "y_routed, w and out are required");
    if (y_shared && !shared_gate) return fail(BRX_EINVAL, "y_shared given without shared_gate");
    if (((uintptr_t)y_routed | (uintptr_t)y_shared | (uintptr_t)out) & 3)
        return fail(BRX_EINVAL, "y_routed, y_shared and out must be 4-byte aligned");
    hipError_t e = launch_combine((const uint16_t*)y_routed, (const uint16_t*)y_shared, w, shared_gate, T,
                                  d->top_k, d->hidden, (uint16_t*)out, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "combine launch");
    return BRX_OK;
}

int brx_dequant(const brx_layer_desc* d, const void* expert, int proj, int shared, float* out, void* stream) {
    int rc = check_desc(d);
    if (rc) return rc;
    if ((rc = ensure_device())) return rc;
    if (!expert || !out) return fail(BRX_EINVAL, "expert and out are required");
    if (proj < 0 || proj > 2) return fail(BRX_EINVAL, "proj %d outside [0, 2]", proj);
    if (proj == 1 && d->act == BRX_ACT_SILU_MLP) return fail(BRX_EINVAL, "a two-layer expert has no projection 1");
    if (shared && !d->shared_inter) return fail(BRX_EINVAL, "layer has no shared expert");
    Layout L = make_layout(*d, shared ? d->shared_inter : d->inter);
    hipError_t e = launch_dequant(*d, L, (const uint8_t*)expert, proj, out, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "dequant launch");
    return BRX_OK;
}

int brx_sort_pairs(const brx_layer_desc* d, const int32_t* idx, int T, int32_t* out_order,
                   int32_t* out_offsets, void* stream) {
    int rc = check_desc(d);
    if (rc) return rc;
    if ((rc = ensure_device())) return rc;
    if (T <= 0) return fail(BRX_EINVAL, "T %d <= 0", T);
    if (!idx || !out_order || !out_offsets) return fail(BRX_EINVAL, "idx, out_order, out_offsets are required");
    void* ws = nullptr;
    if ((rc = ws_reserve(sizeof(int32_t) * (d->n_experts + 2), (hipStream_t)stream, &ws))) return rc;
    hipError_t e = launch_sort_pairs(idx, T * d->top_k, d->n_experts, d->n_experts, 0, 128, out_order,
                                     out_offsets, (int32_t*)ws, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "sort launch");
    return BRX_OK;
}

}  // extern "C"
