// libmbhip.so runtime: device selection, the kernel registry, binding
// validation and the timed dispatch loop.
//
// This is the in-process replacement of the reference's host binary:
//   - device + queue set-up      reference metal/scripts/main.mm:102-117
//   - buffer/scalar binding      reference metal/scripts/main.mm:125-159
//   - warmup + timed dispatches  reference metal/scripts/timing.mm:125-193
//   - chip detection             reference metal/scripts/setup.cpp:116-136
// The manifest's buffers become mb_binding structs holding device pointers
// owned by the caller; timing uses a hipEvent pair per dispatch on one stream.
#include "common.h"

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <vector>

namespace mb {

// ---- errors ---------------------------------------------------------------------
static thread_local char g_err[1024] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { g_err[0] = '\0'; }

// ---- library state ----------------------------------------------------------------
struct State {
    bool inited = false;
    int device = -1;
    hipStream_t lib_stream = nullptr;
    hipStream_t user_stream = nullptr;
    void* ws = nullptr;
    size_t ws_bytes = 0;
    void* flush = nullptr;  // cache-eviction buffer (MB_RUN_COLD)
    uint32_t cu_count = 0;
};
static State g;

bool initialized() { return g.inited; }

uint32_t device_cu_count() { return g.cu_count; }

hipStream_t stream_or_default(void* s) {
    if (s) return static_cast<hipStream_t>(s);
    return g.user_stream ? g.user_stream : g.lib_stream;
}

void* library_workspace(size_t bytes) {
    if (bytes > g.ws_bytes) {
        if (g.ws) {
            // The old workspace may still be read by enqueued work.
            (void)hipDeviceSynchronize();
            (void)hipFree(g.ws);
            g.ws = nullptr;
            g.ws_bytes = 0;
        }
        hipError_t e = hipMalloc(&g.ws, bytes);
        if (e != hipSuccess) {
            g.ws = nullptr;
            fail(MB_E_HIP, "workspace hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
            return nullptr;
        }
        g.ws_bytes = bytes;
    }
    return g.ws;
}

// 512 MiB: twice the 256 MB memory-side cache of an MI355X, far above the
// 4 MB L2 of each XCD.
constexpr size_t FLUSH_BYTES = (size_t)512 << 20;

void* library_flush_buffer(size_t* bytes) {
    if (!g.flush) {
        hipError_t e = hipMalloc(&g.flush, FLUSH_BYTES);
        if (e != hipSuccess) {
            g.flush = nullptr;
            fail(MB_E_HIP, "cache-eviction buffer hipMalloc(%zu) failed: %s", FLUSH_BYTES,
                 hipGetErrorString(e));
            return nullptr;
        }
    }
    *bytes = FLUSH_BYTES;
    return g.flush;
}

// ---- register / LDS usage of the built kernels --------------------------------------
struct KernelResources {
    const char* name;   // mangled kernel symbol
    int arch_vgprs, agprs, sgprs, lds_bytes, private_bytes;
};
static const KernelResources k_resources[] = {
#include "kernel_resources.inc"
    {nullptr, 0, 0, 0, 0, 0}};

static const KernelResources* resources_of(const char* name) {
    if (!name) return nullptr;
    for (const KernelResources* r = k_resources; r->name; ++r)
        if (strcmp(r->name, name) == 0) return r;
    return nullptr;
}

// Waves per SIMD that a workgroup of `threads` lanes can keep resident on
// gfx950: 512 unified VGPRs per lane per SIMD (ArchVGPRs then AGPRs, each
// wave's allocation rounded up to a granule of 8, ArchVGPRs to 4 first), 160
// KB of LDS per CU shared by its 4 SIMDs, at most 8 waves per SIMD.
static int waves_per_simd(int arch_vgprs, int agprs, uint64_t lds_bytes, int threads) {
    const int arch = (arch_vgprs + 3) & ~3;
    const int total = std::max(8, (arch + agprs + 7) & ~7);
    int waves = std::min(8, 512 / total);
    const int waves_per_group = std::max(1, (threads + 63) / 64);
    if (lds_bytes > 0) {
        const int groups = (int)std::min<uint64_t>(64, (160u << 10) / lds_bytes);
        waves = std::min(waves, std::max(0, groups * waves_per_group / 4));
    }
    return std::max(waves, 1);
}

// ---- kernel registry ------------------------------------------------------------
static std::vector<KernelEntry>& table() {
    static std::vector<KernelEntry> t;
    return t;
}

void register_kernel(const KernelEntry& e) { table().push_back(e); }

static std::vector<KernelEntry>& registry() {
    static std::once_flag once;
    std::call_once(once, [] {
        register_transpose();
        register_copy();
        register_gemm_f32();
        register_conv2d();
        register_gemm_bf16();
        register_decoder();
        register_transformer_f32();
    });
    return table();
}

// ---- bindings -----------------------------------------------------------------------
static const char* dtype_name(uint32_t d) {
    switch (d) {
        case MB_DTYPE_F32: return "f32";
        case MB_DTYPE_F16: return "f16";
        case MB_DTYPE_I32: return "i32";
        case MB_DTYPE_U32: return "u32";
        case MB_DTYPE_BF16: return "bf16";
        default: return "?";
    }
}

int Bindings::buffer(uint32_t idx, uint32_t dtype, uint64_t min_bytes, bool output,
                     void** ptr, const char* what) const {
    const mb_binding* b = idx < 32 ? slot[idx] : nullptr;
    if (!b) return fail(MB_E_BINDING, "binding %u (%s) missing", idx, what);
    uint32_t want = output ? MB_ROLE_OUTPUT : MB_ROLE_INPUT;
    if (b->role != want)
        return fail(MB_E_BINDING, "binding %u (%s): role %u, expected %s", idx, what,
                    b->role, output ? "output" : "input");
    if (b->dtype != dtype)
        return fail(MB_E_DTYPE, "binding %u (%s): dtype %s, expected %s", idx, what,
                    dtype_name(b->dtype), dtype_name(dtype));
    if (!b->dev_ptr && min_bytes)   // an empty buffer may come with a null pointer
        return fail(MB_E_BINDING, "binding %u (%s): null pointer", idx, what);
    if (min_bytes && b->nbytes < min_bytes)
        return fail(MB_E_BINDING, "binding %u (%s): %llu bytes, need %llu", idx, what,
                    (unsigned long long)b->nbytes, (unsigned long long)min_bytes);
    *ptr = b->dev_ptr;
    return MB_OK;
}

uint64_t Bindings::nbytes(uint32_t idx) const {
    const mb_binding* b = idx < 32 ? slot[idx] : nullptr;
    return (b && b->role != MB_ROLE_SCALAR) ? b->nbytes : 0;
}

int Bindings::u32(uint32_t idx, uint32_t* v, const char* what) const {
    const mb_binding* b = idx < 32 ? slot[idx] : nullptr;
    if (!b) return fail(MB_E_BINDING, "scalar binding %u (%s) missing", idx, what);
    if (b->role != MB_ROLE_SCALAR)
        return fail(MB_E_BINDING, "binding %u (%s) is not a scalar", idx, what);
    if (b->dtype == MB_DTYPE_U32) { *v = b->scalar.u32; return MB_OK; }
    if (b->dtype == MB_DTYPE_I32 && b->scalar.i32 >= 0) { *v = (uint32_t)b->scalar.i32; return MB_OK; }
    return fail(MB_E_DTYPE, "scalar %u (%s): dtype %s, expected u32", idx, what,
                dtype_name(b->dtype));
}

int Bindings::f32(uint32_t idx, float* v, const char* what) const {
    const mb_binding* b = idx < 32 ? slot[idx] : nullptr;
    if (!b) return fail(MB_E_BINDING, "scalar binding %u (%s) missing", idx, what);
    if (b->role != MB_ROLE_SCALAR)
        return fail(MB_E_BINDING, "binding %u (%s) is not a scalar", idx, what);
    if (b->dtype != MB_DTYPE_F32)
        return fail(MB_E_DTYPE, "scalar %u (%s): dtype %s, expected f32", idx, what,
                    dtype_name(b->dtype));
    *v = b->scalar.f32;
    return MB_OK;
}

}  // namespace mb

using namespace mb;

// ==== C ABI ========================================================================
extern "C" {

int mb_abi_version(void) { return MBHIP_ABI_VERSION; }

int mb_abi_struct_size(int which) {
    switch (which) {
        case 0: return (int)sizeof(mb_binding);
        case 1: return (int)sizeof(mb_timing);
        case 2: return (int)sizeof(mb_device_info);
        case 3: return (int)sizeof(mb_kernel_attrs);
        case 4: return (int)sizeof(mb_decoder_step_args);
        default: return -1;
    }
}

const char* mb_last_error(void) { return g_err; }

int mb_init(int ordinal) {
    clear_error();
    if (g.inited) {
        if (g.device == ordinal) return MB_OK;
        return fail(MB_E_STATE, "already initialised on device %d", g.device);
    }
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0)
        return fail(MB_E_NO_DEVICE, "no HIP device available (%s)",
                    e != hipSuccess ? hipGetErrorString(e) : "count=0");
    if (ordinal < 0 || ordinal >= count)
        return fail(MB_E_NO_DEVICE, "device ordinal %d out of range (%d devices)", ordinal, count);
    hipDeviceProp_t p;
    MB_HIP_TRY(hipGetDeviceProperties(&p, ordinal));
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return fail(MB_E_NO_DEVICE, "device %d is %s; this library is built for gfx950 only",
                    ordinal, p.gcnArchName);
    MB_HIP_TRY(hipSetDevice(ordinal));
    MB_HIP_TRY(hipStreamCreate(&g.lib_stream));
    g.device = ordinal;
    g.cu_count = (uint32_t)p.multiProcessorCount;
    g.inited = true;
    (void)registry();
    // The allocation-free decoder entry point's scratch address on this
    // device; if the lookup fails here, that entry point retries it on its
    // first call and reports the error there.
    if (init_decoder_scratch() != MB_OK) clear_error();
    return MB_OK;
}

int mb_shutdown(void) {
    clear_error();
    if (!g.inited) return MB_OK;
    (void)hipDeviceSynchronize();
    if (g.ws) (void)hipFree(g.ws);
    if (g.flush) (void)hipFree(g.flush);
    if (g.lib_stream) (void)hipStreamDestroy(g.lib_stream);
    g = State{};
    return MB_OK;
}

int mb_device_info_get(mb_device_info* out) {
    clear_error();
    if (!out) return fail(MB_E_ARG, "null output pointer");
    if (!g.inited) return fail(MB_E_STATE, "mb_init() has not been called");
    hipDeviceProp_t p;
    MB_HIP_TRY(hipGetDeviceProperties(&p, g.device));
    memset(out, 0, sizeof(*out));
    snprintf(out->name, sizeof(out->name), "%s", p.name);
    // Without libdrm's amdgpu.ids table HIP reports the generic "AMD Radeon
    // Graphics".  gfx950 parts are the MI350X (2.2 GHz) and MI355X (2.4 GHz).
    if (strstr(p.name, "Radeon Graphics") && strncmp(p.gcnArchName, "gfx950", 6) == 0)
        snprintf(out->name, sizeof(out->name), "%s",
                 p.clockRate >= 2400000 ? "AMD Instinct MI355X" : "AMD Instinct MI350X");
    snprintf(out->arch, sizeof(out->arch), "%s", p.gcnArchName);
    out->ordinal = g.device;
    out->cu_count = p.multiProcessorCount;
    out->clock_khz = p.clockRate;
    out->mem_clock_khz = p.memoryClockRate;
    out->mem_bus_width = p.memoryBusWidth;
    out->warp_size = p.warpSize;
    out->hbm_bytes = p.totalGlobalMem;
    out->lds_per_block = p.sharedMemPerBlock;
    out->lds_per_cu = p.maxSharedMemoryPerMultiProcessor;
    out->l2_bytes = (uint64_t)p.l2CacheSize;
    out->max_threads_per_block = p.maxThreadsPerBlock;
    out->regs_per_block = p.regsPerBlock;
    return MB_OK;
}

int mb_set_stream(void* hip_stream) {
    clear_error();
    if (!g.inited) return fail(MB_E_STATE, "mb_init() has not been called");
    g.user_stream = static_cast<hipStream_t>(hip_stream);
    return MB_OK;
}

int mb_kernel_count(void) { return (int)registry().size(); }

const char* mb_kernel_name(int id) {
    auto& t = registry();
    if (id < 0 || id >= (int)t.size()) return nullptr;
    return t[id].name;
}

int mb_kernel_find(const char* function, int* id) {
    clear_error();
    if (!function || !id) return fail(MB_E_ARG, "null argument");
    auto& t = registry();
    for (size_t i = 0; i < t.size(); ++i)
        if (strcmp(t[i].name, function) == 0) { *id = (int)i; return MB_OK; }
    return fail(MB_E_NOT_FOUND, "function %s not found", function);
}

int mb_kernel_attrs_get(int id, mb_kernel_attrs* out) {
    clear_error();
    if (!out) return fail(MB_E_ARG, "null output pointer");
    auto& t = registry();
    if (id < 0 || id >= (int)t.size()) return fail(MB_E_NOT_FOUND, "kernel id %d not found", id);
    if (!g.inited) return fail(MB_E_STATE, "mb_init() has not been called");
    hipFuncAttributes a;
    MB_HIP_TRY(hipFuncGetAttributes(&a, t[id].dominant_kernel));
    memset(out, 0, sizeof(*out));
    out->static_lds_bytes = a.sharedSizeBytes;
    out->max_threads_per_block = a.maxThreadsPerBlock;
    out->num_regs = a.numRegs;
    out->private_bytes = a.localSizeBytes;
    out->n_parts = t[id].n_parts;
    out->dominant_part = 0;
    out->arch_vgprs = out->agprs = out->sgprs = out->waves_per_simd = -1;
    if (const KernelResources* r = resources_of(hipKernelNameRefByPtr(t[id].dominant_kernel, nullptr))) {
        out->arch_vgprs = r->arch_vgprs;
        out->agprs = r->agprs;
        out->sgprs = r->sgprs;
        out->waves_per_simd = waves_per_simd(r->arch_vgprs, r->agprs, a.sharedSizeBytes,
                                             a.maxThreadsPerBlock);
    }
    return MB_OK;
}

int mb_run(int id, const mb_binding* bindings, int n_bindings, int warmup, int iters,
           uint32_t flags, mb_timing* out) {
    clear_error();
    if (!g.inited) return fail(MB_E_STATE, "mb_init() has not been called");
    auto& t = registry();
    if (id < 0 || id >= (int)t.size()) return fail(MB_E_NOT_FOUND, "kernel id %d not found", id);
    if (!out) return fail(MB_E_ARG, "null timing pointer");
    if (n_bindings < 0 || (n_bindings > 0 && !bindings))
        return fail(MB_E_ARG, "bad bindings array");
    if (warmup < 0) warmup = 0;
    if (iters <= 0) iters = 1;   // reference timing.mm:135
    const bool cold = flags & MB_RUN_COLD;
    if (cold && (flags & MB_RUN_WALL_ONLY))
        return fail(MB_E_ARG, "MB_RUN_COLD needs event timing: not with MB_RUN_WALL_ONLY");

    Bindings bs;
    for (int i = 0; i < n_bindings; ++i) {
        const mb_binding& b = bindings[i];
        if (b.index >= 32) return fail(MB_E_BINDING, "binding index %u >= 32", b.index);
        if (b.role > MB_ROLE_SCALAR) return fail(MB_E_BINDING, "unknown buffer role %u", b.role);
        if (bs.slot[b.index]) return fail(MB_E_BINDING, "binding %u bound twice", b.index);
        bs.slot[b.index] = &b;
    }
    const KernelEntry& k = t[id];
    hipStream_t s = stream_or_default(nullptr);

    for (int i = 0; i < warmup; ++i) {
        int rc = k.launch(bs, s, nullptr);
        if (rc) return rc;
    }
    MB_HIP_TRY(hipStreamSynchronize(s));

    if (flags & MB_RUN_WALL_ONLY) {   // no events: launches back to back, one sync
        auto w0 = std::chrono::steady_clock::now();
        for (int it = 0; it < iters; ++it) {
            int rc = k.launch(bs, s, nullptr);
            if (rc) return rc;
        }
        hipError_t r = hipStreamSynchronize(s);
        if (r != hipSuccess) return fail(MB_E_HIP, "kernel execution failed: %s", hipGetErrorString(r));
        const double wall = std::chrono::duration<double, std::milli>(
                                std::chrono::steady_clock::now() - w0).count();
        memset(out, 0, sizeof(*out));
        out->iters = iters;
        out->wall_ms = wall;
        out->min_ms = out->median_ms = out->mean_ms = wall / iters;
        return MB_OK;
    }
    const bool pipelined = flags & MB_RUN_PIPELINED;
    const bool parts = (flags & MB_RUN_PARTS) && k.n_parts > 1;
    const int np = parts ? std::min(k.n_parts, MB_MAX_PARTS) : 0;
    // Events per iteration: the region's start, np part starts, np part stops
    // (used by parts that time their own kernel) and the region's stop.
    const int per_iter = 2 + (np > 1 ? 2 * np : 0);
    const int n_ev = pipelined ? per_iter * iters : per_iter;
    std::vector<hipEvent_t> ev(n_ev);
    for (auto& e : ev) MB_HIP_TRY(hipEventCreate(&e));
    auto destroy = [&] { for (auto& e : ev) (void)hipEventDestroy(e); };

    std::vector<double> times(iters);
    std::vector<std::vector<double>> part_times(np, std::vector<double>(iters));
    const char* part_names[MB_MAX_PARTS] = {};
    bool part_own[MB_MAX_PARTS] = {};

    auto collect = [&](hipEvent_t* e, int it) -> int {
        float ms = 0.f;
        hipError_t r = hipEventElapsedTime(&ms, e[0], e[per_iter - 1]);
        if (r != hipSuccess) return fail(MB_E_HIP, "hipEventElapsedTime: %s", hipGetErrorString(r));
        times[it] = ms;
        for (int p = 0; p < np; ++p) {
            // a part timed by its kernel's own events runs from that kernel's
            // start to its end; a marked part from its start to the next
            // part's start (the region's stop for the last)
            hipEvent_t a = e[1 + p];
            hipEvent_t b = part_own[p] ? e[1 + np + p] : p == np - 1 ? e[per_iter - 1] : e[2 + p];
            r = hipEventElapsedTime(&ms, a, b);
            if (r != hipSuccess) return fail(MB_E_HIP, "hipEventElapsedTime: %s", hipGetErrorString(r));
            part_times[p][it] = ms;
        }
        return MB_OK;
    };

    auto wall0 = std::chrono::steady_clock::now();
    for (int it = 0; it < iters; ++it) {
        hipEvent_t* e = pipelined ? &ev[(size_t)it * per_iter] : ev.data();
        if (cold) {   // evict the caches, outside the event pair
            int rc = launch_cache_eviction(s);
            if (rc) { destroy(); return rc; }
        }
        hipError_t r = hipEventRecord(e[0], s);
        if (r != hipSuccess) { destroy(); return fail(MB_E_HIP, "hipEventRecord: %s", hipGetErrorString(r)); }
        PartMarks pm;
        if (np > 1) { pm.events = e + 1; pm.stops = e + 1 + np; pm.n_max = np; }
        int rc = k.launch(bs, s, np > 1 ? &pm : nullptr);
        if (rc) { destroy(); return rc; }
        if (np > 1 && pm.n < np) {   // a part that was never started has no events
            destroy();
            return fail(MB_E_HIP, "kernel %s started %d of its %d timed parts", k.name, pm.n, np);
        }
        if (np > 1)
            for (int p = 0; p < np; ++p) { part_names[p] = pm.names[p]; part_own[p] = pm.own_kernel[p]; }
        r = hipEventRecord(e[per_iter - 1], s);
        if (r != hipSuccess) { destroy(); return fail(MB_E_HIP, "hipEventRecord: %s", hipGetErrorString(r)); }
        if (!pipelined) {
            r = hipEventSynchronize(e[per_iter - 1]);
            if (r != hipSuccess) { destroy(); return fail(MB_E_HIP, "kernel execution failed: %s", hipGetErrorString(r)); }
            rc = collect(e, it);
            if (rc) { destroy(); return rc; }
        }
    }
    if (pipelined) {
        hipError_t r = hipStreamSynchronize(s);
        if (r != hipSuccess) { destroy(); return fail(MB_E_HIP, "kernel execution failed: %s", hipGetErrorString(r)); }
        for (int it = 0; it < iters; ++it) {
            int rc = collect(&ev[(size_t)it * per_iter], it);
            if (rc) { destroy(); return rc; }
        }
    }
    auto wall1 = std::chrono::steady_clock::now();
    destroy();

    memset(out, 0, sizeof(*out));
    auto stats = [](std::vector<double> v, double* mn, double* med, double* mean) {
        std::sort(v.begin(), v.end());
        double sum = 0;
        for (double x : v) sum += x;
        *mn = v.front();
        *med = v[v.size() / 2];
        *mean = sum / (double)v.size();
    };
    stats(times, &out->min_ms, &out->median_ms, &out->mean_ms);
    out->iters = iters;
    out->n_parts = np;
    for (int p = 0; p < np; ++p) {
        double mn;
        stats(part_times[p], &mn, &out->part_median_ms[p], &out->part_mean_ms[p]);
        snprintf(out->part_names[p], sizeof(out->part_names[p]), "%s",
                 part_names[p] ? part_names[p] : "?");
    }
    out->wall_ms = std::chrono::duration<double, std::milli>(wall1 - wall0).count();
    return MB_OK;
}

}  // extern "C"
