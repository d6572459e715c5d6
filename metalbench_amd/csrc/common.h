// Internal declarations shared by the libmbhip.so translation units.
// Nothing here is part of the C ABI (that is include/mbhip.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>

#include "../../include/mbhip.h"

namespace mb {

// ---- errors ---------------------------------------------------------------
// Records `msg` for mb_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

#define MB_HIP_TRY(expr)                                                     \
    do {                                                                     \
        hipError_t _e = (expr);                                              \
        if (_e != hipSuccess)                                                \
            return ::mb::fail(MB_E_HIP, "%s failed: %s (%s:%d)", #expr,      \
                              hipGetErrorString(_e), __FILE__, __LINE__);    \
    } while (0)

// Checks the launch that was just enqueued.
#define MB_LAUNCH_CHECK(name)                                                \
    do {                                                                     \
        hipError_t _e = hipGetLastError();                                   \
        if (_e != hipSuccess)                                                \
            return ::mb::fail(MB_E_HIP, "launch of %s failed: %s", name,     \
                              hipGetErrorString(_e));                        \
    } while (0)

// ---- library state ----------------------------------------------------------
bool initialized();
hipStream_t stream_or_default(void* s);   // NULL -> current library stream
uint32_t device_cu_count();               // compute units of the initialised device

// Library-owned device workspace, grown on demand, freed by mb_shutdown().
// Its contents are undefined when handed out: a kernel that needs zeroed
// counters clears them itself.  Returns nullptr (and sets the error) on
// failure.
void* library_workspace(size_t bytes);

// Library-owned buffer twice the size of the memory-side cache, allocated on
// first use and freed by mb_shutdown(); writing it evicts every cache level.
void* library_flush_buffer(size_t* bytes);
// Enqueue that eviction on `s` (copy.hip).
int launch_cache_eviction(hipStream_t s);

// ---- per-kernel timing marks ---------------------------------------------------
// A multi-kernel entry names each part right before enqueuing it, in one of
// two ways.  mark(name): when timing parts, mb_run records an event there,
// and the part runs to the next part's start (so it includes the dispatch
// gap before the next kernel).  kernel(name, &start, &stop): the entry
// launches the part's one kernel with hipExtLaunchKernel and these events,
// which take that kernel's own start and end times (no extra packet between
// kernels), or with a plain launch when both come back null.
struct PartMarks {
    hipEvent_t* events = nullptr;   // n_max start events, or nullptr
    hipEvent_t* stops = nullptr;    // n_max stop events (kernel parts)
    int n_max = 0;
    int n = 0;
    const char* names[MB_MAX_PARTS] = {};
    bool own_kernel[MB_MAX_PARTS] = {};   // part timed by its kernel's own events
    void mark(hipStream_t s, const char* name) {
        if (n < MB_MAX_PARTS) names[n] = name;
        if (events && n < n_max) (void)hipEventRecord(events[n], s);
        ++n;
    }
    void kernel(const char* name, hipEvent_t* start, hipEvent_t* stop) {
        *start = *stop = nullptr;
        if (n < MB_MAX_PARTS) names[n] = name;
        if (events && stops && n < n_max) {
            *start = events[n];
            *stop = stops[n];
            own_kernel[n] = true;
        }
        ++n;
    }
};

// ---- bindings ---------------------------------------------------------------
struct Bindings {
    const mb_binding* slot[32] = {};
    // Fetch binding `idx` and check role, dtype and (if min_bytes > 0) size.
    int buffer(uint32_t idx, uint32_t dtype, uint64_t min_bytes, bool output,
               void** ptr, const char* what) const;
    int u32(uint32_t idx, uint32_t* v, const char* what) const;
    int f32(uint32_t idx, float* v, const char* what) const;
    // Byte size of buffer binding `idx` (0 if it is missing or not a buffer).
    uint64_t nbytes(uint32_t idx) const;
};

// One registry entry: the `metal_function` name and its launcher.
struct KernelEntry {
    const char* name;
    int (*launch)(const Bindings&, hipStream_t, PartMarks*);
    const void* dominant_kernel;   // device function for hipFuncGetAttributes
    int n_parts;
};

// Registration hooks, one per translation unit (called in a fixed order).
void register_kernel(const KernelEntry& e);
void register_transpose();
void register_copy();
void register_gemm_f32();
void register_conv2d();
void register_gemm_bf16();
void register_decoder();
// Looks up the allocation-free decoder entry point's device scratch on the
// current device (decoder.hip); mb_init() calls it once the device is set.
int init_decoder_scratch();
void register_transformer_f32();

static inline uint32_t cdiv(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

// ---- fp32 GEMM family (gemm_f32.hip), shared with the transformer kernels ----
// C[b] = A[b] @ B[b] (row-major, leading dimensions lda/ldb/ldc), batch b at
// blockIdx.y with element strides batch_*.  Kinds:
//   PLAIN       C = A B
//   RMS         C = rmsnorm(A) B            (row scale rsqrt(mean(A_row^2) + eps), K = row length)
//   RMS_BT      C = rmsnorm(A) B^T, B [N][K]
//   RESID       C = A B + R                 (R [M][N], leading dimension ldr)
//   SWIGLU      C = silu(A B) * (A B2)
//   RMS_SWIGLU  C = silu(rmsnorm(A) B) * (rmsnorm(A) B2)
struct GemmF32Args {
    const float* a;
    const float* b;
    const float* b2;
    float* c;
    const float* r;
    uint32_t m, n, k, lda, ldb, ldc, ldr, tiles_n;
    uint64_t batch_a, batch_b, batch_c;
    float eps;
};
enum GemmF32Kind {
    GEMM_F32_PLAIN, GEMM_F32_RMS, GEMM_F32_RMS_BT, GEMM_F32_RESID, GEMM_F32_SWIGLU,
    GEMM_F32_RMS_SWIGLU
};
// ---- global -> LDS DMA ------------------------------------------------------
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;

// Buffer descriptor in SGPRs (raw, stride 0) for dma16.
__device__ __forceinline__ i32x4 dma_rsrc(const void* p, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(p);
    return i32x4{(int32_t)__builtin_amdgcn_readfirstlane((uint32_t)a),
                 (int32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32) & 0xffffu),
                 (int32_t)__builtin_amdgcn_readfirstlane(bytes), 0x00020000};
}

// 16 bytes per lane global -> LDS (lane l lands at lds_addr + 16 l).  Written
// as asm so that the compiler's wait-count pass, which cannot tell which LDS
// buffer a DMA targets, does not add vmcnt(0) before every LDS read; callers
// wait for their DMAs themselves (s_waitcnt vmcnt) and publish them with a
// barrier.
__device__ __forceinline__ void dma16(i32x4 rsrc, uint32_t lds_addr, uint32_t voff, uint32_t soff) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :: "s"(lds_addr), "v"(voff), "s"(rsrc), "s"(soff) : "m0");
}

// Workgroup barrier that orders LDS only (lgkmcnt + s_barrier): global loads
// and DMAs in flight stay in flight.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Tile (tm, tn) of hardware block b in a tiles_m x tiles_n grid, XCD-aware.
// The hardware dispatches block b to XCD b % 8, and each XCD has its own L2.
// When the grid is a multiple of 8, each XCD takes a contiguous range of
// logical tiles; logical tiles walk bands of `band` tile-rows in column order.
// The tiles one XCD runs at a time then share `band` A panels and few B
// panels in its L2.
__device__ __forceinline__ void xcd_band_tile(uint32_t b, uint32_t nblocks, uint32_t tiles_m,
                                              uint32_t tiles_n, uint32_t band, uint32_t* tm,
                                              uint32_t* tn) {
    uint32_t L = b;
    if ((nblocks & 7) == 0) L = (b & 7) * (nblocks >> 3) + (b >> 3);
    const uint32_t per_group = band * tiles_n;
    const uint32_t group = L / per_group;
    const uint32_t first_m = group * band;
    const uint32_t gsize = min(tiles_m - first_m, band);
    const uint32_t in_group = L - group * per_group;
    *tm = first_m + in_group % gsize;
    *tn = in_group / gsize;
}

// LDS address of a __shared__ object.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const lds_void_t*)p;
}

// Dense row-major defaults: lda = k, ldb = ldc = ldr = n, no batch stride.
GemmF32Args gemm_f32_args(const float* a, const float* b, float* c, uint32_t m, uint32_t n,
                          uint32_t k);
int launch_gemm_f32_ex(GemmF32Args g, GemmF32Kind kind, uint32_t batch, hipStream_t s);

}  // namespace mb
