/*
 * mbhip.h — C ABI of libmbhip.so, the gfx950 (MI355X) kernel library behind
 * the MetalBench kernel registry.
 *
 * The reference crosses a process boundary: the harness writes a JSON
 * manifest plus raw .bin inputs, runs `build/metalbench_host --manifest m.json`
 * and reads one JSON line back (reference mlx/scripts/harness.py:36-49,
 * metal/scripts/main.mm:73-197).  This library replaces that host binary with
 * an in-process C ABI: plain pointers and sizes, no torch or C++ types.
 *
 * Ownership: the caller owns every device buffer it passes in.  The library
 * never allocates or frees caller memory; it owns its stream, its events and,
 * for multi-kernel entries, an internal workspace that mb_shutdown() releases.
 *
 * Errors: every call returns MB_OK (0) or a negative MB_E_* code and leaves a
 * message in a thread-local buffer read by mb_last_error().  This replaces the
 * host's `die()` -> stderr + exit 1 (reference metal/scripts/main.mm:28-32).
 *
 * Threading: synchronous entry points (mb_run) return after the GPU finished;
 * one in-flight mb_run per process; not re-entrant.  The mb_launch_* entry
 * points only enqueue work on the given stream and return immediately.
 */
#ifndef MBHIP_H
#define MBHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MBHIP_ABI_VERSION 2

/* ---- status codes ------------------------------------------------------- */
#define MB_OK             0
#define MB_E_NO_DEVICE   -1  /* no HIP device / wrong ordinal / not gfx950   */
#define MB_E_NOT_FOUND   -2  /* unknown kernel name or id                    */
#define MB_E_BINDING     -3  /* missing/duplicate binding, wrong role or size */
#define MB_E_DTYPE       -4  /* wrong dtype for a binding or scalar          */
#define MB_E_HIP         -5  /* a HIP runtime call failed                    */
#define MB_E_STATE       -6  /* mb_init() not called / already shut down     */
#define MB_E_ARG         -7  /* invalid argument (null pointer, bad shape)   */

/* ---- binding roles and dtypes (reference mlx_helpers.py:83-89, 299-312) -- */
#define MB_ROLE_INPUT   0
#define MB_ROLE_OUTPUT  1
#define MB_ROLE_SCALAR  2

#define MB_DTYPE_F32   0
#define MB_DTYPE_F16   1
#define MB_DTYPE_I32   2
#define MB_DTYPE_U32   3
#define MB_DTYPE_BF16  4   /* new: the reference has no bf16 */

/* One buffer or scalar bound at a Metal-style binding index.  Mirrors one
 * element of the manifest's "buffers" list (reference
 * mlx/scripts/mlx_helpers.py:299-312; metal/scripts/main.mm:129-159): an input
 * or output is a device pointer plus its byte size, a scalar is a 4-byte
 * u32/i32/f32 value. */
typedef struct mb_binding {
    uint32_t index;        /* binding slot, < 32                       */
    uint32_t role;         /* MB_ROLE_*                                */
    void*    dev_ptr;      /* device pointer (input/output), else NULL */
    uint64_t nbytes;       /* byte size of the buffer (input/output)   */
    uint32_t dtype;        /* MB_DTYPE_*                               */
    uint32_t _pad;
    union { uint32_t u32; int32_t i32; float f32; } scalar;
    uint32_t _pad2;
} mb_binding;

#define MB_MAX_PARTS 8

/* Timing of one mb_run: GPU time per iteration from a hipEvent pair on the
 * library stream; min / median (= sorted[n/2]) / mean over `iters`, the
 * statistics of reference metal/scripts/timing.mm:150-159 (TimingResult,
 * timing.h:24-33).  Multi-kernel entries also report per-kernel ("part")
 * times when MB_RUN_PARTS is set: for the decode step each kernel's own
 * start-to-end time (hipExtLaunchKernel events, nothing enqueued between the
 * kernels), for the others the time from one kernel's start to the next's
 * (so it includes the dispatch gap). */
typedef struct mb_timing {
    double  min_ms;
    double  median_ms;
    double  mean_ms;
    int32_t iters;
    int32_t n_parts;
    double  part_median_ms[MB_MAX_PARTS];
    double  part_mean_ms[MB_MAX_PARTS];
    char    part_names[MB_MAX_PARTS][48];
    double  wall_ms;       /* host wall clock around the timed loop */
} mb_timing;

/* mb_run flags */
#define MB_RUN_SYNC_EACH  0u  /* event pair + host sync per iteration (reference dispatchOnce) */
#define MB_RUN_PIPELINED  1u  /* event pairs per iteration, one host sync at the end           */
#define MB_RUN_PARTS      2u  /* also time each kernel of a multi-kernel entry                 */
#define MB_RUN_WALL_ONLY  4u  /* no events: iters launches back to back, one host sync; every
                                 statistic = host wall clock / iters (throughput timing)       */
#define MB_RUN_COLD       8u  /* before each timed dispatch, outside its event pair, write a
                                 library-owned 512 MiB buffer so no cache level (L2, the
                                 256 MB memory-side cache) holds the kernel's inputs: the
                                 harness's --cold-start (reference mlx/scripts/harness.py:403,
                                 metal/scripts/timing.mm:236-246 purgeMetalCaches).  Not
                                 with MB_RUN_WALL_ONLY.                                        */

/* Device description; replaces detect_chip()/MChip (reference
 * metal/scripts/setup.h:26-46, setup.cpp:116-136). */
typedef struct mb_device_info {
    char     name[256];          /* e.g. "AMD Instinct MI355X"         */
    char     arch[64];           /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    int32_t  ordinal;
    int32_t  cu_count;
    int32_t  clock_khz;          /* peak shader clock                  */
    int32_t  mem_clock_khz;
    int32_t  mem_bus_width;
    int32_t  warp_size;
    uint64_t hbm_bytes;
    uint64_t lds_per_block;
    uint64_t lds_per_cu;
    uint64_t l2_bytes;
    int32_t  max_threads_per_block;
    int32_t  regs_per_block;
} mb_device_info;

/* Kernel attributes; replaces the PSO's staticThreadgroupMemoryLength and
 * maxTotalThreadsPerThreadgroup (reference metal/scripts/main.mm:119-123,
 * 186-192).  For multi-kernel entries they describe the dominant kernel.
 * The register counts come from this library's own code objects (metadata
 * note and kernel descriptor, read at build time); -1 if not found. */
typedef struct mb_kernel_attrs {
    uint64_t static_lds_bytes;
    int32_t  max_threads_per_block;
    int32_t  num_regs;           /* VGPRs per thread as reported by HIP */
    uint64_t private_bytes;      /* per-thread scratch (spills); 0 is good */
    int32_t  n_parts;            /* kernels launched per dispatch       */
    int32_t  dominant_part;
    int32_t  arch_vgprs;         /* architectural VGPRs per lane        */
    int32_t  agprs;              /* accumulation VGPRs (MFMA) per lane  */
    int32_t  sgprs;              /* scalar registers per wave           */
    int32_t  waves_per_simd;     /* occupancy the registers and LDS allow (1..8) */
} mb_kernel_attrs;

/* ---- lifecycle ----------------------------------------------------------- */

/* Select device `ordinal`, check it is gfx950, create the library stream and
 * events.  Replaces MTLCreateSystemDefaultDevice + newCommandQueue (reference
 * metal/scripts/main.mm:102-117).  Returns MB_E_NO_DEVICE without a GPU. */
int mb_init(int ordinal);

/* Release the stream, events and workspace.  Safe to call twice. */
int mb_shutdown(void);

/* Message of the last failing call on this thread ("" if none). */
const char* mb_last_error(void);

/* ABI version (MBHIP_ABI_VERSION) — callable without a GPU. */
int mb_abi_version(void);

/* sizeof() of the ABI structs, so FFI bindings can check their layouts
 * without a GPU: which = 0 mb_binding, 1 mb_timing, 2 mb_device_info,
 * 3 mb_kernel_attrs, 4 mb_decoder_step_args; -1 for anything else. */
int mb_abi_struct_size(int which);

int mb_device_info_get(mb_device_info* out);

/* Make the library enqueue on `hip_stream` (a hipStream_t) instead of its own
 * stream; NULL restores the library stream. */
int mb_set_stream(void* hip_stream);

/* ---- kernel registry ------------------------------------------------------ */

/* Number of registered kernels and the `metal_function` name of each —
 * callable without a GPU. */
int         mb_kernel_count(void);
const char* mb_kernel_name(int id);

/* Look up a kernel by its registry `metal_function` name.  Replaces
 * newFunctionWithName + "function ... not found" (reference
 * metal/scripts/main.mm:110-112).  Callable without a GPU. */
int mb_kernel_find(const char* function, int* id);

int mb_kernel_attrs_get(int id, mb_kernel_attrs* out);

/* Bind, launch `warmup` untimed dispatches, then `iters` timed ones.
 * Replaces the host's binding loop + runTimedDispatches (reference
 * metal/scripts/main.mm:125-165; metal/scripts/timing.mm:125-193).  The
 * kernel derives its launch geometry from the scalar bindings; the
 * registry's grid/threadgroup are advisory.  Outputs hold the result of the
 * last dispatch on return. */
int mb_run(int id, const mb_binding* bindings, int n_bindings,
           int warmup, int iters, uint32_t flags, mb_timing* out);

/* ---- typed launchers (enqueue only; `stream` is a hipStream_t or NULL for
 *      the library stream) --------------------------------------------------- */

/* B[cols x rows] = A[rows x cols]^T, fp32, bit exact
 * (reference mlx/kernels/common/transpose_2d.py:10-11, registry.py:165-179). */
int mb_launch_transpose_2d_f32(const float* a, float* b,
                               uint32_t rows, uint32_t cols, void* stream);

/* C[M x N] = A[M x K] @ B[K x N], fp32 row-major, fp32 MFMA
 * (reference mlx/kernels/common/sqr_mm.py:10-11, registry.py:43-59,129). */
int mb_launch_matmul_f32(const float* a, const float* b, float* c,
                         uint32_t m, uint32_t n, uint32_t k, void* stream);

/* C[M x N] = bf16(A[M x K] @ B[K x N]), bf16 in/out (uint16 bit patterns),
 * fp32 accumulate, bf16 MFMA.  No reference kernel: the reference's matmul
 * spec (mlx/kernels/common/registry.py:43-59) at bf16. */
int mb_launch_matmul_bf16(const uint16_t* a, const uint16_t* b, uint16_t* c,
                          uint32_t m, uint32_t n, uint32_t k, void* stream);

/* y[N,P,Q,O] = conv2d(x[N,H,W,C], w[O,R,S,C]) cross-correlation, NHWC/OHWI,
 * fp32 MFMA implicit GEMM, zero padding `pad`, stride `stride`
 * (reference mlx/kernels/common/conv2d.py:11-12, registry.py:469-477). */
int mb_launch_conv2d_nhwc_f32(const float* x, const float* w, float* y,
                              uint32_t n, uint32_t h, uint32_t wd, uint32_t c,
                              uint32_t o, uint32_t r, uint32_t s,
                              uint32_t stride, uint32_t pad, void* stream);

/* One decode step of a LLaMA decoder layer (bf16 storage, fp32 math).
 *
 * Follows reference mlx/kernels/full/llama_decoder_layer.py:24-64 (RMSNorm
 * without gain, interleaved-pair RoPE, GQA with head h -> kv head h/G, softmax
 * attention, W_o + residual, RMSNorm, SwiGLU, W_down + residual) for ONE new
 * token per sequence that attends to `cache_len` cached positions plus itself:
 *   - the new token's position is cache_len; RoPE angle = pos * base^(-2i/Dh);
 *   - the cache holds keys that already carry their RoPE rotation;
 *   - weights are x @ W layouts: w_qkv [D][QD + 2*Hkv*Dh] with columns
 *     [Q | K | V], w_gu [D][2*FF] with columns [gate | up] (reference
 *     llama_decoder_layer.py:30-32, 43-44), QD = H * Dh.
 * For a whole layer QD = D.  QD < D runs the work of one GPU's share of a
 * tensor-parallel layer at its real shapes (its H query heads and Hkv kv
 * heads in w_qkv's columns, its QD rows of W_o, its FF columns of gate and up
 * and FF rows of W_down): a per-shard cost proxy for benchmarking, NOT a
 * building block of a tensor-parallel step.  The call still adds the full
 * residual x and normalises its own partial x1 = x + attn @ W_o, so the sum
 * of the shards' y is not the layer's output.  A real shard needs the step
 * split at W_o, with the all-reduce of attn @ W_o between the two halves, the
 * FFN's RMSNorm on the all-reduced x1, and each residual added on one rank
 * only; this library does not provide that split.
 * All tensors are row-major bf16 bit patterns.  The caches are read only; the
 * new token's RoPE'd key and its value are written to k_new / v_new so the
 * caller can append them. */
typedef struct mb_decoder_step_args {
    uint32_t batch;          /* B   sequences in the step          (16)    */
    uint32_t d_model;        /* D   residual width, a multiple of 128 (4096) */
    uint32_t n_heads;        /* H   query heads, H * Dh <= 16384   (32)   */
    uint32_t n_kv_heads;     /* Hkv                                (8)    */
    uint32_t head_dim;       /* Dh  (must be 128)                          */
    uint32_t d_ff;           /* FF                                (14336) */
    uint32_t cache_len;      /* L   cached positions = new token position  */
    uint32_t cache_stride;   /* positions allocated per (b, kv head), >= L */
    float    rope_base;      /* 500000                                      */
    float    eps;            /* 1e-5                                        */
    const uint16_t* x;       /* [B][D]                                     */
    const uint16_t* w_qkv;   /* [D][QD + 2*Hkv*Dh]                         */
    const uint16_t* w_o;     /* [QD][D]                                    */
    const uint16_t* w_gu;    /* [D][2*FF]                                  */
    const uint16_t* w_down;  /* [FF][D]                                    */
    const uint16_t* k_cache; /* [B][Hkv][cache_stride][Dh]                 */
    const uint16_t* v_cache; /* [B][Hkv][cache_stride][Dh]                 */
    uint16_t* y;             /* [B][D]   output hidden state               */
    uint16_t* k_new;         /* [B][Hkv][Dh]  RoPE'd key of the new token  */
    uint16_t* v_new;         /* [B][Hkv][Dh]  value of the new token       */
    void*     workspace;     /* device scratch, see mb_decoder_step_workspace_bytes() */
    uint64_t  workspace_bytes;
} mb_decoder_step_args;

/* Workspace bytes mb_launch_llama_decoder_step_bf16 needs for these shapes
 * (0 and mb_last_error() set if the shapes are unsupported).  A caller-owned
 * workspace needs no initialisation: each step's first kernel clears the
 * completion counters the others use.  Calls sharing one workspace must not
 * overlap.  Callable without a GPU. */
uint64_t mb_decoder_step_workspace_bytes(const mb_decoder_step_args* args);

/* Enqueue one decode step.  `args->workspace` may be NULL: the library then
 * uses (and grows) its own workspace. */
int mb_launch_llama_decoder_step_bf16(const mb_decoder_step_args* args, void* stream);

/* The same decode step, allocating nothing.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory during the call (code
 * under HIP graph capture, allocation-free serving loops, harnesses that
 * forbid hipMalloc).  The workspace is a static device array of
 * MB_DECODER_NOALLOC_MAX_BYTES carried by the library's code object (one per
 * device, held until the process ends), so `args->workspace` must be NULL;
 * shapes whose mb_decoder_step_workspace_bytes() exceeds the limit are
 * rejected with MB_E_ARG.  Results are bit-identical to
 * mb_launch_llama_decoder_step_bf16.  Every call on a device shares that
 * device's scratch and a call leaves its intermediates there: calls that
 * overlap on one device (two streams, two threads) race.  A HIP graph that
 * captured a call may be replayed after calls of other shapes: each step
 * clears its own completion counters. */
#define MB_DECODER_NOALLOC_MAX_BYTES (32u << 20)
int mb_launch_llama_decoder_step_bf16_noalloc(const mb_decoder_step_args* args, void* stream);

/* Plain fp32 copy dst[i] = src[i]: the calibration kernel for HBM traffic
 * counters and the measured-bandwidth ceiling.  No reference counterpart. */
int mb_launch_copy_f32(const float* src, float* dst, uint64_t n, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* MBHIP_H */
