// One decode step of a LLaMA decoder layer, bf16 storage / fp32 math.
//
// Spec: reference mlx/kernels/full/llama_decoder_layer.py:24-64 applied to one
// new token per sequence (see include/mbhip.h, mb_decoder_step_args):
//   h  = x * rsqrt(mean(x^2) + eps)                              (:48-50, no gain)
//   q|k|v = h @ W_qkv; q, k rotated by interleaved-pair RoPE at pos = L (:52-64)
//   attn = softmax(q k^T / sqrt(Dh)) v over L cached keys + the new key,
//          query head h reading kv head h / G                    (:30-36, mx.repeat)
//   x1 = x + attn @ W_o                                          (:37-38)
//   y  = x1 + (silu(h2 W_gate) * h2 W_up) @ W_down, h2 = rmsnorm(x1)   (:41-46)
//
// The step is HBM bound (436 MB of weights + 134 MB of KV cache per step at
// B = 16, L = 2048 against ~7.5 GFLOP), so every kernel is shaped to stream
// its bytes once:
//   1. qkv            skinny GEMM x @ W_qkv that leaves its split-K partials
//                     and per-split sums of x^2 (gathered from the A operand
//                     for free); no finisher;
//   2. attention      flash-decoding: one workgroup per (sequence, kv head,
//                     split of the cached keys).  Its prologue sums the QKV
//                     partials of its heads, applies the RMSNorm row scale
//                     and RoPE (q pre-scaled by 1/sqrt(Dh), bf16; k_new and
//                     v_new bf16, written out by split 0) while the first
//                     K/V block is in flight; q.k^T on MFMA, online softmax,
//                     p.v on VALU; the last split to finish merges the splits
//                     and the new token (log-sum-exp);
//   3. wo_residual    skinny GEMM attn @ W_o, finisher adds x, writes x1
//                     (fp32 + bf16) and per-tile sums of x1^2;
//   4. gate_up_swiglu skinny GEMM x1 @ [W_gate | W_up], each tile holding 256
//                     gate and the matching 256 up columns, finisher applies
//                     the RMSNorm scale and silu(g) * u;
//                     x1 and the SwiGLU output feed the next GEMMs as hi + lo
//                     bf16 pairs (two MFMAs), so their bf16 rounding does not
//                     accumulate over K = 4096 / 14336 terms;
//   5. down_residual  skinny GEMM act @ W_down, finisher adds x1, writes y.
// RMSNorm is a per-row scale, so (r x) W = r (x W): it is applied to the GEMM
// outputs instead of materialising h / h2.
//
// Skinny GEMM (M = batch <= 16): about one workgroup per CU, each owning a
// column tile and one K split, streams its weights through a ring of register
// slots straight into the MFMA B operand (an 8 x 8 register transpose, no LDS
// on the weight path); weights are loaded non-temporal (each byte is read
// once per step).  Split-K partials go to the workspace and the LAST
// workgroup of each column tile (an atomic counter, reset by that workgroup)
// sums them in split order and runs the epilogue; the partials travel through
// device-coherent (sc1) accesses, not fences.  The QKV GEMM has no finisher:
// its partials are summed, in the same order, by the attention kernel that
// reads them.  Details at skinny_gemm_kernel.
#include "common.h"

#include <hip/hip_ext.h>

#include <math.h>

#include <algorithm>
#include <mutex>

namespace mb {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int DH = 128;        // head_dim (fixed)
constexpr int MROWS = 16;      // MFMA rows = max batch
constexpr int BN = 128;        // skinny GEMM column tile (W_gate | W_up: up to 4 x BN)
constexpr int KS = 128;        // k rows of a skinny-GEMM unit with 128-column tiles
constexpr int RING = 2;        // skinny GEMM: units in flight per workgroup
constexpr int MAXG = 16;       // query heads per kv head (MFMA columns)
constexpr float LOG2E = 1.4426950408889634f;

enum { EPI_QKV = 0, EPI_WO = 1, EPI_GU = 2, EPI_DOWN = 3 };


typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Two floats -> a packed bf16 pair (a in the low half), round to nearest even
// (one v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

// hi + lo bf16 terms of a pair: hi = bf16(v), lo = bf16(v - hi).
__device__ __forceinline__ void split_bf16(float a, float b, uint32_t& hi, uint32_t& lo) {
    hi = pack_bf16(a, b);
    lo = pack_bf16(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xffff0000u));
}

// silu(v) = v / (1 + e^-v) with the hardware exp2 and reciprocal (about 1 ulp
// each); e^-v overflowing to inf gives v * 0 = -0 for very negative v.
__device__ __forceinline__ float silu(float v) {
    return v * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-v * LOG2E));
}

// ---- cross-workgroup hand-off without L2 flushes ---------------------------------
// MI355X has one L2 per XCD; an agent-scope fence (__threadfence) writes back
// and invalidates the whole local L2, which at thousands of workgroups per
// kernel costs more than the kernel itself.  Data one workgroup hands to
// another inside a kernel (split-K partials, attention chunk partials) is
// therefore written and read with device-coherent (sc1) buffer accesses, which
// write through to / read from the coherence point, so no cached copy is ever
// trusted:
//   writer: sc1 stores; s_waitcnt (every store acknowledged); barrier;
//           one relaxed agent-scope atomicAdd on the tile's counter;
//   reader: the workgroup that brought the counter to its final value reads
//           every partial with sc1 loads.
constexpr int CPOL_SC1 = 16;                  // cache policy: sc1 (device coherent)
constexpr int CPOL_NT = 2;                    // cache policy: nt (streamed, read once per step)
constexpr uint32_t RSRC_FLAGS = 0x00020000u;  // buffer descriptor word 3: 32-bit data format

__device__ __forceinline__ __amdgpu_buffer_rsrc_t coherent_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, RSRC_FLAGS);
}
__device__ __forceinline__ void st_sc1(__amdgpu_buffer_rsrc_t r, uint32_t off, f32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, CPOL_SC1);
}
__device__ __forceinline__ void st_sc1(__amdgpu_buffer_rsrc_t r, uint32_t off, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, off, 0, CPOL_SC1);
}
__device__ __forceinline__ f32x4 ld4_sc1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, CPOL_SC1));
}
__device__ __forceinline__ float ld_sc1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, CPOL_SC1));
}

// A workgroup-uniform pointer or size, kept in SGPRs (buffer descriptors built
// from it then need no waterfall loop around each load).
__device__ __forceinline__ void* uniform_ptr(const void* ptr) {
    const uint64_t v = reinterpret_cast<uint64_t>(ptr);
    const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<void*>((hi << 32) | lo);
}

// K splits of a skinny GEMM.  Every column tile has `splits` splits of kc
// rows, except the tiles of the slow class ((t & slow_mask) == slow_val),
// which, when splits_slow = splits + 1, have splits_slow splits of kc_slow
// rows.  Blocks 0 .. tiles * splits - 1 are (tile b % tiles, split b /
// tiles); the blocks after them are the last split of each slow tile, in
// tile order.  A tile's partials sit at stride() splits per tile.
struct SplitGeom {
    uint32_t tiles, splits, kc, splits_slow, kc_slow, slow_mask, slow_val;
    __host__ __device__ uint32_t stride() const { return splits_slow > splits ? splits_slow : splits; }
    __host__ __device__ bool slow(uint32_t t) const {
        return splits_slow > splits && (t & slow_mask) == slow_val;
    }
    __host__ __device__ uint32_t nsplits(uint32_t t) const { return slow(t) ? splits_slow : splits; }
    __host__ __device__ uint32_t kc_of(uint32_t t) const { return slow(t) ? kc_slow : kc; }
    __host__ __device__ void block(uint32_t b, uint32_t* t, uint32_t* sp) const {
        const uint32_t nbase = tiles * splits;
        if (b < nbase) { *t = b % tiles; *sp = b / tiles; }
        else { *t = (b - nbase) * (slow_mask + 1) + slow_val; *sp = splits; }
    }
};

// The first two K units of the next skinny GEMM's weights for one block
// index (w = nullptr: none; also for weights of 4 GB or more, which 32-bit
// buffer offsets do not reach).  Column tile t covers bytes [seg_bytes t,
// +seg_bytes) of every weight row, and for the paired gate | up tile also
// the same range seg2_off bytes further on.
struct NextUnits {
    const uint8_t* w;
    uint32_t bytes, ldw_bytes, k, ur, seg_bytes, seg2_off;
    SplitGeom sp;
};

// A workgroup that is not the last of its tile has nothing left to do while
// the last one sums the partials and runs the epilogue (1-3 us), and HBM is
// idle meanwhile.  It touches every 128-byte line of the next GEMM's first
// two units for its own block index, so that the next kernel's first loads
// find them in the 256 MB memory-side cache instead of HBM.  (Not in L2: L2
// does not keep them across the kernel boundary -- the L2-miss counter
// FETCH_SIZE counts those lines in both kernels.)  The wave waits for them
// before it ends, as it would at s_endpgm anyway.  Measured at the benchmark
// shape: 115.7-116.2 -> 113.3-113.9 us per step (three units: the same;
// four: slower).
__device__ __noinline__ void prefetch_next_units(const NextUnits c, uint32_t b) {
    if (!c.w) return;
    uint32_t tile, split;
    c.sp.block(b, &tile, &split);
    if (tile >= c.sp.tiles) return;
    const uint32_t kc = c.sp.kc_of(tile), k0 = split * kc;
    if (k0 >= c.k) return;
    const uint32_t rows = min(2 * c.ur, min(kc, c.k - k0));
    const uint32_t lps = c.seg_bytes / 128;            // lines per segment
    const uint32_t lpr = lps * (c.seg2_off ? 2 : 1);   // lines per weight row
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(c.w), 0, c.bytes, RSRC_FLAGS);
    uint32_t acc = 0;
    for (uint32_t L = threadIdx.x; L < rows * lpr; L += blockDim.x) {
        const uint32_t row = L / lpr, sg = L % lpr;
        const uint32_t off = (k0 + row) * c.ldw_bytes + tile * c.seg_bytes +
                             (sg / lps) * c.seg2_off + (sg % lps) * 128;
        acc ^= __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
    }
    asm volatile("" ::"v"(acc));   // keep the loads
}

// Signal "my sc1 stores are done" and return true in the workgroup that
// completes `target` arrivals on `counter` (which it resets for the next use).
__device__ __forceinline__ bool arrive_last(uint32_t* counter, uint32_t target, uint32_t* s_flag) {
    __builtin_amdgcn_s_waitcnt(0);     // this lane's sc1 stores are acknowledged
    __syncthreads();                   // ... and every other lane's
    if (threadIdx.x == 0) {
        const uint32_t old =
            __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *s_flag = (old == target - 1) ? 1u : 0u;
    }
    __syncthreads();
    return *s_flag != 0u;
}

__device__ __forceinline__ void reset_counter(uint32_t* counter) {
    if (threadIdx.x == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct StepParams {
    uint32_t batch, d, qd, hq, hkv, g, ff, cache_len, cache_stride, nsplit, split_keys;
    float rope_base, eps;
    const uint16_t *x, *k_cache, *v_cache;
    uint16_t *y, *k_new, *v_new;
    uint32_t* counters;        // every tile counter of the step (attention, W_o, gate/up, down)
    uint32_t n_counters;
    uint32_t* attn_counters;   // [B * Hkv]
    float* partial;            // split-K partials [tiles * splits][16][tile columns]
    uint32_t partial_bytes;
    float* sumsq;              // [qkv splits][16] sum of x^2 over each split
    SplitGeom qkv_sp;          // K splits of the QKV GEMM (its partials' layout)
    float* rope;               // [Dh / 2][2] cos, sin of pair i at position cache_len
    float* attn_part;          // [B][Hkv][nsplit][G][DH + 4]  (o[DH], m, l, pad)
    uint32_t attn_part_bytes;
    uint32_t sumsq_bytes;
    uint16_t* attn_out;        // [B][QD]  (QD = Hq * Dh, the attention width)
    float* x1;                 // [B][D]
    uint16_t* x1b;             // [B][D]  bf16(x1)
    uint16_t* x1b_lo;          // [B][D]  bf16(x1 - bf16(x1))
    float* sumsq2;             // [D / 128][16] sum of x1^2 per column tile
    uint16_t* act;             // [B][FF] bf16(silu(g) u)
    uint16_t* act_lo;          // [B][FF] its rounding remainder
    NextUnits next[4];         // indexed by EPI: what the kernel before that GEMM prefetches
};

struct GemmCfg {
    const uint16_t* a;     // activations [batch][k], row stride lda (rows >= batch read as 0)
    const uint16_t* a_lo;  // optional second bf16 term of the activations (same layout)
    uint32_t lda;
    const uint16_t* w;     // weights [k][ldw]
    uint32_t ldw;
    uint32_t k;
    SplitGeom sp;
    uint32_t paired;       // 1: tile t of TBN columns = gate cols [h t, h t + h) + up cols
                           //    ff + [h t, h t + h), h = TBN / 2
    uint32_t* counters;    // [tiles]
};

// ---- skinny GEMM + split-K finisher --------------------------------------------------

// C[16][N] = A[16][K] W[K][N]: A = the batch's activations (rows past the
// batch read as zero), W row-major.  A workgroup owns a column tile of
// TBN = 128 * WW columns and a K split of kc rows.  Its four waves stand WW
// side by side in N (128 columns each) and 4 / WW deep in K (32 rows each), so
// one unit of the split is (128 / WW) rows x TBN columns = 32 KB of weights;
// WW = 4 makes every row segment a workgroup reads 1 KB long (512 B per half
// for the paired gate | up tile), which HBM streams markedly faster than 256
// or 128 B segments.
//
// The weights never touch LDS.  Lane (kq = lane / 16, nl = lane % 16) of a
// wave loads rows 8 kq .. 8 kq + 7 of the wave's 32-row slab, columns
// 8 nl .. 8 nl + 7 of its 128-column slab (eight 16-byte loads; a load
// instruction covers 256 contiguous bytes of four rows), and transposes the
// 8 x 8 block in registers with v_perm_b32 into eight 8-k vectors, one per
// column 8 nl + c.  Vector c is the B operand of v_mfma_f32_16x16x32_bf16 for
// the 16 columns {8 nl + c | nl < 16} (lane group kq = k octet kq); the A
// operand, activation row nl and k octet kq, is one 16-byte load per lane.
// A unit is therefore 8 MFMAs per wave (16 with hi + lo activations), and
// accumulator c holds rows 4 kq .. 4 kq + 3 of column 8 nl + c.
//
// Units stream through a ring of R register slots: consuming unit j waits
// for its slot only (vmcnt = the younger slots still in flight), transposes
// it and re-issues the slot for unit j + R before running the MFMAs, so R
// units stay in flight through the whole split.  Every load is a buffer
// load clipped to the split: weight rows past it, and activation chunks past
// it or past the batch, return zeros without touching memory, so the ring
// runs a fixed number of units (a multiple of R) with one load order and
// no branches.  sched_barrier keeps the compiler from interleaving the slots'
// loads, because vmcnt retires loads in issue order.  The last trip is peeled
// and issues nothing: re-issued slots there would only fetch zeros, and the
// epilogue would wait 0.1-0.2 us for them before reusing their registers
// (0.8 us per step over the four skinny GEMMs, measured).
//
// After the K loop the accumulators meet in LDS as a row-major [16][TBN] tile
// (the 4 / WW row groups summed); the split-K partial in the workspace has the
// same layout (one coalesced sc1 store per float4).  The last workgroup of
// the tile (atomic counter) sums the other splits' partials, with the
// epilogue's own inputs loaded in the same round trip, and runs the epilogue
// (W_o, gate/up, down; the QKV partials are summed by the attention kernel).
template <int TBN>
__device__ __forceinline__ uint32_t tile_col(const GemmCfg& g, uint32_t ff, uint32_t tile,
                                             uint32_t c) {
    if (!g.paired) return tile * TBN + c;
    return c < TBN / 2 ? tile * (TBN / 2) + c : ff + tile * (TBN / 2) + (c - TBN / 2);
}

// The skinny GEMM's leading kernel arguments: what its first loads need,
// as plain scalars and pointers, so that the compiler preloads them into
// SGPRs (gfx950 kernel-argument preloading, -amdgpu-kernarg-preload-count):
// the first weight and activation loads then go out without waiting for a
// kernel-argument fetch (0.28-0.36 us per kernel, measured).
struct SkinnyPre {
    const uint16_t* w;
    const uint16_t* a;
    uint32_t a_lo_off;   // bytes from a to a_lo (hi + lo activations; a_lo follows a in the workspace)
    uint32_t ldw, lda, k;
    uint32_t batch_paired;   // batch | paired << 16
    uint32_t tiles, splits;  // splits | splits_slow << 16
    uint32_t kc32;           // kc / 32 | kc_slow / 32 << 16
    uint32_t cls;            // slow_mask | slow_val << 16
    uint32_t ff;
};
#define SKINNY_PRE_PARAMS                                                                      \
    const uint16_t *pre_w, const uint16_t *pre_a, uint32_t pre_a_lo_off, uint32_t pre_ldw,    \
        uint32_t pre_lda, uint32_t pre_k, uint32_t pre_batch_paired, uint32_t pre_tiles,      \
        uint32_t pre_splits, uint32_t pre_kc32, uint32_t pre_cls, uint32_t pre_ff
#define SKINNY_PRE_ARGS(q)                                                                      \
    (q).w, (q).a, (q).a_lo_off, (q).ldw, (q).lda, (q).k, (q).batch_paired, (q).tiles, (q).splits, \
        (q).kc32, (q).cls, (q).ff

template <int EPI, int WW, int R>
__global__ __launch_bounds__(256, 1)
void skinny_gemm_kernel(SKINNY_PRE_PARAMS, GemmCfg g_arg, StepParams p) {
    constexpr bool SPLIT_A = (EPI == EPI_GU || EPI == EPI_DOWN);   // hi + lo activations
    constexpr int NTERMS = SPLIT_A ? 2 : 1;
    constexpr int TBN = 128 * WW;                 // tile columns
    constexpr int RG = 4 / WW;                    // waves stacked in K
    constexpr int UR = 32 * RG;                   // k rows per unit
    constexpr int NQ = MROWS * TBN / 4 / 256;     // float4s of the tile per thread
    static_assert(WW == 1 || EPI == EPI_GU, "QKV, WO and DOWN epilogues use 128-column tiles");

    // RG accumulator tiles, then 16 x 16 floats of row-statistics scratch
    __shared__ __attribute__((aligned(16))) float red[RG * MROWS * TBN + MROWS * 16];
    __shared__ float red_ss[MROWS];
    __shared__ uint32_t s_last;

    // g_arg with every field the first loads use taken from the preloaded
    // arguments (the same values)
    GemmCfg g = g_arg;
    g.w = pre_w; g.a = pre_a;
    g.a_lo = reinterpret_cast<const uint16_t*>(reinterpret_cast<const uint8_t*>(pre_a) + pre_a_lo_off);
    g.ldw = pre_ldw; g.lda = pre_lda; g.k = pre_k; g.paired = pre_batch_paired >> 16;
    g.sp.tiles = pre_tiles;
    g.sp.splits = pre_splits & 0xffffu; g.sp.splits_slow = pre_splits >> 16;
    g.sp.kc = (pre_kc32 & 0xffffu) * 32; g.sp.kc_slow = (pre_kc32 >> 16) * 32;
    g.sp.slow_mask = pre_cls & 0xffffu; g.sp.slow_val = pre_cls >> 16;
    const uint32_t batch = pre_batch_paired & 0xffffu;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t cw = wave % WW, rw = wave / WW;       // wave's column slab, row slab
    const uint32_t kq = lane >> 4, nl = lane & 15;
    uint32_t tile, split;
    g.sp.block(blockIdx.x, &tile, &split);
    const uint32_t kc = g.sp.kc_of(tile), nsplit = g.sp.nsplits(tile);
    const uint32_t k_begin = split * kc;
    const uint32_t k_rows = min(kc, g.k - k_begin);   // a multiple of 32

    // ---- the ring ----
    const uint32_t a_bytes = __builtin_amdgcn_readfirstlane(batch * g.lda * 2);
    const __amdgpu_buffer_rsrc_t ars0 =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(g.a), 0, a_bytes, RSRC_FLAGS);
    const __amdgpu_buffer_rsrc_t ars1 = __builtin_amdgcn_make_buffer_rsrc(
        uniform_ptr(SPLIT_A ? g.a_lo : g.a), 0, a_bytes, RSRC_FLAGS);
    const uint32_t a_voff = (nl * g.lda + k_begin + 32 * rw + 8 * kq) * 2;
    const bool a_row_ok = nl < batch;
    const uint32_t ldw2 = g.ldw * 2;
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        uniform_ptr(g.w + (size_t)k_begin * g.ldw), 0, __builtin_amdgcn_readfirstlane(k_rows * ldw2),
        RSRC_FLAGS);
    const uint32_t w_voff = (32 * rw + 8 * kq) * ldw2 + tile_col<TBN>(g, pre_ff, tile, 128 * cw + 8 * nl) * 2;

    u32x4 ra[R][NTERMS];
    u32x4 rw8[R][8];
    auto issue = [&](int s, uint32_t j) {
        // (a split may end inside a unit: waves past its last row read zeros)
        const uint32_t ao =
            (a_row_ok && j * UR + 32 * rw < k_rows) ? a_voff + j * UR * 2 : 0x80000000u;
        ra[s][0] = __builtin_amdgcn_raw_buffer_load_b128(ars0, ao, 0, 0);
        if (SPLIT_A) ra[s][NTERMS - 1] = __builtin_amdgcn_raw_buffer_load_b128(ars1, ao, 0, 0);
        const uint32_t wo = w_voff + j * UR * ldw2;
#pragma unroll
        for (int i = 0; i < 8; ++i)   // streamed once per step
            rw8[s][i] = __builtin_amdgcn_raw_buffer_load_b128(wrs, wo + i * ldw2, 0, CPOL_NT);
    };
#pragma unroll
    for (int s = 0; s < R; ++s) {
        issue(s, s);
        __builtin_amdgcn_sched_barrier(0);
    }
    // QKV: workgroup 0 writes the RoPE table (cos, sin) of pair (2i, 2i+1),
    // i = tid < 64, at position cache_len, for the attention kernel, while
    // its first loads are in flight.  The angle pos * base^(-2i/Dh) is formed
    // and reduced mod 2 pi in fp64: an fp32 angle would be off by
    // ~pos * 6e-8 rad (0.06 rad at pos 10^6).
    // QKV: workgroup 0 also clears every counter the step's later kernels
    // count arrivals on.  Those kernels run after this one, so each step
    // starts from zeroed counters whatever the workspace held: a caller's
    // fresh workspace, or the no-alloc scratch after a call of other shapes
    // (which a replayed HIP graph cannot check for).  The finishers also reset
    // their counters when done.
    if (EPI == EPI_QKV && blockIdx.x == 0)
        for (uint32_t i = tid; i < p.n_counters; i += 256)
            __hip_atomic_store(&p.counters[i], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (EPI == EPI_QKV && blockIdx.x == 0 && tid < DH / 2) {
        const double omega = pow((double)p.rope_base, -2.0 * (double)tid / (double)DH);
        const double ang = (double)p.cache_len * omega;
        constexpr double TWO_PI = 6.283185307179586476925;
        float cs, sn;
        sincosf((float)(ang - TWO_PI * rint(ang / TWO_PI)), &sn, &cs);
        *reinterpret_cast<float2*>(p.rope + 2 * tid) = float2{cs, sn};
    }

    f32x4 acc[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[c] = f32x4{};
    float ss = 0.f;
    const uint32_t trips = ((kc + UR - 1) / UR + R - 1) / R;

    auto trip = [&](uint32_t t, auto more_c) {   // more_c: issue the slots' next units
#pragma unroll
        for (int s = 0; s < R; ++s) {
            // 8x8 transpose: b[c] = column 8 nl + c, k = 8 kq .. 8 kq + 7
            bf16x8 b[8];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                u32x4 lo, hi;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    lo[j] = __builtin_amdgcn_perm(rw8[s][2 * j + 1][m], rw8[s][2 * j][m], 0x05040100u);
                    hi[j] = __builtin_amdgcn_perm(rw8[s][2 * j + 1][m], rw8[s][2 * j][m], 0x07060302u);
                }
                b[2 * m] = __builtin_bit_cast(bf16x8, lo);
                b[2 * m + 1] = __builtin_bit_cast(bf16x8, hi);
            }
            const bf16x8 a = __builtin_bit_cast(bf16x8, ra[s][0]);
            const bf16x8 alo = __builtin_bit_cast(bf16x8, ra[s][NTERMS - 1]);
            // slot s is free: its next unit's loads go out now
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (decltype(more_c)::value) issue(s, (t + 1) * R + s);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[c], acc[c], 0, 0, 0);
                if (SPLIT_A)
                    acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(alo, b[c], acc[c], 0, 0, 0);
            }
            if (EPI == EPI_QKV) {   // RMSNorm statistics from the A operand
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float v = (float)a[e];
                    ss += v * v;
                }
            }
        }
    };
    for (uint32_t t = 0; t + 1 < trips; ++t) trip(t, std::true_type{});
    trip(trips - 1, std::false_type{});   // trips >= 1: every K is a positive multiple of 128

    // ---- accumulators -> row-major [16][TBN] tile in LDS, row groups summed ----
    {
        float* buf = red + rw * (MROWS * TBN);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float* dst = buf + (4 * kq + r) * TBN + 128 * cw + 8 * nl;
            *reinterpret_cast<f32x4*>(dst) = f32x4{acc[0][r], acc[1][r], acc[2][r], acc[3][r]};
            *reinterpret_cast<f32x4*>(dst + 4) = f32x4{acc[4][r], acc[5][r], acc[6][r], acc[7][r]};
        }
    }
    if (EPI == EPI_QKV) {   // sum of x^2 per row over this split: lanes nl of every kq and wave
        ss += __shfl_xor(ss, 16);
        ss += __shfl_xor(ss, 32);
        if (lane < 16) red[RG * MROWS * TBN + wave * MROWS + lane] = ss;
    }
    __syncthreads();
    f32x4 v[NQ];
#pragma unroll
    for (int h = 0; h < NQ; ++h) {
        const uint32_t q = tid + 256 * h;
        v[h] = reinterpret_cast<const f32x4*>(red)[q];
#pragma unroll
        for (int r = 1; r < RG; ++r) v[h] += reinterpret_cast<const f32x4*>(red + r * MROWS * TBN)[q];
    }

    // split-K partial: the same row-major tile, float4 q at byte 16 q
    constexpr uint32_t SPLIT_BYTES = MROWS * TBN * 4;
    const __amdgpu_buffer_rsrc_t prs = coherent_rsrc(p.partial, p.partial_bytes);
    const uint32_t tile_base = tile * g.sp.stride() * SPLIT_BYTES;
#pragma unroll
    for (int h = 0; h < NQ; ++h) st_sc1(prs, tile_base + split * SPLIT_BYTES + (tid + 256 * h) * 16, v[h]);
    const __amdgpu_buffer_rsrc_t srs = coherent_rsrc(p.sumsq, p.sumsq_bytes);
    if (EPI == EPI_QKV && tile == 0 && tid < MROWS) {   // every tile sums the same x rows
        const float* sp = red + RG * MROWS * TBN;
        st_sc1(srs, (split * MROWS + tid) * 4,
               sp[tid] + sp[MROWS + tid] + sp[2 * MROWS + tid] + sp[3 * MROWS + tid]);
    }
    // QKV: no finisher; each attention workgroup sums the partials it needs.
    if (EPI == EPI_QKV) return;
    if (!arrive_last(&g.counters[tile], nsplit, &s_last)) {
        if (EPI == EPI_WO || EPI == EPI_GU) prefetch_next_units(p.next[EPI + 1], blockIdx.x);
        return;
    }

    // ---- finisher: this workgroup is the last of its tile ----
    // One memory round trip: the first SB splits' partials and the epilogue's
    // inputs are all issued before the first wait.
    // Partials and sums are read through descriptors clipped to this tile's
    // splits, so loads past the last split return zeros and every load and
    // add is unconditional (a load behind a branch would cost a round trip of
    // its own).  Splits are summed in split order whichever workgroup
    // finishes, so the result does not depend on arrival order.
    constexpr uint32_t SB = NQ >= 8 ? 4 : 8;   // splits per batch of partial loads
    const __amdgpu_buffer_rsrc_t trs = coherent_rsrc(
        reinterpret_cast<const uint8_t*>(p.partial) + tile_base, nsplit * SPLIT_BYTES);
    const uint32_t row = tid & 15, grp = tid >> 4;   // row statistics: row, group of tiles
    f32x4 w[SB][NQ];
#pragma unroll
    for (uint32_t u = 0; u < SB; ++u)
#pragma unroll
        for (int h = 0; h < NQ; ++h) w[u][h] = ld4_sc1(trs, u * SPLIT_BYTES + (tid + 256 * h) * 16);
    const uint32_t eb = tid >> 4, ec = 8 * (tid & 15);   // epilogue: row eb, columns ec .. ec+7
    u32x4 pre_x = {};                                    // WO: x (bf16)
    f32x4 pre_x1[2] = {f32x4{}, f32x4{}};                // DOWN: x1 (fp32)
    float pre_ss[8] = {};                                // GU: x1^2 sums of the W_o tiles
    if (EPI == EPI_WO)
        pre_x = *reinterpret_cast<const u32x4*>(p.x + (size_t)(eb < p.batch ? eb : 0) * p.d +
                                                tile * TBN + ec);
    if (EPI == EPI_DOWN) {
        const float* src = p.x1 + (size_t)(eb < p.batch ? eb : 0) * p.d + tile * TBN + ec;
        pre_x1[0] = *reinterpret_cast<const f32x4*>(src);
        pre_x1[1] = *reinterpret_cast<const f32x4*>(src + 4);
    }
    if (EPI == EPI_GU) {
        const uint32_t ntile = p.d / 128;
#pragma unroll
        for (int u = 0; u < 8; ++u)
            pre_ss[u] = p.sumsq2[min(eb + 16u * u, ntile - 1) * MROWS + (tid & 15)];
    }
    {
        f32x4 sum[NQ];
#pragma unroll
        for (int h = 0; h < NQ; ++h) {
            sum[h] = w[0][h];
#pragma unroll
            for (uint32_t u = 1; u < SB; ++u) sum[h] += w[u][h];
        }
        for (uint32_t sp0 = SB; sp0 < nsplit; sp0 += SB) {   // more than SB splits
#pragma unroll
            for (uint32_t u = 0; u < SB; ++u)
#pragma unroll
                for (int h = 0; h < NQ; ++h)
                    w[u][h] = ld4_sc1(trs, (sp0 + u) * SPLIT_BYTES + (tid + 256 * h) * 16);
#pragma unroll
            for (uint32_t u = 0; u < SB; ++u)
#pragma unroll
                for (int h = 0; h < NQ; ++h) sum[h] += w[u][h];
        }
#pragma unroll
        for (int h = 0; h < NQ; ++h) reinterpret_cast<f32x4*>(red)[tid + 256 * h] = sum[h];
    }
    // GU: the RMSNorm scale of x1, from the sums of x1^2 over the W_o column
    // tiles: thread (row, grp) sums every 16th tile, then the 16 groups
    // through LDS.
    if (EPI == EPI_GU) {
        float* scratch = red + MROWS * TBN;   // 16 x 16 floats past the tile sums
        float sv = 0.f;
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u)
            if (grp + 16 * u < p.d / 128) sv += pre_ss[u];
        scratch[grp * MROWS + row] = sv;
        __syncthreads();
        if (tid < MROWS) {
            float t = 0.f;
#pragma unroll
            for (int q = 0; q < 16; ++q) t += scratch[q * MROWS + tid];
            red_ss[tid] = rsqrtf(t / (float)p.d + p.eps);
        }
    }
    __syncthreads();

    if (EPI == EPI_WO) {
        // thread: row eb, columns ec .. ec+7; x1 = x + attn W_o (rows past
        // the batch computed from x row 0, never stored, their sums zeroed)
        const f32x4 r0 = *reinterpret_cast<const f32x4*>(&red[eb * TBN + ec]);
        const f32x4 r1 = *reinterpret_cast<const f32x4*>(&red[eb * TBN + ec + 4]);
        float xv[8];
        float sq = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t xw = pre_x[e / 2];
            xv[e] = __uint_as_float((e & 1) ? (xw & 0xffff0000u) : (xw << 16)) +
                    (e < 4 ? r0[e] : r1[e - 4]);
            sq += xv[e] * xv[e];
        }
        if (eb < p.batch) {
            const size_t o = (size_t)eb * p.d + tile * TBN + ec;
            *reinterpret_cast<f32x4*>(p.x1 + o) = f32x4{xv[0], xv[1], xv[2], xv[3]};
            *reinterpret_cast<f32x4*>(p.x1 + o + 4) = f32x4{xv[4], xv[5], xv[6], xv[7]};
            uint32_t hi[4], lo[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) split_bf16(xv[2 * e], xv[2 * e + 1], hi[e], lo[e]);
            *reinterpret_cast<u32x4*>(p.x1b + o) = u32x4{hi[0], hi[1], hi[2], hi[3]};
            *reinterpret_cast<u32x4*>(p.x1b_lo + o) = u32x4{lo[0], lo[1], lo[2], lo[3]};
        }
        // row sums of x1^2 over the tile: the 16 threads of a row are 16 adjacent lanes
#pragma unroll
        for (int o2 = 8; o2 > 0; o2 >>= 1) sq += __shfl_xor(sq, o2);
        if ((tid & 15) == 0) p.sumsq2[tile * MROWS + eb] = eb < p.batch ? sq : 0.f;
    } else if (EPI == EPI_GU) {
        // tile = gate columns [TBN/2 tile, +TBN/2) and the matching up columns;
        // thread: row tid / 16, CPT consecutive columns (vector LDS reads and
        // stores, no per-element branch)
        constexpr int HALF = TBN / 2, CPT = HALF / 16;
        const uint32_t b = tid >> 4, c0 = CPT * (tid & 15);
        if (b < p.batch) {
            const float r2 = red_ss[b];
            uint32_t hi[CPT / 2], lo[CPT / 2];
#pragma unroll
            for (int q = 0; q < CPT / 4; ++q) {
                const f32x4 gv = *reinterpret_cast<const f32x4*>(&red[b * TBN + c0 + 4 * q]);
                const f32x4 uv = *reinterpret_cast<const f32x4*>(&red[b * TBN + HALF + c0 + 4 * q]);
#pragma unroll
                for (int e = 0; e < 4; e += 2) {
                    const float a0 = silu(gv[e] * r2) * (uv[e] * r2);
                    const float a1 = silu(gv[e + 1] * r2) * (uv[e + 1] * r2);
                    split_bf16(a0, a1, hi[2 * q + e / 2], lo[2 * q + e / 2]);
                }
            }
            const size_t o = (size_t)b * p.ff + tile * HALF + c0;
#pragma unroll
            for (int q = 0; q < CPT / 8; ++q) {
                *reinterpret_cast<u32x4*>(p.act + o + 8 * q) =
                    u32x4{hi[4 * q], hi[4 * q + 1], hi[4 * q + 2], hi[4 * q + 3]};
                *reinterpret_cast<u32x4*>(p.act_lo + o + 8 * q) =
                    u32x4{lo[4 * q], lo[4 * q + 1], lo[4 * q + 2], lo[4 * q + 3]};
            }
            if (CPT == 4) {
                *reinterpret_cast<uint2*>(p.act + o) = uint2{hi[0], hi[1]};
                *reinterpret_cast<uint2*>(p.act_lo + o) = uint2{lo[0], lo[1]};
            }
        }
    } else {   // EPI_DOWN: y = x1 + act W_down; thread: row eb, columns ec .. ec+7
        const f32x4 r0 = *reinterpret_cast<const f32x4*>(&red[eb * TBN + ec]);
        const f32x4 r1 = *reinterpret_cast<const f32x4*>(&red[eb * TBN + ec + 4]);
        if (eb < p.batch) {
            const u32x4 out = {pack_bf16(pre_x1[0][0] + r0[0], pre_x1[0][1] + r0[1]),
                               pack_bf16(pre_x1[0][2] + r0[2], pre_x1[0][3] + r0[3]),
                               pack_bf16(pre_x1[1][0] + r1[0], pre_x1[1][1] + r1[1]),
                               pack_bf16(pre_x1[1][2] + r1[2], pre_x1[1][3] + r1[3])};
            *reinterpret_cast<u32x4*>(p.y + (size_t)eb * p.d + tile * TBN + ec) = out;
        }
    }
    reset_counter(&g.counters[tile]);   // ready for the next step
}

// ---- flash-decoding attention ------------------------------------------------------------
// The cached keys of each (sequence, kv head) are cut into `nsplit` splits of
// `split_keys` keys; one workgroup streams one split, 64 keys per iteration,
// wave w taking the 16-key block at offset 16 w.  Each wave runs its own
// online softmax, with the next block's K and V loads in flight while the
// current block is computed (register double buffer, no workgroup barrier in
// the loop):
//   scores  S = K q^T on MFMA (A = 16 keys x 32 d, B = 32 d x 16 query heads),
//           lane (j, grp) holds S[key 4 grp + r][head j], r < 4;
//   softmax running max / sum per head, folded over the four lanes of a head
//           with lane shuffles;
//   o = p v on VALU: lane l owns d = 2l, 2l + 1 of every key (one dword per
//           key row, so each V load is one whole 256-byte row per wave); the
//           block's probabilities reach it through a wave-private LDS slot.
// K and V are read through buffer descriptors clipped at the split's last
// key: loads past it return zeros without touching memory, so every load is
// unconditional and the waitcnt pass sees one fixed load order.  The four
// waves are combined through LDS and the split's unnormalised (o, max, sum)
// go out as sc1 partials.  The workgroup that completes the (sequence, kv
// head) merges the splits and the new token (key and value from k_new /
// v_new) with log-sum-exp weights; all its partial loads are issued
// together, so the merge costs one memory round trip.

constexpr int AKEYS = 64;                 // keys per workgroup iteration
constexpr int AR = 2;                     // 64-key blocks in flight per workgroup
constexpr int APITCH = DH + 4;            // floats per (split, head) partial: o[DH], m, l, pad
constexpr int QP = DH + 8;                // LDS pitch (bf16) of a query row
constexpr float NEG_BIG = -1.0e30f;       // "no key yet": finite, so max/exp never see inf - inf

struct KVBlock {
    u32x4 k[4];      // K[key j][32 m + 8 grp .. + 8] for the scores MFMA, m < 4
    uint32_t v[16];  // V[key i][2 lane, 2 lane + 1], i < 16
};

template <int GT>
__global__ __launch_bounds__(256)
void attention_kernel(StepParams p) {
    __shared__ __attribute__((aligned(16))) uint16_t qs[16][QP];   // q rows (rows past G zero)
    __shared__ __attribute__((aligned(16))) uint16_t kvn[2][DH];   // k_new, v_new (bf16)
    // per wave: p[key][head] of the current block.  Row pitch 20 floats: the
    // store of lane (j, grp), row 4 grp + r, lands in bank 16 grp + 20 r + j,
    // so the 64 lanes hit 64 banks (with a pitch of 16 the four grp rows were
    // 64 floats apart: a 4-way conflict on every store).
    __shared__ __attribute__((aligned(16))) float xp[4][16][20];
    __shared__ float xa[4][4][16];        // per wave: rescale factor of each head (row 0 read)
    __shared__ float wo[4][GT][DH];       // per wave: o after the key loop
    __shared__ float wm[4][GT], wl[4][GT];
    __shared__ float s_new[GT];
    __shared__ uint32_t s_last;

    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t j = lane & 15, grp = lane >> 4;
    const uint32_t G = p.g;
    const uint32_t split = blockIdx.x % p.nsplit;
    const uint32_t bk = blockIdx.x / p.nsplit;            // b * hkv + kvh
    const uint32_t b = bk / p.hkv, kvh = bk - b * p.hkv;
    const uint32_t key0 = split * p.split_keys;
    const uint32_t key_end = min(key0 + p.split_keys, p.cache_len);
    const uint32_t nkeys = key_end > key0 ? key_end - key0 : 0u;
    const uint32_t nblk = (nkeys + AKEYS - 1) / AKEYS;
    const size_t row0 = (size_t)bk * p.cache_stride + key0;
    // (the descriptors are workgroup-uniform; readfirstlane lets the compiler
    // keep them in SGPRs instead of wrapping each load in a waterfall loop)
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
        uniform_ptr(nkeys ? p.k_cache + row0 * DH : p.k_new), 0,
        __builtin_amdgcn_readfirstlane(nkeys * DH * 2), RSRC_FLAGS);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
        uniform_ptr(nkeys ? p.v_cache + row0 * DH : p.v_new), 0,
        __builtin_amdgcn_readfirstlane(nkeys * DH * 2), RSRC_FLAGS);

    // Offsets (bytes) inside the split of this lane's first K and V dwords.
    const uint32_t koff = ((16 * wave + j) * DH + 8 * grp) * 2;
    const uint32_t voff = ((16 * wave) * DH + 2 * lane) * 2;
    auto load = [&](KVBlock& blk, uint32_t t) {
        const uint32_t base = t * AKEYS * DH * 2;
#pragma unroll
        for (int m = 0; m < 4; ++m)
            blk.k[m] = __builtin_amdgcn_raw_buffer_load_b128(krs, base + koff + 64 * m, 0, CPOL_NT);
#pragma unroll
        for (int i = 0; i < 16; ++i)
            blk.v[i] = __builtin_amdgcn_raw_buffer_load_b32(vrs, base + voff + i * DH * 2, 0, CPOL_NT);
    };

    // ---- q, the new key and the new value of this (sequence, kv head) ----
    // The QKV GEMM leaves split-K partials, [tile][split][16][128] fp32 with
    // tile = one head of Q, K or V, and per-split row sums of x^2.  Every
    // workgroup of the pair sums row b of its G query heads, its key head and
    // its value head over the splits (left to right, in batches of PB: loads
    // past the last split return zeros), applies the RMSNorm row scale and
    // the RoPE rotation, and keeps q (pre-scaled by 1/sqrt(Dh), the MFMA B
    // operand, re-read per block), k_new and v_new as bf16 in LDS.  These
    // loads go out ahead of the first K/V block's, which do not depend on
    // them; split 0 also writes k_new and v_new out.
    constexpr uint32_t SPLIT_BYTES = MROWS * DH * 4;
    constexpr uint32_t PB = 16;   // splits loaded ahead of the first K/V block
    const SplitGeom& qg = p.qkv_sp;
    const uint32_t qsp0 = qg.nsplits(0);   // tile 0 wrote the per-split sums of x^2
    const uint32_t nitems_q = (G + 2) * (DH / 4);           // (head, column quad) items
    const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(
        p.sumsq, 0, __builtin_amdgcn_readfirstlane(qsp0 * MROWS * 4), RSRC_FLAGS);
    const __amdgpu_buffer_rsrc_t prs =
        __builtin_amdgcn_make_buffer_rsrc(p.partial, 0, p.partial_bytes, RSRC_FLAGS);
    // item -> (its tile's partials at split 0, the tile's split count)
    auto item_tile = [&](uint32_t idx) -> uint32_t {
        const uint32_t ts = idx / (DH / 4);
        return ts < G ? kvh * G + ts : p.qd / DH + (ts - G) * p.hkv + kvh;
    };
    auto item_base = [&](uint32_t idx) -> uint32_t {
        return item_tile(idx) * qg.stride() * SPLIT_BYTES + b * (DH * 4) + 16 * (idx % (DH / 4));
    };
    f32x4 pw[PB];
    auto load_item = [&](uint32_t base, uint32_t n, uint32_t c0) {
#pragma unroll
        for (uint32_t u = 0; u < PB; ++u)
            pw[u] = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                           prs, c0 + u < n ? base + (c0 + u) * SPLIT_BYTES : 0x80000000u, 0, 0));
    };
    // The splits are summed left to right: sum = w0 + w1 + ... (loads past
    // the last split add zeros).
    auto sum_item = [&](uint32_t base, uint32_t n) -> f32x4 {
        f32x4 sum = pw[0];
#pragma unroll
        for (uint32_t u = 1; u < PB; ++u) sum += pw[u];
        for (uint32_t c0 = PB; c0 < n; c0 += PB) {   // more splits: loads after the K/V block's
            load_item(base, n, c0);
#pragma unroll
            for (uint32_t u = 0; u < PB; ++u) sum += pw[u];
        }
        return sum;
    };
    // row b's sum of x^2: lane l < 16 of each wave sums splits l, l + 16, ...,
    // then the 16 lanes are added in order
    constexpr uint32_t XB = 8;
    float xs[XB];
    auto load_xs = [&](uint32_t t0) {
#pragma unroll
        for (uint32_t u = 0; u < XB; ++u)
            xs[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                srs, lane < 16 ? ((t0 + lane + 16 * u) * MROWS + b) * 4 : 0x80000000u, 0, 0));
    };
    // Every load the first item needs is issued before the first K/V block's
    // (vmcnt retires loads in issue order: a wait for a later load would also
    // wait for that block and delay the next block's issue).
    const uint32_t item0 = min(tid, nitems_q - 1);
    const uint32_t base0 = item_base(item0), n0 = qg.nsplits(item_tile(item0));
    load_xs(0);
    load_item(base0, n0, 0);
    const f32x4 rope0 = *reinterpret_cast<const f32x4*>(p.rope + 4 * (item0 % (DH / 4)));
    // Both slots of the ring are filled before the prologue's arithmetic,
    // so 2 x 32 KB per workgroup stream while it waits for the partials.
    KVBlock kv[AR];
#pragma unroll
    for (int u = 0; u < AR; ++u) {
        load(kv[u], u);
        __builtin_amdgcn_sched_barrier(0);
    }
    float r1;
    {
        float sv = 0.f;
#pragma unroll
        for (uint32_t u = 0; u < XB; ++u) sv += xs[u];
        for (uint32_t t0 = 16 * XB; t0 < qsp0; t0 += 16 * XB) {   // more than 128 splits
            load_xs(t0);
#pragma unroll
            for (uint32_t u = 0; u < XB; ++u) sv += xs[u];
        }
        float t = 0.f;
#pragma unroll
        for (int l = 0; l < 16; ++l)
            t += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sv), l));
        r1 = rsqrtf(t / (float)p.d + p.eps);
    }
    auto finish_item = [&](uint32_t idx, f32x4 sum, f32x4 rt) {
        const uint32_t ts = idx / (DH / 4), c = idx % (DH / 4);
        const float v0 = sum[0] * r1, v1 = sum[1] * r1, v2 = sum[2] * r1, v3 = sum[3] * r1;
        uint2 out;
        if (ts < G) {
            const float qsc = rsqrtf((float)DH);
            out.x = pack_bf16((v0 * rt[0] - v1 * rt[1]) * qsc, (v0 * rt[1] + v1 * rt[0]) * qsc);
            out.y = pack_bf16((v2 * rt[2] - v3 * rt[3]) * qsc, (v2 * rt[3] + v3 * rt[2]) * qsc);
            *reinterpret_cast<uint2*>(&qs[ts][4 * c]) = out;
        } else {
            if (ts == G) {
                out.x = pack_bf16(v0 * rt[0] - v1 * rt[1], v0 * rt[1] + v1 * rt[0]);
                out.y = pack_bf16(v2 * rt[2] - v3 * rt[3], v2 * rt[3] + v3 * rt[2]);
            } else {
                out.x = pack_bf16(v0, v1);
                out.y = pack_bf16(v2, v3);
            }
            *reinterpret_cast<uint2*>(&kvn[ts - G][4 * c]) = out;
            if (split == 0)
                *reinterpret_cast<uint2*>((ts == G ? p.k_new : p.v_new) + (size_t)bk * DH + 4 * c) = out;
        }
    };
    if (tid < nitems_q) finish_item(tid, sum_item(base0, n0), rope0);
    for (uint32_t idx = tid + 256; idx < nitems_q; idx += 256) {   // G > 4: more items
        const uint32_t base = item_base(idx);
        const uint32_t n = qg.nsplits(item_tile(idx));
        load_item(base, n, 0);
        finish_item(idx, sum_item(base, n),
                    *reinterpret_cast<const f32x4*>(p.rope + 4 * (idx % (DH / 4))));
    }
    {   // query rows past G are zero
        const uint32_t qh = tid / (DH / 8), qc = tid % (DH / 8);
        if (qh >= G) *reinterpret_cast<u32x4*>(&qs[qh][8 * qc]) = u32x4{};
    }
    __syncthreads();

    float m_run = NEG_BIG, l_run = 0.f;   // lane (j, grp): head j; l over this lane's keys
    float o[GT][2];                       // lane: o[h][d = 2 lane + e]
#pragma unroll
    for (int h = 0; h < GT; ++h) o[h][0] = o[h][1] = 0.f;

    auto compute = [&](const KVBlock& blk, uint32_t t) {
        const uint32_t kb = t * AKEYS + 16 * wave;     // block's first key, relative to key0
        f32x4 s = {};
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const bf16x8 qv = *reinterpret_cast<const bf16x8*>(&qs[j][32 * m + 8 * grp]);
            s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, blk.k[m]), qv,
                                                        s, 0, 0, 0);
        }
        float mloc = NEG_BIG;
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (kb + 4 * grp + r < nkeys) mloc = fmaxf(mloc, s[r]);
        mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
        const float m_new = fmaxf(m_run, mloc);
        const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * LOG2E);
        float pr[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const bool ok = kb + 4 * grp + r < nkeys && j < G;
            pr[r] = ok ? __builtin_amdgcn_exp2f((s[r] - m_new) * LOG2E) : 0.f;
        }
        l_run = l_run * alpha + (pr[0] + pr[1] + pr[2] + pr[3]);
        m_run = m_new;
        // unconditional stores: no branch inside the loop body, which would let
        // the compiler sink one block's FMAs past the next block's loads
#pragma unroll
        for (int r = 0; r < 4; ++r) xp[wave][4 * grp + r][j] = pr[r];
        xa[wave][grp][j] = alpha;
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int h4 = 0; h4 < GT / 4; ++h4) {
            const f32x4 al = *reinterpret_cast<const f32x4*>(&xa[wave][0][4 * h4]);
#pragma unroll
            for (int hh = 0; hh < 4; ++hh) {
                o[4 * h4 + hh][0] *= al[hh];
                o[4 * h4 + hh][1] *= al[hh];
            }
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float v0 = __uint_as_float(blk.v[i] << 16);
            const float v1 = __uint_as_float(blk.v[i] & 0xffff0000u);
#pragma unroll
            for (int h4 = 0; h4 < GT / 4; ++h4) {
                const f32x4 ph = *reinterpret_cast<const f32x4*>(&xp[wave][i][4 * h4]);
#pragma unroll
                for (int hh = 0; hh < 4; ++hh) {
                    o[4 * h4 + hh][0] += ph[hh] * v0;
                    o[4 * h4 + hh][1] += ph[hh] * v1;
                }
            }
        }
        __builtin_amdgcn_wave_barrier();
    };

    // A ring of AR blocks: block t + AR goes into block t's slot as soon as
    // block t is computed, so while block t + 1 is computed block t + 2 is in
    // flight (AR = 2), as when block t + AR - 1 was issued right before block
    // t; only the start differs (both slots already in flight during the
    // prologue).  Four in flight measured 1.5 us slower than two at the
    // benchmark shape (more concurrent streams per CU, less DRAM page
    // locality).  sched_barrier pins the order.
    for (uint32_t t = 0; t < nblk; t += AR) {
#pragma unroll
        for (int u = 0; u < AR; ++u) {
            __builtin_amdgcn_sched_barrier(0);
            compute(kv[u], t + u);
            __builtin_amdgcn_sched_barrier(0);
            load(kv[u], t + u + AR);
        }
    }

    // ---- fold each wave's key groups, then the four waves ----
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
#pragma unroll
    for (int h = 0; h < GT; ++h)
        *reinterpret_cast<float2*>(&wo[wave][h][2 * lane]) = float2{o[h][0], o[h][1]};
    if (grp == 0 && j < GT) { wm[wave][j] = m_run; wl[wave][j] = l_run; }
    __syncthreads();

    const __amdgpu_buffer_rsrc_t ars = coherent_rsrc(p.attn_part, p.attn_part_bytes);
    const uint32_t part0 = (bk * p.nsplit + split) * G * APITCH * 4;
    for (uint32_t idx = tid; idx < G * (DH / 4); idx += 256) {
        const uint32_t h = idx / (DH / 4), d4 = idx % (DH / 4);
        float M = NEG_BIG;
#pragma unroll
        for (int w = 0; w < 4; ++w) M = fmaxf(M, wm[w][h]);
        f32x4 O = {};
        float L = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float sw = __builtin_amdgcn_exp2f((wm[w][h] - M) * LOG2E);
            O += sw * *reinterpret_cast<const f32x4*>(&wo[w][h][4 * d4]);
            L += sw * wl[w][h];
        }
        st_sc1(ars, part0 + (h * APITCH + 4 * d4) * 4, O);
        if (d4 == 0) {
            st_sc1(ars, part0 + (h * APITCH + DH) * 4, M);
            st_sc1(ars, part0 + (h * APITCH + DH + 1) * 4, L);
        }
    }
    if (!arrive_last(&p.attn_counters[bk], p.nsplit, &s_last)) {
        prefetch_next_units(p.next[EPI_WO], blockIdx.x);
        return;
    }

    // ---- merge: the splits' partials plus the new token ----
    // One memory round trip in the common case: the first U splits' partials
    // of this thread's first item (head h, d quad d4) and the new value are
    // loaded together with the q rows and the new key of the q . k_new scores.
    constexpr uint32_t U = 8;                      // splits per batch of loads
    const uint32_t parts = bk * p.nsplit * G * APITCH * 4;
    const uint32_t nitems = G * (DH / 4);
    f32x4 oc[U];
    float mc[U], lc[U];
    auto load_batch = [&](uint32_t idx, uint32_t c0) {
        const uint32_t h = idx / (DH / 4), d4 = idx % (DH / 4);
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {     // past the last split: reload it, weight 0
            const uint32_t c = min(c0 + u, p.nsplit - 1);
            const uint32_t at = parts + (c * G + h) * APITCH * 4;
            oc[u] = ld4_sc1(ars, at + 16 * d4);
            mc[u] = ld_sc1(ars, at + DH * 4);
            lc[u] = ld_sc1(ars, at + (DH + 1) * 4);
        }
    };
    load_batch(min(tid, nitems - 1), 0);
    const uint2 vv0 = *reinterpret_cast<const uint2*>(&kvn[1][4 * (tid % (DH / 4))]);
    {   // s_new = q . k_new (q is pre-scaled); wave w takes heads w, w + 4, ...
        const uint32_t ka = *reinterpret_cast<const uint32_t*>(&kvn[0][2 * lane]);
        uint32_t qa[GT / 4];
#pragma unroll
        for (int i = 0; i < GT / 4; ++i)
            qa[i] = *reinterpret_cast<const uint32_t*>(&qs[min(wave + 4 * i, G - 1)][2 * lane]);
#pragma unroll
        for (int i = 0; i < GT / 4; ++i) {
            float d = __uint_as_float(qa[i] << 16) * __uint_as_float(ka << 16) +
                      __uint_as_float(qa[i] & 0xffff0000u) * __uint_as_float(ka & 0xffff0000u);
#pragma unroll
            for (int o2 = 32; o2 > 0; o2 >>= 1) d += __shfl_xor(d, o2);
            if (lane == 0 && wave + 4 * i < G) s_new[wave + 4 * i] = d;
        }
    }
    __syncthreads();
    for (uint32_t idx = tid; idx < nitems; idx += 256) {
        const uint32_t h = idx / (DH / 4), d4 = idx % (DH / 4);
        if (idx != tid) load_batch(idx, 0);        // a second item per thread (G > 8)
        float M = NEG_BIG, L = 0.f;
        f32x4 O = {};
        for (uint32_t c0 = 0; c0 < p.nsplit; c0 += U) {
            if (c0 > 0) load_batch(idx, c0);
            float Mb = M;
#pragma unroll
            for (uint32_t u = 0; u < U; ++u) Mb = fmaxf(Mb, mc[u]);
            const float sc = __builtin_amdgcn_exp2f((M - Mb) * LOG2E);
            O *= sc;
            L *= sc;
#pragma unroll
            for (uint32_t u = 0; u < U; ++u) {
                const float w = c0 + u < p.nsplit ? __builtin_amdgcn_exp2f((mc[u] - Mb) * LOG2E) : 0.f;
                O += w * oc[u];
                L += w * lc[u];
            }
            M = Mb;
        }
        const float sn = s_new[h];
        const float Mf = fmaxf(M, sn);
        const float so = __builtin_amdgcn_exp2f((M - Mf) * LOG2E);
        const float wn = __builtin_amdgcn_exp2f((sn - Mf) * LOG2E);
        const uint2 vv = idx == tid ? vv0 : *reinterpret_cast<const uint2*>(&kvn[1][4 * d4]);
        const f32x4 vn = {__uint_as_float(vv.x << 16), __uint_as_float(vv.x & 0xffff0000u),
                          __uint_as_float(vv.y << 16), __uint_as_float(vv.y & 0xffff0000u)};
        const f32x4 res = (O * so + wn * vn) / (L * so + wn);
        uint2 out;
        out.x = pack_bf16(res[0], res[1]);
        out.y = pack_bf16(res[2], res[3]);
        *reinterpret_cast<uint2*>(p.attn_out + (size_t)b * p.qd + (kvh * G + h) * DH + 4 * d4) = out;
    }
    reset_counter(&p.attn_counters[bk]);
}

// ---- host side -----------------------------------------------------------------------------

struct Plan {
    uint32_t nqkv, g, nsplit, split_keys;
    uint32_t tiles[4], splits[4], kc[4], ring[4], ww[4];
    SplitGeom geo[4];
    size_t off_counters, off_partial, off_sumsq, off_rope, off_attn_part, off_attn_out, off_x1,
        off_x1b, off_x1b_lo, off_sumsq2, off_act, off_act_lo, total;
    uint32_t counter_base[4];   // attn, wo, gu, down (the QKV GEMM has no finisher)
    uint32_t n_counters;
};

// K split of a skinny GEMM: enough splits that tiles x splits gives about one
// workgroup per CU (fewer, longer streams read HBM faster than two per CU),
// each split a whole number of 32-row groups (so 5 splits of K = 4096 are
// 832, 832, 832, 832 and 768 rows rather than 7, 7, 7, 7 and 4 steps of 128)
// and at least MIN_KC rows: a tile's last workgroup reads every split's
// partial sums, and on the small GEMMs of one 8-way tensor-parallel shard
// (qkv: 6 column tiles, K = 4096; W_o: K = 512) splits of 64-128 rows made
// that reduction the larger part of the kernel (qkv 13.9 -> 11.6 us, W_o
// 9.7 -> 9.4 us at 256 rows; 384 and 512 were slower). The full layer's
// splits are all 512 rows or more, so this leaves its plan unchanged. The
// ring holds RING units of 128 / ww rows, or the split's unit count below that.
constexpr uint32_t KG = 32;       // K split granularity (rows)
constexpr uint32_t MIN_KC = 256;  // fewest K rows per split

// The plan is a function of the shapes alone: it is sized for the 256 CUs of
// a whole gfx950 device (MI350X / MI355X), not for the device in use, so
// mb_decoder_step_workspace_bytes() gives the same answer before and after
// mb_init() and on a partitioned device (which then runs several workgroups
// per CU), and the split-K summation order -- hence every output bit -- does
// not depend on the device.
constexpr uint32_t PLAN_CUS = 256;

static void choose_split(uint32_t tiles, uint32_t k, uint32_t ww, uint32_t* splits, uint32_t* kc,
                         uint32_t* ring) {
    const uint32_t groups = k / KG;
    const uint32_t slots = PLAN_CUS;
    const uint32_t want =
        std::min(std::max(1u, slots / tiles), std::max(1u, groups / (MIN_KC / KG)));
    const uint32_t per = cdiv(groups, want);
    *splits = cdiv(groups, per);
    *kc = per * KG;
    const uint32_t units = cdiv(*kc, KS / ww);
    *ring = units >= RING ? RING : (units >= 2 ? 2 : 1);
}

// Column tiles of the slow address class get one split more (fewer rows
// each) when the grid has room for them.  With the weights 1 KB aligned (as
// hipMalloc'd buffers are) and a row pitch that is a multiple of 1 KB, a
// 128-column tile t reads the 256-byte pieces of address class t % 4 in every
// row, and the workgroups of class 1 stream ~11-18 % slower than the others
// (measured per tile: QKV 8.9 against 7.7 us, down 19.1 against 16.2 us); a
// 512-column gate | up tile holds class 1 when t is even (34.4 against
// 31.0 us).  The classes are taken from the tile index alone, so the split
// layout -- and every output bit -- does not depend on where the weights
// are; weights at another alignment only lose the balance.
static void plan_slow_class(Plan* pl, int e, uint32_t k, uint32_t ldw, bool paired,
                            uint32_t up_offset_bytes) {
    SplitGeom& g = pl->geo[e];
    g.tiles = pl->tiles[e]; g.splits = pl->splits[e]; g.kc = pl->kc[e];
    g.splits_slow = g.splits; g.kc_slow = g.kc; g.slow_mask = 0; g.slow_val = 1;
    if ((ldw * 2) % 1024 || up_offset_bytes % 1024) return;
    if (!paired && pl->ww[e] == 1) { g.slow_mask = 3; g.slow_val = 1; }
    else if (paired && pl->ww[e] == 4) { g.slow_mask = 1; g.slow_val = 0; }
    else return;
    uint32_t n_slow = 0;
    for (uint32_t t = 0; t < g.tiles; ++t) n_slow += (t & g.slow_mask) == g.slow_val;
    const uint32_t groups = k / KG;
    const uint32_t per = cdiv(groups, g.splits + 1);
    if (n_slow == 0 || g.tiles * g.splits + n_slow > PLAN_CUS || per * KG < MIN_KC ||
        cdiv(groups, per) != g.splits + 1)
        return;
    g.splits_slow = g.splits + 1;
    g.kc_slow = per * KG;
}

static uint32_t grid_blocks(const SplitGeom& g) {
    uint32_t n = g.tiles * g.splits;
    if (g.splits_slow > g.splits)
        for (uint32_t t = 0; t < g.tiles; ++t) n += (t & g.slow_mask) == g.slow_val;
    return n;
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

static int make_plan(const mb_decoder_step_args* a, Plan* pl) {
    if (!a) return fail(MB_E_ARG, "decoder step: null args");
    if (a->batch < 1 || a->batch > MROWS)
        return fail(MB_E_ARG, "decoder step: batch %u not in 1..%d", a->batch, MROWS);
    if (a->head_dim != DH) return fail(MB_E_ARG, "decoder step: head_dim must be %d", DH);
    if (a->n_heads == 0 || a->n_kv_heads == 0 || a->n_heads % a->n_kv_heads)
        return fail(MB_E_ARG, "decoder step: n_heads %u not a multiple of n_kv_heads %u",
                    a->n_heads, a->n_kv_heads);
    if (a->n_heads / a->n_kv_heads > MAXG)
        return fail(MB_E_ARG, "decoder step: more than %d query heads per kv head", MAXG);
    // The attention width n_heads * head_dim is d_model for a whole layer and
    // smaller for one tensor-parallel shard (its share of the heads; W_o then
    // has n_heads * head_dim rows).
    if ((uint64_t)a->n_heads * DH > 16384)
        return fail(MB_E_ARG, "decoder step: n_heads * head_dim = %llu > 16384",
                    (unsigned long long)a->n_heads * DH);
    if (a->d_model == 0 || a->d_model % BN)
        return fail(MB_E_ARG, "decoder step: d_model %u must be a positive multiple of %d",
                    a->d_model, BN);
    if (a->d_model > 16384)   // the RMSNorm scale reads at most 8 x 16 column-tile sums per row
        return fail(MB_E_ARG, "decoder step: d_model %u > 16384", a->d_model);
    if (a->d_ff == 0 || a->d_ff % KS)
        return fail(MB_E_ARG, "decoder step: d_ff %u must be a positive multiple of %d", a->d_ff,
                    KS);
    if (a->cache_stride < a->cache_len)
        return fail(MB_E_ARG, "decoder step: cache_stride %u < cache_len %u", a->cache_stride,
                    a->cache_len);
    if (!(a->rope_base > 0.f) || !(a->eps >= 0.f))
        return fail(MB_E_ARG, "decoder step: rope_base must be > 0 and eps >= 0");
    const uint32_t D = a->d_model, FF = a->d_ff, B = a->batch, QD = a->n_heads * DH;
    pl->nqkv = QD + 2 * a->n_kv_heads * DH;
    pl->g = a->n_heads / a->n_kv_heads;
    {   // attention: about one workgroup per CU (fewer, longer streams read HBM
        // faster than several per CU); splits of a multiple of AR x 64 keys
        // (the loop runs AR 64-key iterations per trip)
        const uint32_t pairs = B * a->n_kv_heads;
        const uint32_t want = std::max(1u, cdiv(PLAN_CUS, pairs));
        const uint32_t nmax = std::max(1u, cdiv(a->cache_len, AR * AKEYS));
        const uint32_t per = cdiv(std::max(a->cache_len, 1u), std::min(want, nmax));
        pl->split_keys = cdiv(per, AR * AKEYS) * AR * AKEYS;
        pl->nsplit = std::max(1u, cdiv(a->cache_len, pl->split_keys));
        // the ring's loads run up to AR blocks past the split
        if ((uint64_t)(pl->split_keys + AR * AKEYS) * DH * 2 > 0xffffffffull)
            return fail(MB_E_ARG, "decoder step: cache_len %u too large", a->cache_len);
    }
    pl->tiles[EPI_QKV] = pl->nqkv / BN;
    pl->tiles[EPI_WO] = D / BN;
    // W_gate | W_up in 512-column tiles (1 KB row segments) when d_ff allows
    // and there are at least PLAN_CUS / 8 of them. With fewer (d_ff = 1792 of
    // an 8-way shard has 7) each tile is split 32 ways and its last workgroup
    // sums 4 x 32 partial tiles, 1 MB: 27.0 us against 14.3 us for the 28
    // 128-column tiles.
    pl->ww[EPI_QKV] = pl->ww[EPI_WO] = pl->ww[EPI_DOWN] = 1;
    pl->ww[EPI_GU] = FF % (2 * BN) == 0 && FF / (2 * BN) >= PLAN_CUS / 8 ? 4 : 1;
    pl->tiles[EPI_GU] = FF / (BN / 2 * pl->ww[EPI_GU]);
    pl->tiles[EPI_DOWN] = D / BN;
    const uint32_t ldw[4] = {pl->nqkv, D, 2 * FF, D};
    for (int i = 0; i < 4; ++i) {
        const uint32_t k = i == EPI_DOWN ? FF : i == EPI_WO ? QD : D;
        choose_split(pl->tiles[i], k, pl->ww[i], &pl->splits[i], &pl->kc[i], &pl->ring[i]);
        // the ring's clipped loads run up to RING units past the split
        const uint64_t unit = KS / pl->ww[i];
        const uint64_t trips = cdiv(cdiv(pl->kc[i], (uint32_t)unit), pl->ring[i]);
        if ((trips + 1) * pl->ring[i] * unit * ldw[i] * 2 > 0xffffffffull ||
            (uint64_t)B * k * 2 >= 0x80000000ull)
            return fail(MB_E_ARG, "decoder step: shapes too large for 32-bit weight offsets");
        plan_slow_class(pl, i, k, ldw[i], i == EPI_GU, i == EPI_GU ? 2 * FF : 0);
        // (the skinny GEMM's preloaded arguments pack these in 16-bit fields)
        if (pl->geo[i].kc_slow / KG > 0xffffu || pl->geo[i].kc / KG > 0xffffu ||
            pl->geo[i].splits_slow > 0xffffu)
            return fail(MB_E_ARG, "decoder step: K split geometry too large");
    }
    size_t max_part = 0;
    for (int i = 0; i < 4; ++i)
        max_part = std::max(max_part, (size_t)pl->tiles[i] * pl->geo[i].stride() * pl->ww[i]);
    const uint32_t n_counters =
        B * a->n_kv_heads + pl->tiles[EPI_WO] + pl->tiles[EPI_GU] + pl->tiles[EPI_DOWN];
    pl->n_counters = n_counters;
    pl->counter_base[0] = 0;
    pl->counter_base[1] = pl->counter_base[0] + B * a->n_kv_heads;
    pl->counter_base[2] = pl->counter_base[1] + pl->tiles[EPI_WO];
    pl->counter_base[3] = pl->counter_base[2] + pl->tiles[EPI_GU];
    size_t o = 0;
    pl->off_counters = o; o = align256(o + (size_t)n_counters * 4);
    pl->off_partial = o; o = align256(o + max_part * MROWS * BN * 4);
    pl->off_sumsq = o; o = align256(o + (size_t)pl->geo[EPI_QKV].stride() * MROWS * 4);
    pl->off_rope = o; o = align256(o + DH / 2 * 2 * 4);
    pl->off_attn_part = o;
    o = align256(o + (size_t)B * a->n_kv_heads * pl->nsplit * pl->g * APITCH * 4);
    pl->off_attn_out = o; o = align256(o + (size_t)B * QD * 2);
    pl->off_x1 = o; o = align256(o + (size_t)B * D * 4);
    pl->off_x1b = o; o = align256(o + (size_t)B * D * 2);
    pl->off_x1b_lo = o; o = align256(o + (size_t)B * D * 2);
    pl->off_sumsq2 = o; o = align256(o + (size_t)(D / BN) * MROWS * 4);
    pl->off_act = o; o = align256(o + (size_t)B * FF * 2);
    pl->off_act_lo = o; o = align256(o + (size_t)B * FF * 2);
    pl->total = o;
    if (pl->off_attn_out - pl->off_attn_part > 0x7fffffffull ||
        pl->off_sumsq - pl->off_partial > 0x7fffffffull)
        return fail(MB_E_ARG, "decoder step: shapes too large for 32-bit workspace offsets");
    return MB_OK;
}


// A launch timed by its own start/stop events when they are given (per-part
// timing, PartMarks::kernel), a plain launch otherwise.
#define LAUNCH_TIMED(kern, grid, block, s, e0, e1, ...)                                    \
    do {                                                                                   \
        if (e0) hipExtLaunchKernelGGL(kern, grid, block, 0, s, e0, e1, 0, __VA_ARGS__);  \
        else hipLaunchKernelGGL(kern, grid, block, 0, s, __VA_ARGS__);                     \
    } while (0)

template <int EPI, int WW>
void launch_skinny_ww(const GemmCfg& g, uint32_t ring, const StepParams& p, hipStream_t s,
                      hipEvent_t e0, hipEvent_t e1) {
    const dim3 grid(grid_blocks(g.sp)), block(256);
    SkinnyPre q;
    q.w = g.w; q.a = g.a;
    q.a_lo_off = g.a_lo ? (uint32_t)(reinterpret_cast<const uint8_t*>(g.a_lo) -
                                     reinterpret_cast<const uint8_t*>(g.a))
                        : 0u;
    q.ldw = g.ldw; q.lda = g.lda; q.k = g.k;
    q.batch_paired = p.batch | g.paired << 16;
    q.tiles = g.sp.tiles;
    q.splits = g.sp.splits | g.sp.splits_slow << 16;
    q.kc32 = g.sp.kc / KG | (g.sp.kc_slow / KG) << 16;
    q.cls = g.sp.slow_mask | g.sp.slow_val << 16;
    q.ff = p.ff;
    switch (ring) {
        case 1: LAUNCH_TIMED((skinny_gemm_kernel<EPI, WW, 1>), grid, block, s, e0, e1, SKINNY_PRE_ARGS(q), g, p); break;
        case 2: LAUNCH_TIMED((skinny_gemm_kernel<EPI, WW, 2>), grid, block, s, e0, e1, SKINNY_PRE_ARGS(q), g, p); break;
        default: LAUNCH_TIMED((skinny_gemm_kernel<EPI, WW, RING>), grid, block, s, e0, e1, SKINNY_PRE_ARGS(q), g, p); break;
    }
}

template <int EPI>
void launch_skinny(const GemmCfg& g, const Plan& pl, const StepParams& p, hipStream_t s,
                   hipEvent_t e0, hipEvent_t e1) {
    if constexpr (EPI == EPI_GU) {
        if (pl.ww[EPI] == 4) return launch_skinny_ww<EPI, 4>(g, pl.ring[EPI], p, s, e0, e1);
    }
    launch_skinny_ww<EPI, 1>(g, pl.ring[EPI], p, s, e0, e1);
}

int launch_decoder(const mb_decoder_step_args* a, hipStream_t s, PartMarks* pm) {
    Plan pl;
    int rc = make_plan(a, &pl);
    if (rc) return rc;
    if (!a->x || !a->w_qkv || !a->w_o || !a->w_gu || !a->w_down || !a->y || !a->k_new ||
        !a->v_new || (a->cache_len && (!a->k_cache || !a->v_cache)))
        return fail(MB_E_ARG, "decoder step: null pointer");
    const uintptr_t align_or = (uintptr_t)a->x | (uintptr_t)a->w_qkv | (uintptr_t)a->w_o |
                               (uintptr_t)a->w_gu | (uintptr_t)a->w_down |
                               (uintptr_t)a->k_cache | (uintptr_t)a->v_cache | (uintptr_t)a->y |
                               (uintptr_t)a->k_new | (uintptr_t)a->v_new;
    if (align_or & 15) return fail(MB_E_ARG, "decoder step: buffers must be 16-byte aligned");

    uint8_t* ws = static_cast<uint8_t*>(a->workspace);
    if (ws) {
        if (a->workspace_bytes < pl.total)
            return fail(MB_E_ARG, "decoder step: workspace %llu bytes, need %zu",
                        (unsigned long long)a->workspace_bytes, pl.total);
    } else {
        ws = static_cast<uint8_t*>(library_workspace(pl.total));
        if (!ws) return MB_E_HIP;
    }

    StepParams p;
    p.batch = a->batch; p.d = a->d_model; p.qd = a->n_heads * DH;
    p.hq = a->n_heads; p.hkv = a->n_kv_heads; p.g = pl.g;
    p.ff = a->d_ff; p.cache_len = a->cache_len; p.cache_stride = a->cache_stride;
    p.nsplit = pl.nsplit; p.split_keys = pl.split_keys; p.rope_base = a->rope_base; p.eps = a->eps;
    p.x = a->x; p.k_cache = a->k_cache; p.v_cache = a->v_cache;
    p.y = a->y; p.k_new = a->k_new; p.v_new = a->v_new;
    uint32_t* counters = reinterpret_cast<uint32_t*>(ws + pl.off_counters);
    p.counters = counters;
    p.n_counters = pl.n_counters;
    p.attn_counters = counters + pl.counter_base[0];
    p.partial = reinterpret_cast<float*>(ws + pl.off_partial);
    p.partial_bytes = (uint32_t)(pl.off_sumsq - pl.off_partial);
    p.sumsq_bytes = (uint32_t)(pl.off_rope - pl.off_sumsq);
    p.attn_part_bytes = (uint32_t)(pl.off_attn_out - pl.off_attn_part);
    p.sumsq = reinterpret_cast<float*>(ws + pl.off_sumsq);
    p.rope = reinterpret_cast<float*>(ws + pl.off_rope);
    p.qkv_sp = pl.geo[EPI_QKV];
    p.attn_part = reinterpret_cast<float*>(ws + pl.off_attn_part);
    p.attn_out = reinterpret_cast<uint16_t*>(ws + pl.off_attn_out);
    p.x1 = reinterpret_cast<float*>(ws + pl.off_x1);
    p.x1b = reinterpret_cast<uint16_t*>(ws + pl.off_x1b);
    p.x1b_lo = reinterpret_cast<uint16_t*>(ws + pl.off_x1b_lo);
    p.sumsq2 = reinterpret_cast<float*>(ws + pl.off_sumsq2);
    p.act = reinterpret_cast<uint16_t*>(ws + pl.off_act);
    p.act_lo = reinterpret_cast<uint16_t*>(ws + pl.off_act_lo);

    const uint32_t D = a->d_model, FF = a->d_ff, QD = a->n_heads * DH;
    auto gemm = [&](int epi, const uint16_t* act, const uint16_t* act_lo, uint32_t lda,
                    const uint16_t* w, uint32_t ldw, uint32_t k, uint32_t counter_base) -> GemmCfg {
        GemmCfg g;
        g.a = act; g.a_lo = act_lo; g.lda = lda; g.w = w; g.ldw = ldw; g.k = k;
        g.sp = pl.geo[epi];
        g.paired = epi == EPI_GU ? 1u : 0u;
        g.counters = counters + counter_base;
        return g;
    };
    const GemmCfg g_qkv =
        gemm(EPI_QKV, a->x, nullptr, D, a->w_qkv, pl.nqkv, D, 0);   // (no counters)
    const GemmCfg g_wo =
        gemm(EPI_WO, p.attn_out, nullptr, QD, a->w_o, D, QD, pl.counter_base[1]);
    const GemmCfg g_gu =
        gemm(EPI_GU, p.x1b, p.x1b_lo, D, a->w_gu, 2 * FF, D, pl.counter_base[2]);
    const GemmCfg g_dn =
        gemm(EPI_DOWN, p.act, p.act_lo, FF, a->w_down, D, FF, pl.counter_base[3]);

    auto next_units = [&](int e, const uint16_t* w, uint32_t ldw, uint32_t k, uint32_t seg2) {
        NextUnits c;
        const uint64_t bytes = (uint64_t)k * ldw * 2;
        c.w = bytes <= 0xffffffffull ? reinterpret_cast<const uint8_t*>(w) : nullptr;
        c.bytes = (uint32_t)std::min<uint64_t>(bytes, 0xffffffffull);
        c.ldw_bytes = ldw * 2; c.sp = pl.geo[e]; c.k = k;
        c.ur = KS / pl.ww[e];                                    // k rows per unit
        c.seg_bytes = seg2 ? 128 * pl.ww[e] : 256 * pl.ww[e];   // (paired: each half)
        c.seg2_off = seg2;
        return c;
    };
    p.next[EPI_QKV] = NextUnits{};
    p.next[EPI_WO] = next_units(EPI_WO, a->w_o, D, QD, 0);
    p.next[EPI_GU] = next_units(EPI_GU, a->w_gu, 2 * FF, D, 2 * FF);
    p.next[EPI_DOWN] = next_units(EPI_DOWN, a->w_down, D, FF, 0);
    // each part is one kernel; when parts are timed, by its own events
    hipEvent_t e0 = nullptr, e1 = nullptr;
    auto part = [&](const char* name) { if (pm) pm->kernel(name, &e0, &e1); };
    part("qkv");
    launch_skinny<EPI_QKV>(g_qkv, pl, p, s, e0, e1);
    MB_LAUNCH_CHECK("decoder qkv");
    part("attention");
    {
        const dim3 grid(a->batch * a->n_kv_heads * pl.nsplit), block(256);
        if (pl.g <= 4) LAUNCH_TIMED(attention_kernel<4>, grid, block, s, e0, e1, p);
        else if (pl.g <= 8) LAUNCH_TIMED(attention_kernel<8>, grid, block, s, e0, e1, p);
        else LAUNCH_TIMED(attention_kernel<16>, grid, block, s, e0, e1, p);
    }
    MB_LAUNCH_CHECK("decoder attention");
    part("wo_residual");
    launch_skinny<EPI_WO>(g_wo, pl, p, s, e0, e1);
    MB_LAUNCH_CHECK("decoder wo_residual");
    part("gate_up_swiglu");
    launch_skinny<EPI_GU>(g_gu, pl, p, s, e0, e1);
    MB_LAUNCH_CHECK("decoder gate_up_swiglu");
    part("down_residual");
    launch_skinny<EPI_DOWN>(g_dn, pl, p, s, e0, e1);
    MB_LAUNCH_CHECK("decoder down_residual");
    return MB_OK;
}

// Registry launcher (mlx/kernels/full/registry.py "llama_decoder_step"):
// x@0 W_qkv@1 W_o@2 W_gu@3 W_down@4 K_cache@5 V_cache@6 (bf16 inputs), y@7
// k_new@8 v_new@9 (bf16 outputs), B@10 D@11 H@12 Hkv@13 FF@14 L@15 (u32),
// rope_base@16 eps@17 (f32).  The caches are dense: cache_stride = L.
int run_decoder(const Bindings& bs, hipStream_t s, PartMarks* pm) {
    uint32_t B, D, H, HKV, FF, L;
    float base, eps;
    int rc;
    if ((rc = bs.u32(10, &B, "B")) || (rc = bs.u32(11, &D, "D")) || (rc = bs.u32(12, &H, "H")) ||
        (rc = bs.u32(13, &HKV, "H_kv")) || (rc = bs.u32(14, &FF, "FF")) ||
        (rc = bs.u32(15, &L, "L")) || (rc = bs.f32(16, &base, "rope_base")) ||
        (rc = bs.f32(17, &eps, "eps")))
        return rc;
    mb_decoder_step_args a = {};
    a.batch = B; a.d_model = D; a.n_heads = H; a.n_kv_heads = HKV; a.head_dim = DH; a.d_ff = FF;
    a.cache_len = L; a.cache_stride = L; a.rope_base = base; a.eps = eps;
    Plan pl;
    if ((rc = make_plan(&a, &pl))) return rc;
    const uint64_t nqkv = pl.nqkv, kv = (uint64_t)B * HKV * L * DH;
    void* ptr[10];
    if ((rc = bs.buffer(0, MB_DTYPE_BF16, (uint64_t)B * D * 2, false, &ptr[0], "x")) ||
        (rc = bs.buffer(1, MB_DTYPE_BF16, (uint64_t)D * nqkv * 2, false, &ptr[1], "W_qkv")) ||
        (rc = bs.buffer(2, MB_DTYPE_BF16, (uint64_t)H * DH * D * 2, false, &ptr[2], "W_o")) ||
        (rc = bs.buffer(3, MB_DTYPE_BF16, (uint64_t)D * 2 * FF * 2, false, &ptr[3], "W_gu")) ||
        (rc = bs.buffer(4, MB_DTYPE_BF16, (uint64_t)FF * D * 2, false, &ptr[4], "W_down")) ||
        (rc = bs.buffer(5, MB_DTYPE_BF16, kv * 2, false, &ptr[5], "K_cache")) ||
        (rc = bs.buffer(6, MB_DTYPE_BF16, kv * 2, false, &ptr[6], "V_cache")) ||
        (rc = bs.buffer(7, MB_DTYPE_BF16, (uint64_t)B * D * 2, true, &ptr[7], "y")) ||
        (rc = bs.buffer(8, MB_DTYPE_BF16, (uint64_t)B * HKV * DH * 2, true, &ptr[8], "k_new")) ||
        (rc = bs.buffer(9, MB_DTYPE_BF16, (uint64_t)B * HKV * DH * 2, true, &ptr[9], "v_new")))
        return rc;
    a.x = (const uint16_t*)ptr[0]; a.w_qkv = (const uint16_t*)ptr[1];
    a.w_o = (const uint16_t*)ptr[2]; a.w_gu = (const uint16_t*)ptr[3];
    a.w_down = (const uint16_t*)ptr[4]; a.k_cache = (const uint16_t*)ptr[5];
    a.v_cache = (const uint16_t*)ptr[6]; a.y = (uint16_t*)ptr[7];
    a.k_new = (uint16_t*)ptr[8]; a.v_new = (uint16_t*)ptr[9];
    a.workspace = nullptr;
    a.workspace_bytes = 0;
    return launch_decoder(&a, s, pm);
}

// ---- allocation-free entry point ------------------------------------------------------
// mb_launch_llama_decoder_step_bf16_noalloc runs the same five kernels with
// their workspace in `scratch`, a file-scope device array that the code
// object carries, so the call allocates nothing (callers under HIP graph
// capture or in allocation-free serving loops).  Each device holds its own
// copy of the array for the life of the process; host code uses the device
// address hipGetSymbolAddress returns for it (kept per device in
// g_scratch), never the array's name, which in host code is only a
// host-side stand-in.  Nothing needs clearing before a call: the step's
// first kernel zeroes the completion counters the later ones use, so a call
// -- or a replay of a HIP graph that captured one -- is correct whatever an
// earlier call of other shapes left in the scratch.  Every call on a device
// shares its scratch: calls that overlap on one device race.
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)32 << 20;   // 32 MiB (11.3 MB at the benchmark shape)
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];
static_assert(NOALLOC_SCRATCH_BYTES == MB_DECODER_NOALLOC_MAX_BYTES, "mbhip.h states the limit");

constexpr int MAX_DEVICES = 64;
struct DeviceScratch {
    void* ptr = nullptr;     // device address of `scratch` on that device
};
DeviceScratch g_scratch[MAX_DEVICES];
std::mutex g_scratch_mutex;

// Looks up the scratch of the current device (once per device, with that
// device current).
int scratch_of_current_device(DeviceScratch** out) {
    int dev = -1;
    MB_HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= MAX_DEVICES)
        return fail(MB_E_NO_DEVICE, "decoder scratch: device %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    DeviceScratch& d = g_scratch[dev];
    if (!d.ptr) {
        void* ptr = nullptr;
        hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return fail(MB_E_HIP, "hipGetSymbolAddress(scratch) on device %d failed: %s", dev,
                        hipGetErrorString(e));
        d.ptr = ptr;
    }
    *out = &d;
    return MB_OK;
}

int launch_decoder_noalloc(const mb_decoder_step_args* a, hipStream_t s) {
    Plan pl;
    int rc = make_plan(a, &pl);
    if (rc) return rc;
    if (a->workspace)
        return fail(MB_E_ARG, "decoder step (no-alloc): workspace must be NULL, this entry point "
                              "uses the library's static scratch");
    if (pl.total > NOALLOC_SCRATCH_BYTES)
        return fail(MB_E_ARG, "decoder step (no-alloc): these shapes need %zu bytes of scratch; "
                              "the static scratch holds %zu", pl.total, NOALLOC_SCRATCH_BYTES);
    DeviceScratch* d = nullptr;
    if ((rc = scratch_of_current_device(&d))) return rc;
    // (the step's QKV kernel clears the counters: no clearing here, so a
    // captured graph of this call is complete)
    mb_decoder_step_args b = *a;
    b.workspace = d->ptr;
    b.workspace_bytes = NOALLOC_SCRATCH_BYTES;
    return launch_decoder(&b, s, nullptr);
}

}  // namespace

int init_decoder_scratch() {
    DeviceScratch* d = nullptr;
    return scratch_of_current_device(&d);
}

void register_decoder() {
    register_kernel({"llama_decoder_step_bf16", run_decoder,
                     reinterpret_cast<const void*>(&skinny_gemm_kernel<EPI_GU, 4, RING>), 5});
}

}  // namespace mb

extern "C" uint64_t mb_decoder_step_workspace_bytes(const mb_decoder_step_args* args) {
    mb::clear_error();
    mb::Plan pl;
    if (mb::make_plan(args, &pl)) return 0;
    return pl.total;
}

extern "C" int mb_launch_llama_decoder_step_bf16(const mb_decoder_step_args* args, void* stream) {
    mb::clear_error();
    if (!mb::initialized()) return mb::fail(MB_E_STATE, "mb_init() has not been called");
    return mb::launch_decoder(args, mb::stream_or_default(stream), nullptr);
}

extern "C" int mb_launch_llama_decoder_step_bf16_noalloc(const mb_decoder_step_args* args,
                                                         void* stream) {
    mb::clear_error();
    if (!mb::initialized()) return mb::fail(MB_E_STATE, "mb_init() has not been called");
    return mb::launch_decoder_noalloc(args, mb::stream_or_default(stream));
}
