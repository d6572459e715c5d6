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
//   1. qkv_rope       skinny GEMM x @ W_qkv, finisher applies the RMSNorm row
//                     scale (sum of squares gathered from the A operand for
//                     free), RoPE, writes q (bf16, pre-scaled by 1/sqrt(Dh))
//                     and k_new / v_new (bf16);
//   2. attention      flash-decoding: one workgroup per (sequence, kv head,
//                     split of the cached keys); q.k^T on MFMA, online
//                     softmax, p.v on VALU; the last split to finish merges
//                     the splits and the new token (log-sum-exp);
//   3. wo_residual    skinny GEMM attn @ W_o, finisher adds x, writes x1
//                     (fp32 + bf16) and per-tile sums of x1^2;
//   4. gate_up_swiglu skinny GEMM x1 @ [W_gate | W_up], each tile holding 64
//                     gate and the matching 64 up columns, finisher applies
//                     the RMSNorm scale and silu(g) * u;
//                     x1 and the SwiGLU output feed the next GEMMs as hi + lo
//                     bf16 pairs (two MFMAs), so their bf16 rounding does not
//                     accumulate over K = 4096 / 14336 terms;
//   5. down_residual  skinny GEMM act @ W_down, finisher adds x1, writes y.
// RMSNorm is a per-row scale, so (r x) W = r (x W): it is applied to the GEMM
// outputs instead of materialising h / h2.
//
// Skinny GEMM (M = batch <= 16): a workgroup owns a 128-column tile and one
// K split.  The weights are row-major [K][N] (x @ W), but the MFMA operand
// wants 8 consecutive k per lane, so each lane loads an 8(k) x 8(n) block as
// eight 16-byte rows (one 256-byte row segment per 16 lanes), transposes it in
// registers with v_perm_b32 and stores eight K-contiguous 16-byte chunks into
// LDS (pitch 136 bf16, chunk index XOR-swizzled by (row / 16) so both the
// stores and the ds_read_b128 operand reads are bank-conflict free).  The
// activations are the MFMA A operand (16 rows = the batch, zero-filled above
// it), parked in LDS before the weights arrive.  Weights are loaded
// non-temporal (each byte is read once per step).
// v_mfma_f32_16x16x32_bf16 accumulates; split-K
// partials go to the workspace and the LAST workgroup of each column tile (an
// atomic counter, reset by that workgroup) sums them and runs the epilogue;
// the partials travel through device-coherent (sc1) accesses, not fences.
#include "common.h"

#include <math.h>

#include <algorithm>

namespace mb {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int DH = 128;        // head_dim (fixed)
constexpr int MROWS = 16;      // MFMA rows = max batch
constexpr int BN = 128;        // skinny GEMM column tile
constexpr int KS = 128;        // k rows per LDS step
constexpr int WP = KS + 8;     // LDS pitch (bf16) of one transposed weight column
constexpr int MAXG = 16;       // query heads per kv head (MFMA columns)

enum { EPI_QKV = 0, EPI_WO = 1, EPI_GU = 2, EPI_DOWN = 3 };

__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

__device__ __forceinline__ uint16_t f2bf(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }

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
    uint32_t batch, d, hq, hkv, g, ff, cache_len, cache_stride, nsplit, split_keys;
    float rope_base, eps;
    const uint16_t *x, *k_cache, *v_cache;
    uint16_t *y, *k_new, *v_new;
    uint32_t* attn_counters;   // [B * Hkv]
    float* partial;            // split-K partials [tiles * splits][BN][16] (column-major tile)
    uint32_t partial_bytes;
    float* sumsq;              // [qkv tiles * splits][16] sum of x^2 over each split
    uint16_t* q;               // [B][D] rotated queries * 1/sqrt(Dh), bf16 (MFMA operand)
    float* attn_part;          // [B][Hkv][nsplit][G][DH + 4]  (o[DH], m, l, pad)
    uint32_t attn_part_bytes;
    uint32_t sumsq_bytes;
    uint16_t* attn_out;        // [B][D]
    float* x1;                 // [B][D]
    uint16_t* x1b;             // [B][D]  bf16(x1)
    uint16_t* x1b_lo;          // [B][D]  bf16(x1 - bf16(x1))
    float* sumsq2;             // [D / 128][16] sum of x1^2 per column tile
    uint16_t* act;             // [B][FF] bf16(silu(g) u)
    uint16_t* act_lo;          // [B][FF] its rounding remainder
};

struct GemmCfg {
    const uint16_t* a;     // activations [batch][k], row stride lda (rows >= batch read as 0)
    const uint16_t* a_lo;  // optional second bf16 term of the activations (same layout)
    uint32_t lda;
    const uint16_t* w;     // weights [k][ldw]
    uint32_t ldw;
    uint32_t k, kc, splits, tiles;
    uint32_t paired;       // 1: tile t = gate cols [64t, 64t+64) + up cols ff + [64t, 64t+64)
    uint32_t* counters;    // [tiles]
};

__device__ __forceinline__ uint32_t tile_col(const GemmCfg& g, const StepParams& p, uint32_t tile,
                                             uint32_t c) {
    if (!g.paired) return tile * BN + c;
    return c < 64 ? tile * 64 + c : p.ff + tile * 64 + (c - 64);
}

// ---- skinny GEMM + split-K finisher --------------------------------------------------

// A workgroup owns one 128-column tile and one K split of NSTEPS x 128 rows
// (NSTEPS = 1, 2 or 4).  The step is HBM bound with long memory latency under
// load, so what matters is bytes in flight per CU:
//   1. the split's activation slice (16 rows x NSTEPS*128, hi and lo terms) is
//      loaded first and parked in LDS, so the MFMA A fragments come from LDS
//      (lgkmcnt) and never sit in the vmcnt queue ahead of weight data;
//   2. then ALL of the split's weight loads are issued at once (NSTEPS x 32 KB
//      per workgroup, two workgroups per CU);
//   3. step s waits only for its own weight rows (vmcnt = 8 x steps still in
//      flight behind them), transposes them through LDS and runs its MFMAs.
// sched_barrier keeps the compiler from interleaving these groups, because
// vmcnt retires loads in issue order.
template <int EPI, int NSTEPS>
__global__ __launch_bounds__(256, 2)
void skinny_gemm_kernel(GemmCfg g, StepParams p) {
    constexpr bool SPLIT_A = (EPI == EPI_GU || EPI == EPI_DOWN);   // hi + lo activations
    constexpr int NTERMS = SPLIT_A ? 2 : 1;
    constexpr int KC = NSTEPS * KS;                 // k rows of this split
    constexpr int AP = KC + 8;                      // LDS pitch (bf16) of an activation row
    constexpr int ACH = MROWS * KC / 8 / 256;       // 16-byte activation chunks per thread per term

    __shared__ __attribute__((aligned(16))) uint16_t wt[BN * WP];
    __shared__ __attribute__((aligned(16))) uint16_t as[NTERMS][MROWS * AP];
    float* red = reinterpret_cast<float*>(wt);   // finisher sums, after the K loop
    __shared__ float red_ss[MROWS];
    __shared__ uint32_t s_last;

    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t tile = blockIdx.x % g.tiles;
    const uint32_t split = blockIdx.x / g.tiles;
    const uint32_t k_begin = split * KC;

    // ---- 1. activations -> registers (issued first) ----
    // chunk q (0 .. 16*KC/8): row q / (KC/8), k octet q % (KC/8)
    u32x4 ar[NTERMS][ACH];
#pragma unroll
    for (int t = 0; t < NTERMS; ++t) {
        const uint16_t* src = t == 0 ? g.a : g.a_lo;
#pragma unroll
        for (int i = 0; i < ACH; ++i) {
            const uint32_t q = tid + 256 * i, row = q / (KC / 8), oct = q % (KC / 8);
            const bool ok = row < p.batch;
            // rows past the batch read row 0 (valid) and are zeroed
            const u32x4 v = *reinterpret_cast<const u32x4*>(
                src + (size_t)(ok ? row : 0) * g.lda + k_begin + 8 * oct);
            ar[t][i] = ok ? v : u32x4{};
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- 2. every weight load of the split ----
    const uint32_t co = tid & 15, ko = tid >> 4;
    const uint16_t* wp = g.w + (size_t)(k_begin + 8 * ko) * g.ldw + tile_col(g, p, tile, 8 * co);
    u32x4 r[NSTEPS][8];
#pragma unroll
    for (int s = 0; s < NSTEPS; ++s)
#pragma unroll
        for (int i = 0; i < 8; ++i)
            r[s][i] = __builtin_nontemporal_load(   // streamed once per step
                reinterpret_cast<const u32x4*>(wp + (size_t)(s * KS + i) * g.ldw));
    __builtin_amdgcn_sched_barrier(0);

    // ---- epilogue inputs, in case this workgroup finishes the tile ----
    // (issued behind the weights, so no weight wait grows; the finisher then
    // needs one memory round trip, for the other splits' partials)
    const uint32_t eb = tid >> 4, ec = 8 * (tid & 15);   // epilogue: row eb, columns ec .. ec+7
    u32x4 pre_x = {};                                    // WO: x (bf16)
    f32x4 pre_x1[2] = {f32x4{}, f32x4{}};                // DOWN: x1 (fp32)
    float pre_ss[8] = {};                                // GU: sumsq2 terms, see finish_rows
    if (EPI == EPI_WO)
        pre_x = *reinterpret_cast<const u32x4*>(p.x + (size_t)(eb < p.batch ? eb : 0) * p.d +
                                                tile * BN + ec);
    if (EPI == EPI_DOWN) {
        const float* src = p.x1 + (size_t)(eb < p.batch ? eb : 0) * p.d + tile * BN + ec;
        pre_x1[0] = *reinterpret_cast<const f32x4*>(src);
        pre_x1[1] = *reinterpret_cast<const f32x4*>(src + 4);
    }
    if (EPI == EPI_GU) {
        const uint32_t ntile = p.d / BN;
#pragma unroll
        for (int u = 0; u < 8; ++u)
            pre_ss[u] = p.sumsq2[min(eb + 16u * u, ntile - 1) * MROWS + (tid & 15)];
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- activations -> LDS (they are the oldest loads) ----
#pragma unroll
    for (int t = 0; t < NTERMS; ++t)
#pragma unroll
        for (int i = 0; i < ACH; ++i) {
            const uint32_t q = tid + 256 * i, row = q / (KC / 8), oct = q % (KC / 8);
            *reinterpret_cast<u32x4*>(&as[t][row * AP + 8 * oct]) = ar[t][i];
        }
    __builtin_amdgcn_sched_barrier(0);

    const uint32_t arow = lane & 15, agrp = lane >> 4;
    f32x4 acc[2] = {f32x4{}, f32x4{}};
    float ss = 0.f;

    // ---- 3. steps ----
#pragma unroll
    for (int s = 0; s < NSTEPS; ++s) {
        // 8x8 transpose of this lane's block: LDS row (8co + c) = weight
        // column, 16-byte chunk ko (XOR-swizzled by row/16) = k octet.
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            uint32_t lo[4], hi[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                lo[j] = __builtin_amdgcn_perm(r[s][2 * j + 1][m], r[s][2 * j][m], 0x05040100u);
                hi[j] = __builtin_amdgcn_perm(r[s][2 * j + 1][m], r[s][2 * j][m], 0x07060302u);
            }
            const uint32_t row0 = 8 * co + 2 * m, row1 = row0 + 1;
            *reinterpret_cast<u32x4*>(wt + row0 * WP + 8 * (ko ^ ((row0 >> 4) & 7))) =
                u32x4{lo[0], lo[1], lo[2], lo[3]};
            *reinterpret_cast<u32x4*>(wt + row1 * WP + 8 * (ko ^ ((row1 >> 4) & 7))) =
                u32x4{hi[0], hi[1], hi[2], hi[3]};
        }
        __syncthreads();
        bf16x8 a[4], alo[4];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            const uint32_t ao = arow * AP + s * KS + 32 * kb + 8 * agrp;
            a[kb] = *reinterpret_cast<const bf16x8*>(&as[0][ao]);
            if (SPLIT_A) alo[kb] = *reinterpret_cast<const bf16x8*>(&as[NTERMS - 1][ao]);
        }
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            const uint32_t row = (wave * 2 + cb) * 16 + (lane & 15);
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                const uint32_t chunk = (4 * kb + agrp) ^ ((row >> 4) & 7);
                const bf16x8 bfrag = *reinterpret_cast<const bf16x8*>(wt + row * WP + 8 * chunk);
                acc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[kb], bfrag, acc[cb], 0, 0, 0);
                if (SPLIT_A)
                    acc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(alo[kb], bfrag, acc[cb], 0,
                                                                       0, 0);
            }
        }
        if (EPI == EPI_QKV && wave == 0) {   // RMSNorm statistics from the A operand
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float v = (float)a[kb][e];
                    ss += v * v;
                }
        }
        __syncthreads();
    }

    // Split-K partial, column-major per tile: lane holds rows 4*agrp .. +3 of
    // column (wave*2 + cb)*16 + lane%16 -> one 16-byte sc1 store.
    const __amdgpu_buffer_rsrc_t prs = coherent_rsrc(p.partial, p.partial_bytes);
    const uint32_t part_base = (tile * g.splits + split) * (MROWS * BN * 4);
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
        const uint32_t c = (wave * 2 + cb) * 16 + (lane & 15);
        st_sc1(prs, part_base + (c * MROWS + 4 * agrp) * 4, acc[cb]);
    }
    const __amdgpu_buffer_rsrc_t srs = coherent_rsrc(p.sumsq, p.sumsq_bytes);
    if (EPI == EPI_QKV && wave == 0) {
        ss += __shfl_xor(ss, 16);
        ss += __shfl_xor(ss, 32);
        if (lane < 16) st_sc1(srs, ((tile * g.splits + split) * MROWS + lane) * 4, ss);
    }
    if (!arrive_last(&g.counters[tile], g.splits, &s_last)) return;

    // ---- finisher: this workgroup is the last of its tile ----
    // float4 q of a tile = column q/4, rows 4*(q%4) .. +3; sum over the splits
    // with eight splits' loads in flight together (past the last split the
    // last one is re-read and dropped, so no load sits behind a branch).
    {
        constexpr uint32_t SPLIT_BYTES = MROWS * BN * 4, SB = 8;
        const uint32_t tile_base = tile * g.splits * SPLIT_BYTES;
        f32x4 v0 = {}, v1 = {};
        for (uint32_t sp0 = 0; sp0 < g.splits; sp0 += SB) {
            f32x4 a[SB], b[SB];
#pragma unroll
            for (uint32_t u = 0; u < SB; ++u) {
                const uint32_t o = tile_base + min(sp0 + u, g.splits - 1) * SPLIT_BYTES;
                a[u] = ld4_sc1(prs, o + tid * 16);
                b[u] = ld4_sc1(prs, o + (256 + tid) * 16);
            }
#pragma unroll
            for (uint32_t u = 0; u < SB; ++u)
                if (sp0 + u < g.splits) { v0 += a[u]; v1 += b[u]; }
        }
        // red is row-major [16][BN] for the epilogues
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t q = tid + 256 * h, c = q >> 2, r0 = 4 * (q & 3);
            const f32x4 v = h ? v1 : v0;
#pragma unroll
            for (int e = 0; e < 4; ++e) red[(r0 + e) * BN + c] = v[e];
        }
    }
    // Row statistics, thread (row = tid % 16, group = tid / 16) summing every
    // 16th term, then the 16 groups through LDS:
    //   QKV: sum of x^2 over the splits (sc1 loads, all in flight together);
    //   GU:  sum of x1^2 over the W_o column tiles (prefetched) -> RMSNorm scale.
    if (EPI == EPI_QKV || EPI == EPI_GU) {
        float* scratch = red + MROWS * BN;   // 16 x 16 floats past the tile sums
        const uint32_t row = tid & 15, grp = tid >> 4;
        float v = 0.f;
        if (EPI == EPI_QKV) {
            constexpr uint32_t UT = 8;
            for (uint32_t t0 = 0; t0 < g.splits; t0 += 16 * UT) {
                float x[UT];
#pragma unroll
                for (uint32_t u = 0; u < UT; ++u) {
                    const uint32_t t = min(t0 + grp + 16 * u, g.splits - 1);
                    x[u] = ld_sc1(srs, ((tile * g.splits + t) * MROWS + row) * 4);
                }
#pragma unroll
                for (uint32_t u = 0; u < UT; ++u)
                    if (t0 + grp + 16 * u < g.splits) v += x[u];
            }
        } else {
#pragma unroll
            for (uint32_t u = 0; u < 8; ++u)
                if (grp + 16 * u < p.d / BN) v += pre_ss[u];
        }
        scratch[grp * MROWS + row] = v;
        __syncthreads();
        if (tid < MROWS) {
            float t = 0.f;
#pragma unroll
            for (int q = 0; q < 16; ++q) t += scratch[q * MROWS + tid];
            red_ss[tid] = EPI == EPI_QKV ? t : rsqrtf(t / (float)p.d + p.eps);
        }
    }
    __syncthreads();

    if (EPI == EPI_QKV) {
        // Tile = one head of Q, K or V (all three regions are multiples of 128).
        const uint32_t base = tile * BN;
        const uint32_t i = tid & 63;                       // rotation pair (2i, 2i+1)
        const float omega = powf(p.rope_base, -2.0f * (float)i / (float)DH);
        float sn, cs;
        sincosf((float)p.cache_len * omega, &sn, &cs);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const uint32_t b = 4 * (tid >> 6) + rr;
            if (b >= p.batch) continue;
            const float r1 = rsqrtf(red_ss[b] / (float)p.d + p.eps);
            const float v0 = red[b * BN + 2 * i] * r1, v1 = red[b * BN + 2 * i + 1] * r1;
            if (base < p.d) {
                // pre-scaled by 1/sqrt(Dh) and rounded once for the q.k^T MFMA
                const float qs = rsqrtf((float)DH);
                uint16_t* qd = p.q + (size_t)b * p.d + base + 2 * i;
                qd[0] = f2bf((v0 * cs - v1 * sn) * qs);
                qd[1] = f2bf((v0 * sn + v1 * cs) * qs);
            } else if (base < p.d + p.hkv * DH) {
                const uint32_t kvh = (base - p.d) / DH;
                uint16_t* kd = p.k_new + ((size_t)b * p.hkv + kvh) * DH + 2 * i;
                kd[0] = f2bf(v0 * cs - v1 * sn);
                kd[1] = f2bf(v0 * sn + v1 * cs);
            } else {
                const uint32_t kvh = (base - p.d - p.hkv * DH) / DH;
                uint16_t* vd = p.v_new + ((size_t)b * p.hkv + kvh) * DH + 2 * i;
                vd[0] = f2bf(v0);
                vd[1] = f2bf(v1);
            }
        }
    } else if (EPI == EPI_WO) {
        // thread: row eb, columns ec .. ec+7; x1 = x + attn W_o
        float v[8];
        float sq = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t xb = pre_x[e / 2] >> (16 * (e & 1));
            v[e] = eb < p.batch ? bf2f((uint16_t)xb) + red[eb * BN + ec + e] : 0.f;
            sq += v[e] * v[e];
        }
        if (eb < p.batch) {
            const size_t o = (size_t)eb * p.d + tile * BN + ec;
            *reinterpret_cast<f32x4*>(p.x1 + o) = f32x4{v[0], v[1], v[2], v[3]};
            *reinterpret_cast<f32x4*>(p.x1 + o + 4) = f32x4{v[4], v[5], v[6], v[7]};
            u32x4 hi, lo;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint16_t h0 = f2bf(v[2 * e]), h1 = f2bf(v[2 * e + 1]);
                hi[e] = (uint32_t)h0 | ((uint32_t)h1 << 16);
                lo[e] = (uint32_t)f2bf(v[2 * e] - bf2f(h0)) |
                        ((uint32_t)f2bf(v[2 * e + 1] - bf2f(h1)) << 16);
            }
            *reinterpret_cast<u32x4*>(p.x1b + o) = hi;
            *reinterpret_cast<u32x4*>(p.x1b_lo + o) = lo;
        }
        // row sums of x1^2 over the tile: the 16 threads of a row are 16 adjacent lanes
#pragma unroll
        for (int o2 = 8; o2 > 0; o2 >>= 1) sq += __shfl_xor(sq, o2);
        if ((tid & 15) == 0) p.sumsq2[tile * MROWS + eb] = sq;
    } else if (EPI == EPI_GU) {
#pragma unroll
        for (int i = 0; i < (MROWS * 64) / 256; ++i) {
            const uint32_t idx = tid + 256 * i, b = idx / 64, c = idx % 64;
            if (b >= p.batch) continue;
            const float r2 = red_ss[b];
            const float gate = red[b * BN + c] * r2, up = red[b * BN + 64 + c] * r2;
            const float av = silu(gate) * up;
            const uint16_t hi = f2bf(av);
            const size_t o = (size_t)b * p.ff + tile * 64 + c;
            p.act[o] = hi;
            p.act_lo[o] = f2bf(av - bf2f(hi));
        }
    } else {   // EPI_DOWN: y = x1 + act W_down; thread: row eb, columns ec .. ec+7
        if (eb < p.batch) {
            u32x4 out;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float y0 = pre_x1[e / 2][2 * (e & 1)] + red[eb * BN + ec + 2 * e];
                const float y1 = pre_x1[e / 2][2 * (e & 1) + 1] + red[eb * BN + ec + 2 * e + 1];
                out[e] = (uint32_t)f2bf(y0) | ((uint32_t)f2bf(y1) << 16);
            }
            *reinterpret_cast<u32x4*>(p.y + (size_t)eb * p.d + tile * BN + ec) = out;
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
constexpr int APITCH = DH + 4;            // floats per (split, head) partial: o[DH], m, l, pad
constexpr int QP = DH + 8;                // LDS pitch (bf16) of a query row
constexpr float NEG_BIG = -1.0e30f;       // "no key yet": finite, so max/exp never see inf - inf
constexpr float LOG2E = 1.4426950408889634f;
constexpr uint32_t ATTN_WGS = 1024;      // attention grid target: 4 workgroups per CU

__device__ __forceinline__ void* uniform_ptr(const void* ptr) {
    const uint64_t v = reinterpret_cast<uint64_t>(ptr);
    const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<void*>((hi << 32) | lo);
}

struct KVBlock {
    u32x4 k[4];      // K[key j][32 m + 8 grp .. + 8] for the scores MFMA, m < 4
    uint32_t v[16];  // V[key i][2 lane, 2 lane + 1], i < 16
};

template <int GT>
__global__ __launch_bounds__(256)
void attention_kernel(StepParams p) {
    __shared__ uint16_t qs[16][QP];        // q rows of this kv head (rows past G zero)
    __shared__ float xp[4][16][16];       // per wave: p[key][head] of the current block
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
    const uint16_t* knew = p.k_new + (size_t)bk * DH;
    const uint16_t* vnew = p.v_new + (size_t)bk * DH;

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

    // q rows of the G heads go to LDS (the MFMA B operand is re-read per
    // block); their loads are issued ahead of the first K/V block.
    static_assert(16 * (DH / 8) == 256, "one 16-byte q chunk per thread");
    const uint32_t qh = tid / (DH / 8), qc = tid % (DH / 8);
    const u32x4 qv = *reinterpret_cast<const u32x4*>(
        p.q + (size_t)b * p.d + (kvh * G + (qh < G ? qh : 0)) * DH + 8 * qc);
    KVBlock ba, bb;
    load(ba, 0);
    __builtin_amdgcn_sched_barrier(0);
    *reinterpret_cast<u32x4*>(&qs[qh][8 * qc]) = qh < G ? qv : u32x4{};
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

    // sched_barrier pins the order: a block's loads are issued right after the
    // previous block's compute, so exactly two blocks are ever live.
    for (uint32_t t = 0; t < nblk; t += 2) {
        __builtin_amdgcn_sched_barrier(0);
        load(bb, t + 1);
        __builtin_amdgcn_sched_barrier(0);
        compute(ba, t);
        __builtin_amdgcn_sched_barrier(0);
        load(ba, t + 2);
        __builtin_amdgcn_sched_barrier(0);
        compute(bb, t + 1);
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
    if (!arrive_last(&p.attn_counters[bk], p.nsplit, &s_last)) return;

    // ---- merge: the splits' partials plus the new token ----
    for (uint32_t h = wave; h < G; h += 4) {       // s_new = q . k_new (q is pre-scaled)
        const uint32_t qa = *reinterpret_cast<const uint32_t*>(
            p.q + (size_t)b * p.d + (kvh * G + h) * DH + 2 * lane);
        const uint32_t ka = *reinterpret_cast<const uint32_t*>(knew + 2 * lane);
        float d = __uint_as_float(qa << 16) * __uint_as_float(ka << 16) +
                  __uint_as_float(qa & 0xffff0000u) * __uint_as_float(ka & 0xffff0000u);
#pragma unroll
        for (int o2 = 32; o2 > 0; o2 >>= 1) d += __shfl_xor(d, o2);
        if (lane == 0) s_new[h] = d;
    }
    __syncthreads();
    constexpr uint32_t U = 8;                      // splits per batch of loads
    const uint32_t parts = bk * p.nsplit * G * APITCH * 4;
    for (uint32_t idx = tid; idx < G * (DH / 4); idx += 256) {
        const uint32_t h = idx / (DH / 4), d4 = idx % (DH / 4);
        float M = NEG_BIG, L = 0.f;
        f32x4 O = {};
        for (uint32_t c0 = 0; c0 < p.nsplit; c0 += U) {
            f32x4 oc[U];
            float mc[U], lc[U];
#pragma unroll
            for (uint32_t u = 0; u < U; ++u) {     // past the last split: reload it, weight 0
                const uint32_t c = min(c0 + u, p.nsplit - 1);
                const uint32_t at = parts + (c * G + h) * APITCH * 4;
                oc[u] = ld4_sc1(ars, at + 16 * d4);
                mc[u] = ld_sc1(ars, at + DH * 4);
                lc[u] = ld_sc1(ars, at + (DH + 1) * 4);
            }
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
        const uint2 vv = *reinterpret_cast<const uint2*>(vnew + 4 * d4);
        const f32x4 vn = {__uint_as_float(vv.x << 16), __uint_as_float(vv.x & 0xffff0000u),
                          __uint_as_float(vv.y << 16), __uint_as_float(vv.y & 0xffff0000u)};
        const f32x4 res = (O * so + wn * vn) / (L * so + wn);
        uint2 out;
        out.x = (uint32_t)f2bf(res[0]) | ((uint32_t)f2bf(res[1]) << 16);
        out.y = (uint32_t)f2bf(res[2]) | ((uint32_t)f2bf(res[3]) << 16);
        *reinterpret_cast<uint2*>(p.attn_out + (size_t)b * p.d + (kvh * G + h) * DH + 4 * d4) = out;
    }
    reset_counter(&p.attn_counters[bk]);
}

// ---- host side -----------------------------------------------------------------------------

struct Plan {
    uint32_t nqkv, g, nsplit, split_keys;
    uint32_t tiles[4], splits[4];
    size_t off_counters, off_partial, off_sumsq, off_q, off_attn_part, off_attn_out, off_x1,
        off_x1b, off_x1b_lo, off_sumsq2, off_act, off_act_lo, total;
    uint32_t counter_base[5];   // qkv, attn, wo, gu, down
};

// Steps per K split: 4 (128 KB of weights in flight per workgroup) when the
// K range divides, else 2 or 1.
static uint32_t choose_steps(uint32_t ksteps) {
    return ksteps % 4 == 0 ? 4u : (ksteps % 2 == 0 ? 2u : 1u);
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
    if ((uint64_t)a->n_heads * DH != a->d_model)
        return fail(MB_E_ARG, "decoder step: d_model %u != n_heads * head_dim", a->d_model);
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
    const uint32_t D = a->d_model, FF = a->d_ff, B = a->batch;
    pl->nqkv = D + 2 * a->n_kv_heads * DH;
    pl->g = a->n_heads / a->n_kv_heads;
    {   // attention: ~ATTN_WGS workgroups; splits of a multiple of 128 keys (an even
        // number of 64-key iterations, as the loop is unrolled by two)
        const uint32_t pairs = B * a->n_kv_heads;
        const uint32_t want = std::max(1u, cdiv(ATTN_WGS, pairs));
        const uint32_t nmax = std::max(1u, cdiv(a->cache_len, 2 * AKEYS));
        const uint32_t per = cdiv(std::max(a->cache_len, 1u), std::min(want, nmax));
        pl->split_keys = cdiv(per, 2 * AKEYS) * 2 * AKEYS;
        pl->nsplit = std::max(1u, cdiv(a->cache_len, pl->split_keys));
        if ((uint64_t)(pl->split_keys + 2 * AKEYS) * DH * 2 > 0xffffffffull)
            return fail(MB_E_ARG, "decoder step: cache_len %u too large", a->cache_len);
    }
    pl->tiles[EPI_QKV] = pl->nqkv / BN;
    pl->tiles[EPI_WO] = D / BN;
    pl->tiles[EPI_GU] = FF / 64;
    pl->tiles[EPI_DOWN] = D / BN;
    pl->splits[EPI_QKV] = (D / KS) / choose_steps(D / KS);
    pl->splits[EPI_WO] = (D / KS) / choose_steps(D / KS);
    pl->splits[EPI_GU] = (D / KS) / choose_steps(D / KS);
    pl->splits[EPI_DOWN] = (FF / KS) / choose_steps(FF / KS);
    size_t max_part = 0;
    for (int i = 0; i < 4; ++i)
        max_part = std::max(max_part, (size_t)pl->tiles[i] * pl->splits[i]);
    const uint32_t n_counters = pl->tiles[EPI_QKV] + B * a->n_kv_heads + pl->tiles[EPI_WO] +
                                pl->tiles[EPI_GU] + pl->tiles[EPI_DOWN];
    pl->counter_base[0] = 0;
    pl->counter_base[1] = pl->tiles[EPI_QKV];
    pl->counter_base[2] = pl->counter_base[1] + B * a->n_kv_heads;
    pl->counter_base[3] = pl->counter_base[2] + pl->tiles[EPI_WO];
    pl->counter_base[4] = pl->counter_base[3] + pl->tiles[EPI_GU];
    size_t o = 0;
    pl->off_counters = o; o = align256(o + (size_t)n_counters * 4);
    pl->off_partial = o; o = align256(o + max_part * MROWS * BN * 4);
    pl->off_sumsq = o; o = align256(o + (size_t)pl->tiles[EPI_QKV] * pl->splits[EPI_QKV] * MROWS * 4);
    pl->off_q = o; o = align256(o + (size_t)B * D * 2);
    pl->off_attn_part = o;
    o = align256(o + (size_t)B * a->n_kv_heads * pl->nsplit * pl->g * APITCH * 4);
    pl->off_attn_out = o; o = align256(o + (size_t)B * D * 2);
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

// Only the counters must start at zero; every other region is written before
// it is read within a step.
static size_t counters_bytes(const Plan& pl) { return pl.off_partial; }

template <int EPI>
void launch_skinny(const GemmCfg& g, const StepParams& p, hipStream_t s) {
    const dim3 grid(g.tiles * g.splits), block(256);
    switch (g.kc / KS) {
        case 1: hipLaunchKernelGGL((skinny_gemm_kernel<EPI, 1>), grid, block, 0, s, g, p); break;
        case 2: hipLaunchKernelGGL((skinny_gemm_kernel<EPI, 2>), grid, block, 0, s, g, p); break;
        default: hipLaunchKernelGGL((skinny_gemm_kernel<EPI, 4>), grid, block, 0, s, g, p); break;
    }
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
        ws = static_cast<uint8_t*>(library_workspace(pl.total, counters_bytes(pl), s));
        if (!ws) return MB_E_HIP;
    }

    StepParams p;
    p.batch = a->batch; p.d = a->d_model; p.hq = a->n_heads; p.hkv = a->n_kv_heads; p.g = pl.g;
    p.ff = a->d_ff; p.cache_len = a->cache_len; p.cache_stride = a->cache_stride;
    p.nsplit = pl.nsplit; p.split_keys = pl.split_keys; p.rope_base = a->rope_base; p.eps = a->eps;
    p.x = a->x; p.k_cache = a->k_cache; p.v_cache = a->v_cache;
    p.y = a->y; p.k_new = a->k_new; p.v_new = a->v_new;
    uint32_t* counters = reinterpret_cast<uint32_t*>(ws + pl.off_counters);
    p.attn_counters = counters + pl.counter_base[1];
    p.partial = reinterpret_cast<float*>(ws + pl.off_partial);
    p.partial_bytes = (uint32_t)(pl.off_sumsq - pl.off_partial);
    p.sumsq_bytes = (uint32_t)(pl.off_q - pl.off_sumsq);
    p.attn_part_bytes = (uint32_t)(pl.off_attn_out - pl.off_attn_part);
    p.sumsq = reinterpret_cast<float*>(ws + pl.off_sumsq);
    p.q = reinterpret_cast<uint16_t*>(ws + pl.off_q);
    p.attn_part = reinterpret_cast<float*>(ws + pl.off_attn_part);
    p.attn_out = reinterpret_cast<uint16_t*>(ws + pl.off_attn_out);
    p.x1 = reinterpret_cast<float*>(ws + pl.off_x1);
    p.x1b = reinterpret_cast<uint16_t*>(ws + pl.off_x1b);
    p.x1b_lo = reinterpret_cast<uint16_t*>(ws + pl.off_x1b_lo);
    p.sumsq2 = reinterpret_cast<float*>(ws + pl.off_sumsq2);
    p.act = reinterpret_cast<uint16_t*>(ws + pl.off_act);
    p.act_lo = reinterpret_cast<uint16_t*>(ws + pl.off_act_lo);

    const uint32_t D = a->d_model, FF = a->d_ff;
    auto gemm = [&](int epi, const uint16_t* act, const uint16_t* act_lo, uint32_t lda,
                    const uint16_t* w, uint32_t ldw, uint32_t k, uint32_t counter_base) -> GemmCfg {
        GemmCfg g;
        g.a = act; g.a_lo = act_lo; g.lda = lda; g.w = w; g.ldw = ldw; g.k = k;
        g.tiles = pl.tiles[epi]; g.splits = pl.splits[epi]; g.kc = k / g.splits;
        g.paired = epi == EPI_GU ? 1u : 0u;
        g.counters = counters + counter_base;
        return g;
    };
    const GemmCfg g_qkv =
        gemm(EPI_QKV, a->x, nullptr, D, a->w_qkv, pl.nqkv, D, pl.counter_base[0]);
    const GemmCfg g_wo =
        gemm(EPI_WO, p.attn_out, nullptr, D, a->w_o, D, D, pl.counter_base[2]);
    const GemmCfg g_gu =
        gemm(EPI_GU, p.x1b, p.x1b_lo, D, a->w_gu, 2 * FF, D, pl.counter_base[3]);
    const GemmCfg g_dn =
        gemm(EPI_DOWN, p.act, p.act_lo, FF, a->w_down, D, FF, pl.counter_base[4]);

    auto mark = [&](const char* name) { if (pm) pm->mark(s, name); };
    mark("qkv_rope");
    launch_skinny<EPI_QKV>(g_qkv, p, s);
    MB_LAUNCH_CHECK("decoder qkv_rope");
    mark("attention");
    {
        const dim3 grid(a->batch * a->n_kv_heads * pl.nsplit), block(256);
        if (pl.g <= 4) hipLaunchKernelGGL(attention_kernel<4>, grid, block, 0, s, p);
        else if (pl.g <= 8) hipLaunchKernelGGL(attention_kernel<8>, grid, block, 0, s, p);
        else hipLaunchKernelGGL(attention_kernel<16>, grid, block, 0, s, p);
    }
    MB_LAUNCH_CHECK("decoder attention");
    mark("wo_residual");
    launch_skinny<EPI_WO>(g_wo, p, s);
    MB_LAUNCH_CHECK("decoder wo_residual");
    mark("gate_up_swiglu");
    launch_skinny<EPI_GU>(g_gu, p, s);
    MB_LAUNCH_CHECK("decoder gate_up_swiglu");
    mark("down_residual");
    launch_skinny<EPI_DOWN>(g_dn, p, s);
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
        (rc = bs.buffer(2, MB_DTYPE_BF16, (uint64_t)D * D * 2, false, &ptr[2], "W_o")) ||
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

}  // namespace

void register_decoder() {
    register_kernel({"llama_decoder_step_bf16", run_decoder,
                     reinterpret_cast<const void*>(&skinny_gemm_kernel<EPI_GU, 4>), 5});
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
