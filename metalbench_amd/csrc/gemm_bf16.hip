// bf16 GEMM C[M][N] = bf16(A[M][K] @ B[K][N]), fp32 accumulation, on bf16 MFMA.
//
// No reference kernel: the reference has no bf16 (its dtype tables stop at
// f32/f16/i32/u32, reference mlx/scripts/mlx_helpers.py:83-89).  The spec is
// the reference's matmul (mlx/kernels/common/sqr_mm.py:10-11; registry
// helper mlx/kernels/common/registry.py:43-59: A@0, B@1, C@2, M@3, N@4, K@5)
// at bf16, rounded to bf16 (round to nearest even) once, from fp32.
//
// gfx950 design (MFMA bound: 2*M*N*K flops vs 2*(MK+KN+MN) bytes):
//  * workgroup tile 256x256, BK = 64, 4 waves in a 2x2 grid, each wave a
//    128x128 sub-tile = 4x4 v_mfma_f32_32x32x16_bf16 accumulators (256 fp32
//    per lane, held in AccVGPRs); one workgroup per CU, 1024 tiles at 8192^3 =
//    exactly four rounds of 256 CUs;
//  * (the guarded / element-wise kernel; the full-tile kernel further down
//    keeps the tile shape but swizzles A and stages loads two ahead)
//    LDS double buffer: both operands stored K-contiguous, row pitch 72 bf16
//    (144 B), 2 x 2 x 36 KB = 144 KB of the 160 KB.  With that pitch the MFMA
//    operand reads (ds_read_b128 of 16 consecutive rows) and both store
//    patterns below touch distinct bank groups;
//  * A is row-major [M][K], already K-contiguous: 16-byte global loads go
//    straight to LDS rows;
//  * B is row-major [K][N] (N-contiguous), but the MFMA B operand wants 8
//    consecutive k per lane: each lane loads an 8(k) x 8(n) block as eight
//    16-byte rows, transposes it in registers with 32 v_perm_b32 (pairing
//    k and k+1 halves into dwords) and stores eight K-contiguous 16-byte rows;
//  * global loads of stage s+1 are issued before the MFMAs of stage s, and
//    the LDS operand reads of k-step kk+1 are in flight during the MFMAs of kk;
//  * XCD-aware tile order: hardware dispatches block b to XCD b % 8, so the
//    block id is remapped so that each XCD walks one band of GM = 4 tile-rows
//    in column order; the 32 tiles one XCD runs at a time share 4 A panels and
//    8 B panels in that XCD's L2;
//  * shapes that are not tile multiples take guarded loads (zero fill) and
//    guarded stores; K % 8 or N % 8 != 0 fall back to element-wise loads.
#include "common.h"

namespace mb {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int PITCH = BK + 8;             // bf16 per LDS row (144 B)
constexpr int TILE_ELEMS = BM * PITCH;    // per operand per stage
constexpr int GM = 4;                     // tile-rows per XCD band

enum { MODE_FULL = 0, MODE_GUARD = 1, MODE_ELEM = 2 };

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);   // quiet NaN
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ void tile_coords(uint32_t b, uint32_t nblocks, uint32_t tiles_m,
                                            uint32_t tiles_n, uint32_t* tm, uint32_t* tn) {
    // Hardware block b runs on XCD b % 8: give each XCD a contiguous range of
    // logical tiles, then walk GM-row bands in column order.
    uint32_t L = b;
    if ((nblocks & 7) == 0) L = (b & 7) * (nblocks >> 3) + (b >> 3);
    const uint32_t per_group = GM * tiles_n;
    const uint32_t group = L / per_group;
    const uint32_t first_m = group * GM;
    const uint32_t gsize = min(tiles_m - first_m, (uint32_t)GM);
    const uint32_t in_group = L - group * per_group;
    *tm = first_m + in_group % gsize;
    *tn = in_group / gsize;
}

template <int MODE>
__global__ __launch_bounds__(256, 1)
void gemm_bf16_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                      uint16_t* __restrict__ C, uint32_t M, uint32_t N, uint32_t K,
                      uint32_t tiles_m, uint32_t tiles_n) {
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
    uint16_t* As = smem;                       // [2][BM][PITCH]
    uint16_t* Bs = smem + 2 * TILE_ELEMS;      // [2][BN][PITCH]

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63;
    const uint32_t wave = tid >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1;
    uint32_t tm, tn;
    tile_coords(blockIdx.x, gridDim.x, tiles_m, tiles_n, &tm, &tn);
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const uint32_t nstages = (K + BK - 1) / BK;

    // A loader: row = tid/8 + 32*i, 16-byte chunk = tid%8.
    // B loader: k-octet ko = tid%8, n-octet no = tid/8 (8 rows of 16 B each).
    const uint32_t a_row = tid >> 3, a_chunk = tid & 7;
    const uint32_t b_ko = tid & 7, b_no = tid >> 3;

    u32x4 ra[8], rb[8];

    auto load = [&](uint32_t k0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t gm = m0 + a_row + 32 * i, gk = k0 + 8 * a_chunk;
            const uint16_t* p = A + (size_t)gm * K + gk;
            if (MODE == MODE_FULL) {
                ra[i] = *reinterpret_cast<const u32x4*>(p);
            } else if (MODE == MODE_GUARD) {
                ra[i] = (gm < M && gk < K) ? *reinterpret_cast<const u32x4*>(p) : u32x4{};
            } else {
                uint16_t e[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) e[j] = (gm < M && gk + j < K) ? p[j] : (uint16_t)0;
                ra[i] = u32x4{e[0] | (uint32_t)e[1] << 16, e[2] | (uint32_t)e[3] << 16,
                              e[4] | (uint32_t)e[5] << 16, e[6] | (uint32_t)e[7] << 16};
            }
        }
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const uint32_t gk = k0 + 8 * b_ko + r, gn = n0 + 8 * b_no;
            const uint16_t* p = B + (size_t)gk * N + gn;
            if (MODE == MODE_FULL) {
                rb[r] = *reinterpret_cast<const u32x4*>(p);
            } else if (MODE == MODE_GUARD) {
                rb[r] = (gk < K && gn < N) ? *reinterpret_cast<const u32x4*>(p) : u32x4{};
            } else {
                uint16_t e[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) e[j] = (gk < K && gn + j < N) ? p[j] : (uint16_t)0;
                rb[r] = u32x4{e[0] | (uint32_t)e[1] << 16, e[2] | (uint32_t)e[3] << 16,
                              e[4] | (uint32_t)e[5] << 16, e[6] | (uint32_t)e[7] << 16};
            }
        }
    };

    auto store = [&](int buf) {
        uint16_t* as = As + buf * TILE_ELEMS;
        uint16_t* bs = Bs + buf * TILE_ELEMS;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            *reinterpret_cast<u32x4*>(as + (a_row + 32 * i) * PITCH + 8 * a_chunk) = ra[i];
        // 8x8 transpose: column c of the block = n0 + 8*no + c gets k = 8*ko .. +7.
        // Dword j of column c pairs (k = 2j, 2j+1): lo halves for even c, hi for odd.
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            uint32_t lo[4], hi[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t e = rb[2 * j][m];
                const uint32_t o = rb[2 * j + 1][m];
                lo[j] = __builtin_amdgcn_perm(o, e, 0x05040100u);
                hi[j] = __builtin_amdgcn_perm(o, e, 0x07060302u);
            }
            *reinterpret_cast<u32x4*>(bs + (8 * b_no + 2 * m) * PITCH + 8 * b_ko) =
                u32x4{lo[0], lo[1], lo[2], lo[3]};
            *reinterpret_cast<u32x4*>(bs + (8 * b_no + 2 * m + 1) * PITCH + 8 * b_ko) =
                u32x4{hi[0], hi[1], hi[2], hi[3]};
        }
    };

    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

    const uint32_t li = lane & 31, lh = lane >> 5;

    if (nstages > 0) {
        load(0);
        store(0);
        __syncthreads();
    }
    for (uint32_t s = 0; s < nstages; ++s) {
        const int cur = s & 1;
        if (s + 1 < nstages) load((s + 1) * BK);
        const uint16_t* as = As + cur * TILE_ELEMS + (wm * 128 + li) * PITCH + 8 * lh;
        const uint16_t* bs = Bs + cur * TILE_ELEMS + (wn * 128 + li) * PITCH + 8 * lh;
        // Operands of k-step kk+1 are read from LDS while the 16 MFMAs of kk run.
        bf16x8 a[2][4], b[2][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[0][i] = *reinterpret_cast<const bf16x8*>(as + 32 * i * PITCH);
#pragma unroll
        for (int j = 0; j < 4; ++j) b[0][j] = *reinterpret_cast<const bf16x8*>(bs + 32 * j * PITCH);
#pragma unroll
        for (int kk = 0; kk < BK / 16; ++kk) {
            const int c = kk & 1;
            if (kk + 1 < BK / 16) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    a[c ^ 1][i] = *reinterpret_cast<const bf16x8*>(as + 32 * i * PITCH + 16 * (kk + 1));
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    b[c ^ 1][j] = *reinterpret_cast<const bf16x8*>(bs + 32 * j * PITCH + 16 * (kk + 1));
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[c][i], b[c][j], acc[i][j],
                                                                         0, 0, 0);
        }
        if (s + 1 < nstages) store(cur ^ 1);
        __syncthreads();
    }

    // Epilogue: lane l, reg r of a 32x32 block -> row 8*(r/4) + 4*(l/32) + r%4, col l%32.
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t gc = n0 + wn * 128 + 32 * j + li;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t gr = m0 + wm * 128 + 32 * i + 8 * (r >> 2) + 4 * lh + (r & 3);
                if (MODE == MODE_FULL || (gr < M && gc < N))
                    C[(size_t)gr * N + gc] = f32_to_bf16_rne(acc[i][j][r]);
            }
        }
}

// ---- full-tile kernel (M, N multiples of 256, K of 128, operands < 2 GiB) ----
// Both operands are register-staged TWO LDS stages ahead: the global loads
// for stage s+2 are issued during the MFMAs of stage s, so a load has about
// 2 x 64 MFMAs per wave (~4 us at the power-limited clock) to arrive.
//  * A rows are stored unpadded (128 B = 8 chunks of 8 k) with chunk c of row
//    r in slot c ^ ((r / 2) % 8): a ds_read_b128 serves 16 lanes = 16
//    consecutive rows per LDS cycle, and their 16-byte bank groups
//    8 (r % 2) + slot are then all distinct (conflict free);
//  * B (N-contiguous in HBM) is loaded as 8 x 16-byte rows per lane,
//    transposed in registers with v_perm_b32 and stored K-contiguous into
//    the pitch-72 layout;
//  * stage s: loads of stage s+2 -> register set s % 2 (A in k steps 0-1, B
//    in k steps 2-3, 4 loads per 16 MFMAs), MFMAs on LDS buffers s % 2, and
//    in k step 3 the stores of register set (s+1) % 2 into buffers
//    (s+1) % 2; then an LDS-only barrier (lgkmcnt + s_barrier, the global
//    loads stay in flight).  sched_group_barrier interleaves one MFMA with
//    each group of loads / operand reads / transposes / stores, so the MFMA
//    pipe never waits on issue.
// Buffer-to-LDS DMA for A (no registers, no LDS store instructions) was
// measured slower than this on MI355X (49% vs 50.6% of peak at 8192^3).
constexpr int ROWB = BK * 2;              // bytes per unpadded A row in LDS

__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__global__ __launch_bounds__(256, 1)
void gemm_bf16_full_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                           uint16_t* __restrict__ C, uint32_t M, uint32_t N, uint32_t K,
                           uint32_t tiles_m, uint32_t tiles_n) {
    __shared__ __attribute__((aligned(1024))) uint16_t As0[BM * BK];
    __shared__ __attribute__((aligned(1024))) uint16_t As1[BM * BK];
    __shared__ __attribute__((aligned(16))) uint16_t Bs0[TILE_ELEMS];
    __shared__ __attribute__((aligned(16))) uint16_t Bs1[TILE_ELEMS];

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: DMA bases
    const uint32_t wm = wave >> 1, wn = wave & 1;
    uint32_t tm, tn;
    tile_coords(blockIdx.x, gridDim.x, tiles_m, tiles_n, &tm, &tn);
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(tm * BM);
    const uint32_t n0 = __builtin_amdgcn_readfirstlane(tn * BN);
    const uint32_t nstages = K / BK;
    const uint32_t last_k0 = (nstages - 1) * BK;

    const __amdgpu_buffer_rsrc_t ars =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(A), 0, M * K * 2, 0x00020000u);
    const __amdgpu_buffer_rsrc_t brs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(B), 0, K * N * 2, 0x00020000u);

    // A: lane loads rows a_row + 32 i (i < 8), 16-byte chunk a_chunk, and
    // stores them into the swizzled layout (slot = chunk ^ ((row / 2) % 8)).
    const uint32_t a_row = tid >> 3, a_chunk = tid & 7;
    const uint32_t a_voff = (a_row * K + 8 * a_chunk) * 2;
    u32x4 ra[2][8];
    auto load_a = [&](int st, uint32_t k0, int i0, int i1) {
#pragma unroll
        for (int i = i0; i < i1; ++i)
            ra[st][i] = __builtin_amdgcn_raw_buffer_load_b128(ars, a_voff, ((m0 + 32 * i) * K + k0) * 2, 0);
    };
    auto store_a = [&](int st, uint16_t* as_dst) {
        uint8_t* as = reinterpret_cast<uint8_t*>(as_dst);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t row = a_row + 32 * i;
            *reinterpret_cast<u32x4*>(as + row * ROWB + 16 * (a_chunk ^ ((row >> 1) & 7))) = ra[st][i];
        }
    };
    // B: k-octet ko = tid%8, n-octet no = tid/8 (8 rows of 16 B each).
    const uint32_t b_ko = tid & 7, b_no = tid >> 3;
    const uint32_t b_voff = (8 * b_ko * N + 8 * b_no) * 2;
    u32x4 rb[2][8];
    auto load_b = [&](int st, uint32_t k0, int r0, int r1) {   // rows [r0, r1)
#pragma unroll
        for (int r = r0; r < r1; ++r)
            rb[st][r] = __builtin_amdgcn_raw_buffer_load_b128(brs, b_voff, ((k0 + r) * N + n0) * 2, 0);
    };
    auto store_b = [&](int st, uint16_t* bs) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            uint32_t lo[4], hi[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                lo[j] = __builtin_amdgcn_perm(rb[st][2 * j + 1][m], rb[st][2 * j][m], 0x05040100u);
                hi[j] = __builtin_amdgcn_perm(rb[st][2 * j + 1][m], rb[st][2 * j][m], 0x07060302u);
            }
            *reinterpret_cast<u32x4*>(bs + (8 * b_no + 2 * m) * PITCH + 8 * b_ko) =
                u32x4{lo[0], lo[1], lo[2], lo[3]};
            *reinterpret_cast<u32x4*>(bs + (8 * b_no + 2 * m + 1) * PITCH + 8 * b_ko) =
                u32x4{hi[0], hi[1], hi[2], hi[3]};
        }
    };

    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

    const uint32_t li = lane & 31, lh = lane >> 5;
    // One LDS stage of MFMAs.  The next stages' global loads are spread over
    // the four k steps (`pre(kk)` issues a quarter: 4 loads per 16 MFMAs, so
    // the texture unit never backs up into the wave's in-order issue), and
    // `post` (the B transpose + LDS stores of the next stage) runs inside k
    // step 3; one instruction group per MFMA, so nothing but the initial
    // operand reads sits outside the MFMA shadow.
    auto mfma_stage = [&](const uint16_t* as_base, const uint16_t* bs_base, auto&& pre,
                          auto&& post) {
        const uint8_t* as = reinterpret_cast<const uint8_t*>(as_base) + (wm * 128 + li) * ROWB;
        const uint16_t* bs = bs_base + (wn * 128 + li) * PITCH + 8 * lh;
        auto a_at = [&](int i, int kk) {   // rows wm*128 + 32 i + li, k chunk 2 kk + lh, swizzled
            return *reinterpret_cast<const bf16x8*>(as + 32 * i * ROWB +
                                                    16 * ((2 * kk + lh) ^ ((li >> 1) & 7)));
        };
        bf16x8 a[2][4], b[2][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[0][i] = a_at(i, 0);
#pragma unroll
        for (int j = 0; j < 4; ++j) b[0][j] = *reinterpret_cast<const bf16x8*>(bs + 32 * j * PITCH);
#pragma unroll
        for (int kk = 0; kk < BK / 16; ++kk) {
            const int c = kk & 1;
            __builtin_amdgcn_sched_barrier(0);
            pre(kk);
            if (kk + 1 < BK / 16) {
#pragma unroll
                for (int i = 0; i < 4; ++i) a[c ^ 1][i] = a_at(i, kk + 1);
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    b[c ^ 1][j] = *reinterpret_cast<const bf16x8*>(bs + 32 * j * PITCH + 16 * (kk + 1));
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[c][i], b[c][j], acc[i][j],
                                                                         0, 0, 0);
            if (kk == BK / 16 - 1) post();
            if (kk + 1 < BK / 16) {   // 16 MFMA, 8 operand reads, 4 global loads
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
                    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // VMEM read
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
                    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);   // 2 MFMA
                }
            } else {                  // 16 MFMA, 4 global loads, 32 v_perm + 16 LDS stores
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // VMEM read
                    __builtin_amdgcn_sched_group_barrier(0x200, 2, 0);   // DS write
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);   // VALU
                    __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);   // DS write
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);   // VALU
                    __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);   // DS write
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    load_a(0, 0, 0, 8);
    load_b(0, 0, 0, 8);
    __builtin_amdgcn_s_waitcnt(0);
    store_a(0, As0);
    store_b(0, Bs0);
    __syncthreads();
    load_a(1, min((uint32_t)BK, last_k0), 0, 8);
    load_b(1, min((uint32_t)BK, last_k0), 0, 8);
    // Stage s: MFMAs on buffers s % 2; register set s % 2 receives stage s+2
    // (A in k steps 0-1, B in 2-3); set (s+1) % 2, loaded one stage earlier,
    // is stored to the other buffers inside k step 3.  nstages is even
    // (K % 128 == 0), so the body is straight-line: past the last stage the
    // clamped loads re-read it and land in buffers never read again.
    for (uint32_t s = 0; s < nstages; s += 2) {
        const uint32_t k2 = min((s + 2) * BK, last_k0), k3 = min((s + 3) * BK, last_k0);
        mfma_stage(As0, Bs0,
                   [&](int kk) {
                       if (kk < 2) load_a(0, k2, 4 * kk, 4 * kk + 4);
                       else load_b(0, k2, 4 * (kk - 2), 4 * (kk - 2) + 4);
                   },
                   [&] { store_a(1, As1); store_b(1, Bs1); });
        lds_barrier();
        mfma_stage(As1, Bs1,
                   [&](int kk) {
                       if (kk < 2) load_a(1, k3, 4 * kk, 4 * kk + 4);
                       else load_b(1, k3, 4 * (kk - 2), 4 * (kk - 2) + 4);
                   },
                   [&] { store_a(0, As0); store_b(0, Bs0); });
        lds_barrier();
    }


    // Epilogue through LDS: each wave converts its 128 x 128 tile to bf16
    // (hardware round-to-nearest-even convert), writes it row-major into its
    // own 32 KB of the now idle operand buffers, and streams it out as 16-byte
    // row chunks (a wave store instruction covers four 256-byte row segments).
    // Lane l, reg r of 32x32 block (i, j): row 32 i + 8 (r/4) + 4 (l/32) + r%4,
    // column 32 j + l%32.
    lds_barrier();   // every wave is done reading the operand buffers
    uint16_t* ct = wave == 0 ? As0 : wave == 1 ? As1 : wave == 2 ? Bs0 : Bs1;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t row = 32 * i + 8 * (r >> 2) + 4 * lh + (r & 3);
                ct[row * 128 + 32 * j + li] = __builtin_bit_cast(uint16_t, (__bf16)acc[i][j][r]);
            }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
#pragma unroll
    for (int q = 0; q < 32; ++q) {
        const uint32_t row = 4 * q + (lane >> 4), ch = lane & 15;
        const u32x4 v = *reinterpret_cast<const u32x4*>(ct + row * 128 + 8 * ch);
        *reinterpret_cast<u32x4*>(C + (size_t)(m0 + wm * 128 + row) * N + n0 + wn * 128 + 8 * ch) = v;
    }
}

constexpr size_t SMEM_BYTES = 4 * TILE_ELEMS * sizeof(uint16_t);   // 147456

int launch_gemm_bf16(const uint16_t* a, const uint16_t* b, uint16_t* c, uint32_t m, uint32_t n,
                     uint32_t k, hipStream_t s) {
    if (m == 0 || n == 0) return MB_OK;
    if (!a || !b || !c) return fail(MB_E_ARG, "matmul_bf16: null pointer");
    const uint32_t tiles_m = cdiv(m, BM), tiles_n = cdiv(n, BN);
    const uint64_t nblocks = (uint64_t)tiles_m * tiles_n;
    if (nblocks > 0x7fffffffull) return fail(MB_E_ARG, "matmul_bf16: shape too large");
    const bool aligned = (k % 8 == 0) && (n % 8 == 0) &&
                         ((((uintptr_t)a) | ((uintptr_t)b)) & 15) == 0;
    const bool full = aligned && m % BM == 0 && n % BN == 0 && k % (2 * BK) == 0 && k > 0 &&
                      (uint64_t)m * k * 2 < (1ull << 31) && (uint64_t)k * n * 2 < (1ull << 31);
    static bool attr_set[3] = {false, false, false};
    auto go = [&](auto kernel, int mode) -> int {
        if (!attr_set[mode]) {
            MB_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)SMEM_BYTES));
            attr_set[mode] = true;
        }
        hipLaunchKernelGGL(kernel, dim3((uint32_t)nblocks), dim3(256), SMEM_BYTES, s, a, b, c, m,
                           n, k, tiles_m, tiles_n);
        MB_LAUNCH_CHECK("matmul_bf16");
        return MB_OK;
    };
    if (full) {
        hipLaunchKernelGGL(gemm_bf16_full_kernel, dim3((uint32_t)nblocks), dim3(256), 0, s, a, b, c,
                           m, n, k, tiles_m, tiles_n);
        MB_LAUNCH_CHECK("matmul_bf16");
        return MB_OK;
    }
    if (aligned) return go(gemm_bf16_kernel<MODE_GUARD>, MODE_GUARD);
    return go(gemm_bf16_kernel<MODE_ELEM>, MODE_ELEM);
}

// Registry launcher: A@0, B@1 (bf16 inputs), C@2 (bf16 output), M@3, N@4, K@5.
int run_gemm_bf16(const Bindings& bs, hipStream_t s, PartMarks*) {
    uint32_t m, n, k;
    int rc;
    if ((rc = bs.u32(3, &m, "M")) || (rc = bs.u32(4, &n, "N")) || (rc = bs.u32(5, &k, "K")))
        return rc;
    void *a, *b, *c;
    if ((rc = bs.buffer(0, MB_DTYPE_BF16, (uint64_t)m * k * 2, false, &a, "A")) ||
        (rc = bs.buffer(1, MB_DTYPE_BF16, (uint64_t)k * n * 2, false, &b, "B")) ||
        (rc = bs.buffer(2, MB_DTYPE_BF16, (uint64_t)m * n * 2, true, &c, "C")))
        return rc;
    return launch_gemm_bf16((const uint16_t*)a, (const uint16_t*)b, (uint16_t*)c, m, n, k, s);
}

}  // namespace

void register_gemm_bf16() {
    register_kernel({"large_matmul_bf16", run_gemm_bf16,
                     reinterpret_cast<const void*>(&gemm_bf16_full_kernel), 1});
}

}  // namespace mb

extern "C" int mb_launch_matmul_bf16(const uint16_t* a, const uint16_t* b, uint16_t* c, uint32_t m,
                                     uint32_t n, uint32_t k, void* stream) {
    mb::clear_error();
    if (!mb::initialized()) return mb::fail(MB_E_STATE, "mb_init() has not been called");
    return mb::launch_gemm_bf16(a, b, c, m, n, k, mb::stream_or_default(stream));
}
