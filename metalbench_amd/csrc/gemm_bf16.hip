// bf16 GEMM C[M][N] = bf16(A[M][K] @ B[K][N]), fp32 accumulation, on bf16 MFMA.
//
// No reference kernel: the reference has no bf16 (its dtype tables stop at
// f32/f16/i32/u32, reference mlx/scripts/mlx_helpers.py:83-89).  The spec is
// the reference's matmul (mlx/kernels/common/sqr_mm.py:10-11; registry
// helper mlx/kernels/common/registry.py:43-59: A@0, B@1, C@2, M@3, N@4, K@5)
// at bf16, rounded to bf16 (round to nearest even) once, from fp32.
//
// gfx950 design (MFMA bound: 2*M*N*K flops vs 2*(MK+KN+MN) bytes):
//  * workgroup tile 256x256, 4 waves in a 2x2 grid, each wave a 128x128
//    sub-tile (256 fp32 accumulators per lane, held in AccVGPRs); one
//    workgroup per CU, 1024 tiles at 8192^3 = exactly four rounds of 256 CUs;
//  * full tiles (the large_mm shape) take gemm_bf16_full_kernel further down:
//    8 x 8 v_mfma_f32_16x16x32_bf16 per wave and 32-deep k stage, both
//    operands global -> LDS by DMA (no staging registers, no LDS store
//    instructions) into rings that fill all 160 KB of LDS (A in 64-deep
//    slots of whole 128-byte lines, B in 32-deep slots), B transposed by the
//    LDS reads (ds_read_b64_tr_b16);
//  * other shapes take gemm_bf16_kernel (4 x 4 v_mfma_f32_32x32x16_bf16 per
//    wave), BK = 64 with an LDS double buffer:
//    both operands stored K-contiguous, row pitch 72 bf16 (144 B), 2 x 2 x
//    36 KB = 144 KB of the 160 KB.  With that pitch the MFMA operand reads
//    (ds_read_b128 of 16 consecutive rows) and both store patterns below
//    touch distinct bank groups.  A is row-major [M][K], already
//    K-contiguous: 16-byte global loads go straight to LDS rows.  B is
//    row-major [K][N] (N-contiguous), but the MFMA B operand wants 8
//    consecutive k per lane: each lane loads an 8(k) x 8(n) block as eight
//    16-byte rows, transposes it in registers with 32 v_perm_b32 (pairing k
//    and k+1 halves into dwords) and stores eight K-contiguous 16-byte rows.
//    Global loads of stage s+1 are issued before the MFMAs of stage s, and
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
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
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
    xcd_band_tile(b, nblocks, tiles_m, tiles_n, GM, tm, tn);
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
// Both operands go global -> LDS by DMA (buffer_load ... lds): no staging
// registers and no LDS store instructions, whose VGPR reads stall the MFMA
// issue.  All 160 KB of LDS hold the operand rings:
//  * A in three 64-deep slots (32 KB each: 256 rows of 128 bytes).  Each A
//    DMA instruction fills 8 whole 128-byte lines (8 rows x 8 chunks); chunk c
//    (8 k) of row r sits in slot c ^ ((r / 2) % 8).  The 16x16x32 A operand of
//    row block i is one ds_read_b128: lane l reads row 16 i + l%16, chunk
//    4 h + l/16 (h = which 32-k half of the slot); each 16 lanes hit 16
//    distinct 16-byte bank groups;
//  * B in four 32-deep slots (16 KB each: [32 k][256 n] row-major as in HBM,
//    512-byte k-rows); chunk c (8 n) of k-row r sits in slot c ^ f(r),
//    f(r) = 4 (r % 4) ^ 2 ((r / 8) % 2).  The B operand (8 consecutive k of one
//    column) is two ds_read_b64_tr_b16: in 16-lane group g lane s points at
//    k-row 8 g + 4 q + s/4, columns n0 + 4 (s % 4) .. +3, and receives column
//    n0 + s, those 4 k-rows.  The ^ 2 ((r/8) % 2) term puts k-rows r and r + 8
//    (groups 0 and 1, read in the same LDS cycle) in different banks;
//  * each DMA instruction writes a wave's 64 x 16 B contiguously, so lane l
//    fetches the global chunk that its slot holds.
// The MFMA is v_mfma_f32_16x16x32_bf16, not 32x32x16: on random bf16 data
// the chip is power-limited, and a register-only loop of 16x16x32 sustains
// 1.90-2.12 PF against 1.50-1.85 PF for 32x32x16 at the same power.
//
// Stage s (32 k; B slot s % 4, operands in register set s % 2): wait for this
// wave's DMAs issued three stages earlier and pass one LDS barrier (every
// wave finished reading the slots refilled below, and stage s+1 has landed);
// then the wave's 8 x 8 blocks (64 MFMAs) run with one DMA instruction per
// row of 8 MFMAs (B stage s+4 into slot s % 4 on even rows, a quarter of A
// pair (s+1)/2 + 2 on odd rows) and the 24 reads of stage s+1's operands
// spread under them.  Measured on random operands, power-limited (1400 W),
// same box, 8192^3: 32-deep A and B slots with both DMAs every other row
// 762-772 us; one DMA per row 758-763 us (on zero operands, not
// power-limited, 585 -> 521 us: two DMAs at once stall the MFMA issue); A
// in 128-byte lines as here 735-742 us.  Per 32-k stage the loop takes ~1256
// cycles for 1024 cycles of MFMA work: ~62 at the barrier, ~8 waiting for
// DMAs, the rest issue gaps, ~16 cycles per DMA instruction.  A 64-byte A
// row (the 32-deep A slot) makes each DMA instruction touch 16 half lines
// instead of 8 whole ones; in cycles both run alike, but the whole-line
// version spends less energy per GEMM, so at the power limit it keeps a
// higher clock.
constexpr int KS = 32;                    // k per B slot and per barrier
constexpr int BROWB = BN * 2;             // bytes per B k-row in LDS
constexpr int A_SLOT_BYTES = BM * 128;    // one A slot: 64 k
constexpr int B_SLOT_BYTES = KS * BROWB;  // one B slot: 32 k

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4_t;
typedef float f32x4 __attribute__((ext_vector_type(4)));
template <int V> struct TailC { static constexpr int v = V; };

// dma16 with the LDS address given as a base plus an offset (both SGPRs;
// the offsets are loop-invariant), added straight into M0: one scalar
// instruction per DMA.
__device__ __forceinline__ void dma16_at(i32x4 rsrc, uint32_t lds_base, uint32_t lds_off,
                                         uint32_t voff, uint32_t soff) {
    asm volatile("s_add_u32 m0, %0, %1\n\tbuffer_load_dwordx4 %2, %3, %4 offen lds"
                 :: "s"(lds_base), "s"(lds_off), "v"(voff), "s"(rsrc), "s"(soff) : "m0", "scc");
}

__global__ __launch_bounds__(256, 1)
void gemm_bf16_full_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                           uint16_t* __restrict__ C, uint32_t M, uint32_t N, uint32_t K,
                           uint32_t tiles_m, uint32_t tiles_n) {
    __shared__ __attribute__((aligned(1024))) uint8_t AL[3 * A_SLOT_BYTES];
    __shared__ __attribute__((aligned(1024))) uint8_t BL[4 * B_SLOT_BYTES];

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: DMA bases
    const uint32_t wm = wave >> 1, wn = wave & 1;
    uint32_t tm, tn;
    tile_coords(blockIdx.x, gridDim.x, tiles_m, tiles_n, &tm, &tn);
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(tm * BM);
    const uint32_t n0 = __builtin_amdgcn_readfirstlane(tn * BN);
    const uint32_t nstages = K / KS;   // a multiple of 4
    const uint32_t npairs = nstages / 2;

    const i32x4 ars = dma_rsrc(A, M * K * 2), brs = dma_rsrc(B, K * N * 2);
    const uint32_t al = lds_addr(AL), bl = lds_addr(BL);

    // A DMA instruction i (0..7) of wave w for pair q (k 64 q .. 64 q + 63):
    // rows 64 w + 8 i + l/8, slot l%8, which holds chunk
    // (l%8) ^ ((row/2) % 8) = (l%8) ^ ((4 i + l/16) % 8).
    uint32_t a_voff[2];
#pragma unroll
    for (int p = 0; p < 2; ++p)
        a_voff[p] = ((lane >> 3) * K + 8 * ((lane & 7) ^ ((4 * p + (lane >> 4)) & 7))) * 2;
    const uint32_t a_dst = 64 * wave * 128;
    const uint32_t a_src = (m0 + 64 * wave) * K * 2;
    // B DMA instruction i (0..3) of wave w: k-rows r = 8 w + 2 i + l/32, slot
    // l%32, which holds chunk (l%32) ^ f(r).
    const uint32_t b_r = lane >> 5;
    const uint32_t bx = 2 * (wave & 1);
    const uint32_t b_voff0 = (b_r * N + 8 * ((lane & 31) ^ (4 * b_r) ^ bx)) * 2;
    const uint32_t b_voff1 = (b_r * N + 8 * ((lane & 31) ^ (4 * (2 + b_r)) ^ bx)) * 2;
    const uint32_t b_dst = 8 * wave * BROWB;
    const uint32_t b_src = (8 * wave * N + n0) * 2;
    // DMA instruction i of a stage: lds = the slot's LDS address for this
    // wave, glb = the operand's byte offset for this wave and stage.  What
    // depends on i is a per-lane voffset (one VGPR per instruction) and a
    // loop-invariant LDS offset added into M0, so a DMA costs one scalar
    // instruction besides the load.
    uint32_t a_vo[8], b_vo[4];
#pragma unroll
    for (int i = 0; i < 8; ++i) a_vo[i] = a_voff[i & 1] + 8 * i * K * 2;
#pragma unroll
    for (int i = 0; i < 4; ++i) b_vo[i] = ((i & 1) ? b_voff1 : b_voff0) + 2 * i * N * 2;
    const uint32_t bl_w = bl + b_dst;
    const uint32_t al_w = al + a_dst;
    auto dma_a = [&](uint32_t lds, uint32_t glb, int i) {
        dma16_at(ars, lds, 8 * i * 128, a_vo[i], glb);
    };
    auto dma_b = [&](int slot, uint32_t glb, int i) {
        dma16_at(brs, bl_w, slot * B_SLOT_BYTES + 2 * i * BROWB, b_vo[i], glb);
    };

    f32x4 acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{};

    // 16x16x32 operands.  A (i): lane l holds row wm*128 + 16 i + l%16,
    // k octet l/16 of the stage's 32-k half h.
    const uint32_t g = lane >> 4, t = lane & 15;
    const uint32_t a_row = (wm * 128 + t) * 128;
    const uint32_t a_half[2] = {16 * ((0 + g) ^ ((t >> 1) & 7)), 16 * ((4 + g) ^ ((t >> 1) & 7))};
    const uint32_t a_rh[2] = {a_row + a_half[0], a_row + a_half[1]};
    // B (j): lane l needs column wn*128 + 16 j + l%16, k = 8 (l/16) .. +7:
    // two ds_read_b64_tr_b16 (k-rows 8g + 4q + t/4, columns 4 (t%4) .. +3 of
    // the 16-column block), each returning 4 k of column t.
    uint32_t b_off[8][2];
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const uint32_t r = 8 * g + 4 * q + (t >> 2);
            const uint32_t c = wn * 128 + 16 * j + 4 * (t & 3);
            const uint32_t f = 4 * (r & 3) ^ 2 * ((r >> 3) & 1);
            b_off[j][q] = r * BROWB + 16 * ((c >> 3) ^ f) + 2 * (c & 7);
        }
    auto b_at = [&](const uint8_t* bs, int j) {
        u32x2 h[2];
#pragma unroll
        for (int q = 0; q < 2; ++q)
            h[q] = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_s16x4_t*)(bs + b_off[j][q])));
        return __builtin_bit_cast(bf16x8, u32x4{h[0][0], h[0][1], h[1][0], h[1][1]});
    };
    auto a_at = [&](const uint8_t* as, int i) {
        return *reinterpret_cast<const bf16x8*>(as + 16 * i * 128);
    };
    bf16x8 a[2][8], b[2][8];
    // The MFMAs are inline asm with the accumulators pinned to AccVGPRs
    // ("+a"): with 64 four-register accumulators the register allocator
    // otherwise shuttles them between AccVGPRs and VGPRs every iteration.
    // The wait-count pass sees the asm operands (it waits for the operand
    // reads); the one hazard it cannot see -- reading an accumulator right
    // after the MFMA that writes it -- is padded before the epilogue.
    // Consecutive MFMAs share an operand register (snake order over j).
    // The B fragment goes in the MFMA's first operand and the A fragment in
    // its second, so the MFMA computes the 16x16 block transposed: lane l,
    // register r of acc[i][j] is C row 16 i + l%16, column 16 j + 4 (l/16) + r
    // (four consecutive columns of one row, which the epilogue packs into
    // one 8-byte LDS write).  The products and their k order are the same.
    auto mfma = [&](int c, int i, int jj) {
        const int j = (i & 1) ? 7 - jj : jj;
        asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0"
                     : "+a"(acc[i][j]) : "v"(b[c][j]), "v"(a[c][i]));
    };
    // Stage s at unrolled position u = s % 4.  A pair q occupies slot q % 3
    // and is fetched a quarter per stage over stages 2q - 5 and 2q - 4, i.e.
    // three stages before its first read; its slot held pair q - 3, whose
    // last operands were read during stage 2q - 6.
    // TAIL: 0 = steady state; 1..4 = the last four stages (no DMAs: every
    // operand is already requested), waiting for vmcnt 16 / 8 / 0 and, in the
    // last stage, nothing (its operands were read in stage n-2).
    // Stage s = 4 t + u.  Its scalar operands come from the loop, which
    // carries them from iteration to iteration instead of recomputing them
    // (a pair's slot is pair % 3).  With the divisions, the clamps and the
    // per-DMA address arithmetic the loop issued ~34 scalar and ~3 vector
    // ALU instructions per stage; now ~15 (8 of them the M0 adds) and 1,
    // and the 8192^3 GEMM runs ~4 % faster (715-723 -> 699-700 us,
    // alternated on one box, with the move of the operands ahead of the
    // barrier described below):
    //   rd_slot  slot byte offset of the pair holding stage s+1 (read side);
    //   dma_slot slot byte offset of the pair being fetched;
    //   a_glb, b_glb  this wave's byte offsets of the A pair and B stage being fetched.
    // They are formed before the barrier, under the previous stage's last
    // MFMAs (the empty asm statements keep them there), so that after the
    // barrier the stage's first MFMA follows at once.
    auto stage = [&](int u, uint32_t rd_slot, uint32_t dma_slot, uint32_t a_glb, uint32_t b_glb,
                     auto TL) {
        constexpr int TAIL = decltype(TL)::v;
        const int c = u & 1;
        const int ih = 4 * ((u + 1) & 1);          // its instructions 0-3 (s odd) or 4-7
        uint32_t a_lds = al_w + dma_slot;
        uint32_t nas_off = rd_slot + a_rh[(u + 1) & 1];
        if (TAIL == 0) asm volatile("" : "+s"(a_lds), "+s"(a_glb), "+s"(b_glb));
        if (TAIL != 4) asm volatile("" : "+v"(nas_off));
        __builtin_amdgcn_sched_barrier(0);
        if (TAIL <= 1) __builtin_amdgcn_s_waitcnt(0x4F70);   // vmcnt(16): stages s-1, s-2 may be in flight
        else if (TAIL == 2) __builtin_amdgcn_s_waitcnt(0x0F78);   // vmcnt(8)
        else if (TAIL == 3) __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
        if (TAIL != 4) lds_barrier();
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t* nas = AL + nas_off;
        const uint8_t* nbs = BL + ((u + 1) & 3) * B_SLOT_BYTES;
        // unit v < 8: B v (two transposing reads); v >= 8: A v-8 (one read),
        // in the order stage s+1 consumes them (its first row needs every B)
        auto rd = [&](int v) {
            if (v < 8) b[c ^ 1][v] = b_at(nbs, v);
            else a[c ^ 1][v - 8] = a_at(nas, v - 8);
        };
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            mfma(c, r, 0);
            if (TAIL == 0) {
                if (r & 1) dma_a(a_lds, a_glb, ih + (r >> 1));
                else dma_b(u, b_glb, r >> 1);
            }
            mfma(c, r, 1);
            if (TAIL != 4) rd(2 * r);
            mfma(c, r, 2);
            mfma(c, r, 3);
            mfma(c, r, 4);
            if (TAIL != 4) rd(2 * r + 1);
            mfma(c, r, 5);
            mfma(c, r, 6);
            mfma(c, r, 7);
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    // Prologue: A pairs 0-2 and B stages 0-3, in the order A0 B0 B1 A1 B2 B3
    // A2 (40 DMA instructions per wave).  Stage 0's barrier then waits for
    // the first 24 (A0 B0 B1 A1) and stage 0 reloads the second half of A2.
    // The last four stages are peeled: every byte they need is requested
    // by then, so they issue no DMAs and the epilogue waits for none
    // (waiting for clamped reloads there had cost 571 against 550 us on zero
    // operands).
#pragma unroll
    for (int i = 0; i < 8; ++i) dma_a(al_w, a_src, i);
#pragma unroll
    for (int i = 0; i < 4; ++i) dma_b(0, b_src, i);
#pragma unroll
    for (int i = 0; i < 4; ++i) dma_b(1, b_src + KS * N * 2, i);
#pragma unroll
    for (int i = 0; i < 8; ++i) dma_a(al_w + A_SLOT_BYTES, a_src + 128, i);
#pragma unroll
    for (int i = 0; i < 4; ++i) dma_b(2, b_src + 2 * KS * N * 2, i);
#pragma unroll
    for (int i = 0; i < 4; ++i) dma_b(3, b_src + 3 * KS * N * 2, i);
#pragma unroll
    for (int i = 0; i < 8; ++i) dma_a(al_w + 2 * A_SLOT_BYTES, a_src + 2 * 128, i);
    __builtin_amdgcn_s_waitcnt(0x4F7C);   // vmcnt(28): A pair 0 and B stage 0 have landed
    lds_barrier();
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a[0][i] = a_at(AL + a_row + a_half[0], i);
        b[0][i] = b_at(BL, i);
    }
    // Iteration t (stages 4t .. 4t+3) reads pairs 2t, 2t+1, 2t+1, 2t+2 and
    // fetches pairs 2t+2, 2t+3, 2t+3, 2t+4 and B stages 4t+4 .. 4t+7.  sl0,
    // sl1, sl2 are the slots of pairs 2t, 2t+1, 2t+2 (= 2t+3, 2t+4, ... mod
    // 3); the next iteration's are sl2, sl0, sl1.  Pair 2t+4 is past the last
    // one only in the last iteration (a stage of the tail then reloads pair
    // 2t+3 into its own slot instead: the same bytes, so a concurrent read of
    // it is unaffected).
    uint32_t sl0 = 0, sl1 = A_SLOT_BYTES, sl2 = 2 * A_SLOT_BYTES;
    uint32_t a_t = a_src;                          // A pair 2t
    uint32_t b_t = b_src + 4 * KS * N * 2;         // B stage 4t + 4
    const uint32_t b_u = KS * N * 2;               // one B stage
    uint32_t t2 = 0;                               // 2t
    for (uint32_t s = 0; s + 4 < nstages; s += 4, t2 += 2) {
        const bool last = t2 + 4 > npairs - 1;
        stage(0, sl0, sl2, a_t + 2 * 128, b_t, TailC<0>{});
        stage(1, sl1, sl0, a_t + 3 * 128, b_t + b_u, TailC<0>{});
        stage(2, sl1, sl0, a_t + 3 * 128, b_t + 2 * b_u, TailC<0>{});
        stage(3, sl2, last ? sl0 : sl1, a_t + (last ? 3 : 4) * 128, b_t + 3 * b_u, TailC<0>{});
        const uint32_t s2 = sl2;
        sl2 = sl1;
        sl1 = sl0;
        sl0 = s2;
        a_t += 2 * 128;
        b_t += 4 * b_u;
    }
    stage(0, sl0, 0, 0, 0, TailC<1>{});
    stage(1, sl1, 0, 0, 0, TailC<2>{});
    stage(2, sl1, 0, 0, 0, TailC<3>{});
    stage(3, sl2, 0, 0, 0, TailC<4>{});
    __builtin_amdgcn_s_waitcnt(0);   // no DMA may still target LDS
    // the last MFMAs' results must be written before they are read
    asm volatile("s_nop 15\n\ts_nop 15\n\ts_nop 15\n\ts_nop 15" ::: "memory");

    // Epilogue through LDS (32 KB per wave: the three A slots and the first
    // two B slots, 128 rows of 256 B): lane l holds, for block (i, j), row
    // 16 i + l%16, columns 16 j + 4 (l/16) .. +3, written as one packed 8-byte
    // LDS store (the first version wrote 2-byte elements from the
    // untransposed layout: ~2.8 us per tile, LDS-instruction bound; a DPP
    // exchange to 4-byte pairs still took 2.0 us, VALU bound).  The 8-byte
    // chunk c of row r sits at c ^ 4 (r % 8): the 64 lanes of a write (16 rows
    // x 4 chunks) then fill every bank twice, the fewest for 512 bytes, and
    // 16-byte row chunks stay contiguous for the reads below.
    lds_barrier();
    uint8_t* ct = wave < 3 ? AL + wave * A_SLOT_BYTES : BL;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t row = 16 * i + t;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const f32x4 v = acc[i][j];
            const u32x2 w = {
                __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{v[0], v[1]}, bf16x2)),
                __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{v[2], v[3]}, bf16x2))};
            const uint32_t c8 = (4 * j + g) ^ (4 * (row & 7));
            *reinterpret_cast<u32x2*>(ct + row * 256 + 8 * c8) = w;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    // C is written once and never read here: non-temporal stores keep it out
    // of L2's way (8192^3 random operands at the power limit: 740-748 ->
    // 730-737 us, the same in either run order; output unchanged).
#pragma unroll
    for (int q = 0; q < 32; ++q) {
        const uint32_t row = 4 * q + (lane >> 4), ch = lane & 15;
        const u32x4 v = *reinterpret_cast<const u32x4*>(
            ct + row * 256 + 16 * (ch ^ (2 * (row & 7))));
        __builtin_nontemporal_store(
            v, reinterpret_cast<u32x4*>(C + (size_t)(m0 + wm * 128 + row) * N + n0 + wn * 128 + 8 * ch));
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
