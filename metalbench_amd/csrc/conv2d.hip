// conv2d as an implicit GEMM on fp32 MFMA: NHWC input, OHWI weight, NHWC output.
//
// Spec: reference mlx/kernels/common/conv2d.py:11-12 (mx.conv2d: cross-
// correlation, dilation 1, groups 1), registry mlx/kernels/common/registry.py:
// 469-477 (x@0, w@1, y@2, N@3 H@4 W@5 C@6 O@7 R@8 S@9 stride@10).  This build
// adds zero padding (pad@11); the reference kernel only has valid padding.
//
// GEMM view: M = N*P*Q output pixels, N_gemm = O channels, K = R*S*C with
// k = (r*S + s)*C + c, so
//   A[m][k] = x[n][p*st + r - pad][q*st + s - pad][c]   (0 outside the image)
//   B[k][o] = w[o][k]                                    (OHWI rows are K-contiguous)
// and y[m][o] is exactly the NHWC output.
//
// gfx950 design (v_mfma_f32_32x32x2f32 on 32x32 sub-tiles; two K halves per
// stage on separate waves, summed through LDS at the end):
//  * fast path (C % 32 == 0, conv2d_f32_dma_kernel): a BK = 32 stage never
//    straddles a filter tap (r, s), so the tap is uniform per stage and each
//    A row is one contiguous 128-byte NHWC channel run, fetched by DMA
//    straight into LDS or zero-filled at the image border.  The per-row
//    (n, p, q) decomposition is hoisted out of the K loop (the reference
//    kernel hoists its im2col math the same way,
//    metal/kernels/common/conv2d/default.metal:80-89).  Tiles are 32 pixels
//    x 64 channels (details at the kernel);
//  * any other shape (conv2d_f32_kernel): 64 x 64 tiles with 8 waves, both
//    operands gathered element-wise, staged two stages ahead in registers
//    and stored K-contiguous in LDS (row stride 36 floats: 16 lanes reading
//    16 consecutive rows with ds_read_b128 cover all 64 banks once), so one
//    ds_read_b128 per operand feeds four MFMAs.
#include "common.h"

namespace mb {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BM = 64, BN = 64, BK = 32;
constexpr int SK = BK + 4;   // LDS row stride (floats), both operands
constexpr int KQ = BK / 4;   // float4s per K-contiguous row of a stage

struct ConvShape {
    uint32_t n, h, w, c, o, r, s, stride, pad, p, q;
    uint32_t m;   // n*p*q
    uint32_t k;   // r*s*c
    uint32_t q_mul, q_sh, p_mul, p_sh;   // x / q and x / p for x < 2^31 (mul 0: divisor 1)
};

// floor(x / d) for x < 2^31 from (mul, sh) = magic_u31(d) (launch_conv2d).
// The DMA kernel divides pixel indices below M, and its path requires
// M O 4 < 2^31.
__device__ __forceinline__ uint32_t div_magic(uint32_t x, uint32_t mul, uint32_t sh) {
    return mul ? __umulhi(x, mul) >> sh : x;
}

template <int KSPLIT>
__global__ __launch_bounds__(256 * KSPLIT)
void conv2d_f32_kernel(const float* __restrict__ X, const float* __restrict__ Wt,
                       float* __restrict__ Y, ConvShape sh, uint32_t tiles_n) {
    constexpr int NT = 256 * KSPLIT;
    constexpr int LOADS = (BM * BK / 4) / NT;   // float4 per thread per operand per stage
    __shared__ __attribute__((aligned(16))) float As[2][BM * SK];
    __shared__ __attribute__((aligned(16))) float Bs[2][BN * SK];

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63;
    const uint32_t wave = tid >> 6;
    const uint32_t wk = wave >> 2;
    const uint32_t wm = (wave >> 1) & 1;
    const uint32_t wn = wave & 1;
    const uint32_t tm = blockIdx.x / tiles_n;
    const uint32_t tn = blockIdx.x - tm * tiles_n;
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const uint32_t nstages = (sh.k + BK - 1) / BK;

    // Per-thread rows of the A tile: row = q / KQ (q = tid + i*NT), float4 column q % KQ.
    // Hoisted im2col decomposition: pixel (n, p, q) -> image base and top-left tap.
    int32_t row_h0[LOADS], row_w0[LOADS];
    uint64_t row_base[LOADS];
    bool row_ok[LOADS];
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const uint32_t m = m0 + (tid + i * NT) / KQ;
        row_ok[i] = m < sh.m;
        const uint32_t mm = row_ok[i] ? m : 0;
        const uint32_t qq = mm % sh.q;
        const uint32_t t = mm / sh.q;
        const uint32_t pp = t % sh.p;
        const uint32_t nn = t / sh.p;
        row_h0[i] = (int32_t)(pp * sh.stride) - (int32_t)sh.pad;
        row_w0[i] = (int32_t)(qq * sh.stride) - (int32_t)sh.pad;
        row_base[i] = (uint64_t)nn * sh.h * sh.w * sh.c;
    }

    // Two register stages (see the stage loop below); element-wise gathers.
    float4 ra[2][LOADS], rb[2][LOADS];
    auto load = [&](int set, uint32_t k0) {
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const uint32_t q4 = ((tid + i * NT) % KQ) * 4;
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t kk = k0 + q4 + e;
                v[e] = 0.f;
                if (row_ok[i] && kk < sh.k) {
                    const uint32_t rs = kk / sh.c, c = kk - rs * sh.c;
                    const uint32_t r = rs / sh.s, s = rs - r * sh.s;
                    const int32_t hi = row_h0[i] + (int32_t)r, wi = row_w0[i] + (int32_t)s;
                    if (hi >= 0 && hi < (int32_t)sh.h && wi >= 0 && wi < (int32_t)sh.w)
                        v[e] = X[row_base[i] + ((uint64_t)hi * sh.w + wi) * sh.c + c];
                }
            }
            ra[set][i] = make_float4(v[0], v[1], v[2], v[3]);
        }
        // B tile: 64 output channels x 32 k, rows of w are K-contiguous.
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const uint32_t q = tid + i * NT;
            const uint32_t oc = n0 + q / KQ, kq = k0 + (q % KQ) * 4;
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                v[e] = (oc < sh.o && kq + e < sh.k) ? Wt[(uint64_t)oc * sh.k + kq + e] : 0.f;
            rb[set][i] = make_float4(v[0], v[1], v[2], v[3]);
        }
    };
    auto store = [&](int set, int buf) {
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const uint32_t q = tid + i * NT;
            *reinterpret_cast<float4*>(&As[buf][(q / KQ) * SK + (q % KQ) * 4]) = ra[set][i];
            *reinterpret_cast<float4*>(&Bs[buf][(q / KQ) * SK + (q % KQ) * 4]) = rb[set][i];
        }
    };

    f32x16 acc = {};
    const uint32_t li = lane & 31, lh = lane >> 5;
    if (nstages > 0) {
        load(0, 0);
        if (nstages > 1) load(1, BK);
        store(0, 0);
        __syncthreads();
    }
    // Stage st: the loads of stage st+2 go into the register set stored at
    // the end of stage st-1 and stay in flight for two stages; stage st+1's
    // registers go to LDS in the middle of stage st's MFMAs.  The operands of
    // group g+1 are read from LDS while group g's MFMAs run.
    auto stage = [&](uint32_t st, int cur) {
        if (st + 2 < nstages) load(cur, (st + 2) * BK);
        __builtin_amdgcn_sched_barrier(0);
        const float* as = &As[cur][(wm * 32 + li) * SK + 4 * lh];
        const float* bs = &Bs[cur][(wn * 32 + li) * SK + 4 * lh];
        constexpr int NG = BK / 8 / KSPLIT;
        float4 a4[2], b4[2];
        auto read_ops = [&](int gg, int slot) {
            const int g = (int)wk * NG + gg;
            a4[slot] = *reinterpret_cast<const float4*>(as + 8 * g);
            b4[slot] = *reinterpret_cast<const float4*>(bs + 8 * g);
        };
        read_ops(0, 0);
#pragma unroll
        for (int gg = 0; gg < NG; ++gg) {
            __builtin_amdgcn_sched_barrier(0);
            if (gg + 1 < NG) read_ops(gg + 1, (gg + 1) & 1);
            if (gg == NG / 2 && st + 1 < nstages) store(cur ^ 1, cur ^ 1);
            __builtin_amdgcn_sched_barrier(0);
            const int sl = gg & 1;
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a4[sl].x, b4[sl].x, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a4[sl].y, b4[sl].y, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a4[sl].z, b4[sl].z, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a4[sl].w, b4[sl].w, acc, 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
    };
    for (uint32_t st = 0; st < nstages; st += 2) {
        stage(st, 0);
        if (st + 1 < nstages) stage(st + 1, 1);
    }

    if (KSPLIT == 2) {
        float* red = &As[0][0];   // 4 waves x 16 x 64 floats = 16 KB < sizeof(As)
        if (wk == 1) {
#pragma unroll
            for (int r = 0; r < 16; ++r) red[((wave & 3) * 16 + r) * 64 + lane] = acc[r];
        }
        __syncthreads();
        if (wk == 1) return;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] += red[((wave & 3) * 16 + r) * 64 + lane];
    }

    // 32x32 accumulator: lane l, reg r -> row 8*(r/4) + 4*(l/32) + r%4, col l%32.
    const uint32_t gc = n0 + wn * 32 + li;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const uint32_t gr = m0 + wm * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
        if (gr < sh.m && gc < sh.o) Y[(uint64_t)gr * sh.o + gc] = acc[r];
    }
}

// Fast-path kernel (C % 32 == 0): the operands go global -> LDS by DMA
// (buffer_load ... lds) into a ring of NBUF = 2 32-deep k stages: no staging
// registers and no LDS store instructions, whose VGPR reads stall the MFMA
// issue.  A tile is 32 WMS pixels x 64 channels with 4 WMS waves (K halves x
// row groups x column halves, v_mfma_f32_32x32x2f32 on 32x32 sub-tiles, the
// K halves summed through LDS).  The launcher uses WMS = 1: 32-pixel tiles,
// 12 KB per ring slot, six workgroups per CU, so the 3136 tiles of the
// 32x56x56 shape finish in finer rounds than 64-pixel tiles would.
//  * a slot holds BMT A rows (output pixels: one NHWC channel run of the
//    stage's tap) and 64 B rows (output channels: OHWI weight rows are
//    K-contiguous), each 32 k = 128 bytes; 16-byte chunk c of row r sits in
//    slot c ^ ((r / 2) % 8), so a ds_read_b128 of 16 consecutive rows touches
//    16 distinct bank groups 8 (r % 2) + slot;
//  * a DMA instruction writes a wave's 64 x 16 B = eight rows contiguously;
//    wave w fetches A rows 8 w .. 8 w + 7 and 8 x BI B rows, lane l the chunk
//    that slot l % 8 of its row holds.  Taps outside the image use an
//    out-of-range offset, which the DMA lands as zeros; fetches past the last
//    stage re-fetch it into a slot that is never read;
//  * stage s (slot s % NBUF): group 0 reads group 1's operands under its 4
//    MFMAs; before group 1 the wave waits for its DMAs of stage s+1, passes an
//    LDS barrier, refills slot s % NBUF with stage s+NBUF and reads stage
//    s+1's first operands under group 1's MFMAs.
// Tiles are taken in XCD-aware order (each XCD a contiguous pixel range, 4
// whole images at this shape), so the rows a filter's halo shares between
// neighbouring tiles are fetched into one L2: FETCH_SIZE per launch fell from
// 3.17x to 1.04x the input + weight bytes, at unchanged time.
// Measured on the 32x56x56x64 -> 64 shape, alternated on one box: 90.2-91.3
// us against 95.2-96.1 us for the register-staged version of this path
// (conv2d_f32_kernel's layout with buffer loads); 64-pixel tiles (WMS = 2)
// 91.5-92.5 us; a ring of three or four stages was slower (fewer workgroups
// per CU).  The stage's tap used to be decoded from k0 in the loop (two
// runtime divisions, bounds checks as branches: ~8 scalar and ~4 vector
// instructions per MFMA, the MFMA pipe 71 % busy); advanced incrementally
// instead, with the k and channel offsets in the DMA's scalar offset, the
// same launch went from 74.8 to 64.3 us at the working clock (bit-identical).
constexpr int NBUF = 2;
template <uint32_t V> struct SlotC { static constexpr uint32_t v = V; };

// WMS = 32-pixel row groups per tile (tile BMT = 32 WMS pixels x 64 channels,
// 4 WMS waves).
template <int WMS>
__global__ __launch_bounds__(256 * WMS)
void conv2d_f32_dma_kernel(const float* __restrict__ X, const float* __restrict__ Wt,
                           float* __restrict__ Y, ConvShape sh, uint32_t tiles_n) {
    constexpr int BMT = 32 * WMS, NW = 4 * WMS;
    constexpr int A_BYTES = BMT * BK * 4, C_SLOT = (BMT + BN) * BK;   // floats per ring slot
    constexpr int BI = 2 / WMS;            // B DMA instructions per wave per stage
    constexpr int D = 1 + BI;              // DMA instructions per wave per stage
    __shared__ __attribute__((aligned(1024))) float L[NBUF * C_SLOT];

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wk = wave / (2 * WMS), wm = (wave >> 1) % WMS, wn = wave & 1;
    // XCD-aware order: hardware block b runs on XCD b % 8, so XCD x gets the
    // contiguous logical range [x G/8, (x+1) G/8) of the G tiles (pixel
    // order): tiles that share input rows (the filter's halo) share an L2.
    uint32_t lb = blockIdx.x;
    if ((gridDim.x & 7) == 0) lb = (blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3);
    const uint32_t tm = lb / tiles_n;
    const uint32_t tn = lb - tm * tiles_n;
    const uint32_t m0 = tm * BMT, n0 = tn * BN;
    const uint32_t nstages = (sh.k + BK - 1) / BK;

    const i32x4 xrs = dma_rsrc(X, sh.n * sh.h * sh.w * sh.c * 4);
    const i32x4 wrs = dma_rsrc(Wt, sh.o * sh.k * 4);
    // This lane's DMA row (8 w + l/8) and chunk; the pixel's image base and
    // top-left tap are hoisted out of the K loop.
    const uint32_t drow = 8 * wave + (lane >> 3);
    const uint32_t dch = (lane & 7) ^ ((drow >> 1) & 7);
    const uint32_t m = m0 + drow;
    const bool m_ok = m < sh.m;
    const uint32_t mm = m_ok ? m : 0;
    // (multiply-high divisions: the compiler's 32-bit divide is ~20 VALU
    // instructions, and this set-up runs beside other workgroups' MFMA loops)
    const uint32_t t = div_magic(mm, sh.q_mul, sh.q_sh), qq = mm - t * sh.q;
    const uint32_t nn = div_magic(t, sh.p_mul, sh.p_sh), pp = t - nn * sh.p;
    const int32_t h0 = (int32_t)(pp * sh.stride) - (int32_t)sh.pad;
    const int32_t w0 = (int32_t)(qq * sh.stride) - (int32_t)sh.pad;
    const uint32_t xbase = (nn * sh.h * sh.w * sh.c + 4 * dch) * 4;   // bytes
    // This lane's byte offset of tap (r, s), or an out-of-range offset (the
    // DMA lands zeros) when the tap falls outside the image.
    auto tap_off = [&](uint32_t r, uint32_t s) -> uint32_t {
        const uint32_t hi = (uint32_t)(h0 + (int32_t)r), wi = (uint32_t)(w0 + (int32_t)s);
        const bool in = m_ok && hi < sh.h && wi < sh.w;
        return in ? xbase + (hi * sh.w + wi) * sh.c * 4 : 0x80000000u;
    };
    // B rows (output channels) of this wave: BI instructions of 8 rows each
    uint32_t wbase[BI];
#pragma unroll
    for (int i = 0; i < BI; ++i) {
        const uint32_t brow = 8 * (BI * wave + i) + (lane >> 3);
        const uint32_t bch = (lane & 7) ^ ((brow >> 1) & 7);
        const uint32_t oc = n0 + brow;
        wbase[i] = oc < sh.o ? (oc * sh.k + 4 * bch) * 4 : 0x80000000u;
    }
    const uint32_t l0 = lds_addr(L);
    const uint32_t dst = 8 * wave * 128;   // this wave's A rows in a slot
    // The next stage to fetch: k offset kd, tap (tr, ts), channel offset tc.
    // Advanced incrementally (no division in the loop); the k and channel
    // offsets ride in the DMA's scalar offset, so only a tap change touches
    // the per-lane offset.  Fetches past the last stage re-fetch it into a
    // slot that is never read (the same bytes, in bounds).
    uint32_t kd = 0, tr = 0, ts = 0, tc = 0;
    uint32_t xoff = tap_off(0, 0);
    auto dma_next = [&](uint32_t slot) {
        dma16(xrs, l0 + slot * (C_SLOT * 4) + dst, xoff, tc * 4);
#pragma unroll
        for (int i = 0; i < BI; ++i)
            dma16(wrs, l0 + slot * (C_SLOT * 4) + A_BYTES + 8 * (BI * wave + i) * 128, wbase[i],
                  kd * 4);
        if (kd + BK < sh.k) {
            kd += BK;
            tc += BK;
            if (tc == sh.c) {
                tc = 0;
                if (++ts == sh.s) { ts = 0; ++tr; }
                xoff = tap_off(tr, ts);
            }
        }
    };

    const uint32_t li = lane & 31, lh = lane >> 5;
    // operand of group g (8 k): row wm*32 + li (A) / wn*32 + li (B), chunk
    // 2 g + lh, in slot chunk ^ ((li/2) % 8)
    const uint32_t a_row = (wm * 32 + li) * 128, b_row = A_BYTES + (wn * 32 + li) * 128;
    const uint32_t sw = (li >> 1) & 7;
    const uint8_t* l8 = reinterpret_cast<const uint8_t*>(L);
    float4 a4[2], b4[2];
    auto read_ops = [&](uint32_t slot, int gg, int c) {
        const uint32_t g = 2 * wk + gg;
        const uint8_t* base = l8 + slot * (C_SLOT * 4) + 16 * ((2 * g + lh) ^ sw);
        a4[c] = *reinterpret_cast<const float4*>(base + a_row);
        b4[c] = *reinterpret_cast<const float4*>(base + b_row);
    };
    f32x16 acc = {};
    auto mfma4 = [&](int c) {
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a4[c].x, b4[c].x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a4[c].y, b4[c].y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a4[c].z, b4[c].z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a4[c].w, b4[c].w, acc, 0, 0, 0);
    };
    // Stage s in slot s % 2: group 0 reads group 1's operands under its 4
    // MFMAs; the wave waits for its DMAs of stage s+1, passes an LDS barrier,
    // refills slot s % 2 with stage s+2 and reads stage s+1's first operands
    // under group 1's MFMAs.
    auto stage = [&](auto SL) {
        constexpr uint32_t slot = decltype(SL)::v, nslot = slot ^ 1u;
        __builtin_amdgcn_sched_barrier(0);
        read_ops(slot, 1, 1);
        mfma4(0);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): stage s+1 has landed
        lds_barrier();
        __builtin_amdgcn_sched_barrier(0);
        dma_next(slot);
        read_ops(nslot, 0, 0);
        mfma4(1);
        __builtin_amdgcn_sched_barrier(0);
    };

    static_assert(NBUF == 2, "the loop below alternates two slots");
    dma_next(0);
    dma_next(1);
    __builtin_amdgcn_s_waitcnt(0x0F70 | D);   // vmcnt(D): stage 0 has landed
    lds_barrier();
    read_ops(0, 0, 0);
    for (uint32_t st = 0; st < nstages; st += 2) {
        stage(SlotC<0>{});
        if (st + 1 < nstages) stage(SlotC<1>{});
    }
    __builtin_amdgcn_s_waitcnt(0);   // no DMA may still target LDS
    lds_barrier();

    // The two K halves of each 32 x 32 block finish half of it each.  In the
    // 32x32 accumulator layout (lane l, reg r -> row 8 (r / 4) + 4 (l / 32) +
    // r % 4, col l % 32) registers 0-7 hold rows 0-15 and registers 8-15 rows
    // 16-31: the wk = 0 wave keeps 0-7 and hands 8-15 to its partner through
    // LDS, the wk = 1 wave keeps 8-15 and hands 0-7.  Each adds the partner's
    // partial to its own (a + b == b + a exactly) and stores its 16 rows, so
    // each wave issues half the epilogue's LDS accesses and stores.
    const uint32_t rw = wave % (NW / 2);
    float* mine = L + (rw * 2 + wk) * 8 * 64;   // NW waves x 8 x 64 floats
    const float* theirs = L + (rw * 2 + (wk ^ 1)) * 8 * 64;
    if (wk == 0) {
#pragma unroll
        for (int r = 0; r < 8; ++r) mine[r * 64 + lane] = acc[8 + r];
    } else {
#pragma unroll
        for (int r = 0; r < 8; ++r) mine[r * 64 + lane] = acc[r];
    }
    __syncthreads();

    // Buffer stores through a descriptor clipped to the output: rows past M
    // fall outside it, columns past O take an out-of-range offset.  One
    // 32-bit add per store instead of a guarded 64-bit address: this
    // epilogue runs beside five other workgroups' MFMA loops, where every
    // VALU instruction waits for an issue slot (3.9-4.3 us per tile with the
    // guarded stores, stamped).
    const uint32_t gc = n0 + wn * 32 + li;
    const __amdgpu_buffer_rsrc_t yrs = __builtin_amdgcn_make_buffer_rsrc(
        Y, 0, __builtin_amdgcn_readfirstlane(sh.m * sh.o * 4), 0x00020000);
    const uint32_t ybase = gc < sh.o ? ((m0 + wm * 32 + 4 * lh) * sh.o + gc) * 4 : 0x80000000u;
    const uint32_t o4 = sh.o * 4;
    auto finish = [&](auto base_c) {
        constexpr int R0 = decltype(base_c)::value;
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const float v = acc[R0 + r] + theirs[r * 64 + lane];
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), yrs,
                                                  ybase + (8 * ((R0 + r) >> 2) + (r & 3)) * o4, 0, 0);
        }
    };
    if (wk == 0) finish(std::integral_constant<int, 0>{});
    else finish(std::integral_constant<int, 8>{});
}

int launch_conv2d(const float* x, const float* w, float* y, uint32_t n, uint32_t h, uint32_t wd,
                  uint32_t c, uint32_t o, uint32_t r, uint32_t s, uint32_t stride, uint32_t pad,
                  hipStream_t st) {
    if (!x || !w || !y) return fail(MB_E_ARG, "conv2d_f32: null pointer");
    if (stride == 0) return fail(MB_E_ARG, "conv2d_f32: stride must be >= 1");
    if (r == 0 || s == 0 || h + 2 * pad < r || wd + 2 * pad < s)
        return fail(MB_E_ARG, "conv2d_f32: filter %ux%u larger than padded input %ux%u", r, s,
                    h + 2 * pad, wd + 2 * pad);
    ConvShape sh;
    sh.n = n; sh.h = h; sh.w = wd; sh.c = c; sh.o = o; sh.r = r; sh.s = s;
    sh.stride = stride; sh.pad = pad;
    sh.p = (h + 2 * pad - r) / stride + 1;
    sh.q = (wd + 2 * pad - s) / stride + 1;
    const uint64_t m = (uint64_t)n * sh.p * sh.q, k = (uint64_t)r * s * c;
    if (m > 0xffffffffull || k > 0xffffffffull ||
        (uint64_t)n * h * wd * c > (1ull << 40))
        return fail(MB_E_ARG, "conv2d_f32: shape too large");
    sh.m = (uint32_t)m;
    sh.k = (uint32_t)k;
    // floor(x / d) = umulhi(x, M) >> (s - 1) for x < 2^31, with s = ceil(log2 d)
    // and M = floor(2^(31+s) / d) + 1 < 2^32: M d - 2^(31+s) lies in (0, d],
    // so x (M d - 2^(31+s)) < 2^31 d <= 2^(31+s) and the error stays below
    // one step.  d = 1 takes the plain path (mul 0).
    auto magic_u31 = [](uint32_t d, uint32_t* mul, uint32_t* shift) {
        if (d <= 1) { *mul = 0; *shift = 0; return; }
        uint32_t l = 0;
        while ((1ull << l) < d) ++l;
        *mul = (uint32_t)(((1ull << (31 + l)) / d) + 1);
        *shift = l - 1;
    };
    magic_u31(sh.q, &sh.q_mul, &sh.q_sh);
    magic_u31(sh.p, &sh.p_mul, &sh.p_sh);
    if (sh.m == 0 || o == 0) return MB_OK;
    const uint32_t tiles_m = cdiv(sh.m, BM), tiles_n = cdiv(o, BN);
    const uint64_t nblocks = (uint64_t)tiles_m * tiles_n;
    if (nblocks > 0x7fffffffull) return fail(MB_E_ARG, "conv2d_f32: shape too large");
    // fast path: a stage never straddles a tap, 16-byte aligned rows, and
    // buffer offsets of both operands and of the output within 2 GB
    const bool fast = (c % BK == 0) && ((((uintptr_t)x) | ((uintptr_t)w)) & 15) == 0 &&
                      (uint64_t)n * h * wd * c * 4 < 0x80000000ull &&
                      (uint64_t)o * k * 4 < 0x80000000ull && (uint64_t)sh.m * o * 4 < 0x80000000ull;
    if (fast) {
        const uint64_t dma_blocks = (uint64_t)cdiv(sh.m, 32) * tiles_n;
        if (dma_blocks > 0x7fffffffull) return fail(MB_E_ARG, "conv2d_f32: shape too large");
        hipLaunchKernelGGL(conv2d_f32_dma_kernel<1>, dim3((uint32_t)dma_blocks), dim3(256), 0, st,
                           x, w, y, sh, tiles_n);
    } else {
        hipLaunchKernelGGL((conv2d_f32_kernel<2>), dim3((uint32_t)nblocks), dim3(512), 0, st,
                           x, w, y, sh, tiles_n);
    }
    MB_LAUNCH_CHECK("conv2d_f32");
    return MB_OK;
}

// Registry launcher: x@0, w@1 (inputs), y@2 (output), N@3 H@4 W@5 C@6 O@7 R@8
// S@9 stride@10 and, optionally, pad@11 (default 0 = the reference's valid conv).
int run_conv2d(const Bindings& bs, hipStream_t st, PartMarks*) {
    uint32_t n, h, w, c, o, r, s, stride = 1, pad = 0;
    int rc;
    if ((rc = bs.u32(3, &n, "N")) || (rc = bs.u32(4, &h, "H")) || (rc = bs.u32(5, &w, "W")) ||
        (rc = bs.u32(6, &c, "C")) || (rc = bs.u32(7, &o, "O")) || (rc = bs.u32(8, &r, "R")) ||
        (rc = bs.u32(9, &s, "S")))
        return rc;
    if (bs.slot[10] && (rc = bs.u32(10, &stride, "stride"))) return rc;
    if (bs.slot[11] && (rc = bs.u32(11, &pad, "pad"))) return rc;
    if (stride == 0) return fail(MB_E_ARG, "conv2d_f32: stride must be >= 1");
    if (h + 2 * pad < r || w + 2 * pad < s)
        return fail(MB_E_ARG, "conv2d_f32: filter larger than padded input");
    const uint64_t p = (h + 2 * pad - r) / stride + 1, q = (w + 2 * pad - s) / stride + 1;
    void *xp, *wp, *yp;
    if ((rc = bs.buffer(0, MB_DTYPE_F32, (uint64_t)n * h * w * c * 4, false, &xp, "x")) ||
        (rc = bs.buffer(1, MB_DTYPE_F32, (uint64_t)o * r * s * c * 4, false, &wp, "w")) ||
        (rc = bs.buffer(2, MB_DTYPE_F32, (uint64_t)n * p * q * o * 4, true, &yp, "y")))
        return rc;
    return launch_conv2d((const float*)xp, (const float*)wp, (float*)yp, n, h, w, c, o, r, s,
                         stride, pad, st);
}

}  // namespace

void register_conv2d() {
    register_kernel({"conv2d_f32", run_conv2d,
                     reinterpret_cast<const void*>(&conv2d_f32_dma_kernel<1>), 1});
}

}  // namespace mb

extern "C" int mb_launch_conv2d_nhwc_f32(const float* x, const float* w, float* y, uint32_t n,
                                         uint32_t h, uint32_t wd, uint32_t c, uint32_t o,
                                         uint32_t r, uint32_t s, uint32_t stride, uint32_t pad,
                                         void* stream) {
    mb::clear_error();
    if (!mb::initialized()) return mb::fail(MB_E_STATE, "mb_init() has not been called");
    return mb::launch_conv2d(x, w, y, n, h, wd, c, o, r, s, stride, pad,
                             mb::stream_or_default(stream));
}
