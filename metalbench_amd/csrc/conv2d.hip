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
// gfx950 design:
//  * workgroup tile 64 pixels x 64 channels, BK = 32; 4 waves each own a 32x32
//    sub-tile (v_mfma_f32_32x32x2f32); KSPLIT = 2 doubles the waves (two per
//    SIMD), the second set taking the other half of each stage's K range;
//  * both operands are staged K-contiguous in LDS (row stride 36 floats: 16
//    lanes reading 16 consecutive rows with ds_read_b128 cover all 64 banks
//    once), so one ds_read_b128 per operand feeds four MFMAs;
//  * fast path (C % 32 == 0): a BK = 32 stage never straddles a filter tap
//    (r, s), so the tap is uniform per stage and each A row is one contiguous
//    128-byte NHWC channel run, loaded as float4 or zero-filled at the image
//    border.  The per-row (n, p, q) decomposition is hoisted out of the K loop
//    (the reference kernel hoists its im2col math the same way,
//    metal/kernels/common/conv2d/default.metal:80-89);
//  * any other shape takes the generic path: element-wise gathers with the
//    (r, s, c) decomposition per element.
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
};

template <int KSPLIT, bool FAST>
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

    // Two register stages (see the stage loop below).  FAST loads are buffer
    // loads: taps outside the image and k past the filter read zeros through
    // an out-of-range offset, so the loads carry no branches.
    float4 ra[2][LOADS], rb[2][LOADS];
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(X), 0, sh.n * sh.h * sh.w * sh.c * 4, 0x00020000u);
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(Wt), 0, sh.o * sh.k * 4, 0x00020000u);
    auto ld4 = [](__amdgpu_buffer_rsrc_t rsrc, uint32_t off) {
        return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0));
    };
    auto load = [&](int set, uint32_t k0) {
        if (FAST) {
            // Uniform tap for the stage: k0 = (r*S + s)*C + c0 (k0 past the filter
            // gives r >= R, which the row test below turns into zeros).
            const uint32_t rs = k0 / sh.c, c0 = k0 - rs * sh.c;
            const uint32_t r = rs / sh.s, s = rs - r * sh.s;
#pragma unroll
            for (int i = 0; i < LOADS; ++i) {
                const uint32_t q4 = ((tid + i * NT) % KQ) * 4;
                const int32_t hi = row_h0[i] + (int32_t)r, wi = row_w0[i] + (int32_t)s;
                const bool in = row_ok[i] && k0 < sh.k && hi >= 0 && hi < (int32_t)sh.h &&
                                wi >= 0 && wi < (int32_t)sh.w;
                const uint32_t off =
                    in ? ((uint32_t)row_base[i] + ((uint32_t)hi * sh.w + wi) * sh.c + c0 + q4) * 4
                       : 0x80000000u;
                ra[set][i] = ld4(xrs, off);
            }
        } else {
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
        }
        // B tile: 64 output channels x 32 k, rows of w are K-contiguous.
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const uint32_t q = tid + i * NT;
            const uint32_t oc = n0 + q / KQ, kq = k0 + (q % KQ) * 4;
            if (FAST) {
                rb[set][i] = ld4(wrs, (oc < sh.o && kq < sh.k) ? (oc * sh.k + kq) * 4 : 0x80000000u);
            } else {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    v[e] = (oc < sh.o && kq + e < sh.k) ? Wt[(uint64_t)oc * sh.k + kq + e] : 0.f;
                rb[set][i] = make_float4(v[0], v[1], v[2], v[3]);
            }
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
    // FAST: an even number of stages and no branch in the loop body (a stage
    // past K multiplies the zeros its out-of-range loads stored).
    const uint32_t nrun = FAST ? (nstages + 1) & ~1u : nstages;
    if (nstages > 0) {
        load(0, 0);
        if (FAST || nstages > 1) load(1, BK);
        store(0, 0);
        __syncthreads();
    }
    // Stage st: the loads of stage st+2 go into the register set stored at
    // the end of stage st-1 and stay in flight for two stages; stage st+1's
    // registers go to LDS in the middle of stage st's MFMAs.  The operands of
    // group g+1 are read from LDS while group g's MFMAs run.
    auto stage = [&](uint32_t st, int cur) {
        if (FAST || st + 2 < nstages) load(cur, (st + 2) * BK);
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
            if (gg == NG / 2 && (FAST || st + 1 < nstages)) store(cur ^ 1, cur ^ 1);
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
    for (uint32_t st = 0; st < nrun; st += 2) {
        stage(st, 0);
        if (FAST || st + 1 < nstages) stage(st + 1, 1);
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
    if (sh.m == 0 || o == 0) return MB_OK;
    const uint32_t tiles_m = cdiv(sh.m, BM), tiles_n = cdiv(o, BN);
    const uint64_t nblocks = (uint64_t)tiles_m * tiles_n;
    if (nblocks > 0x7fffffffull) return fail(MB_E_ARG, "conv2d_f32: shape too large");
    // FAST: a stage never straddles a tap, 16-byte aligned rows, and buffer-load
    // offsets of both operands within 2 GB
    const bool fast = (c % BK == 0) && ((((uintptr_t)x) | ((uintptr_t)w)) & 15) == 0 &&
                      (uint64_t)n * h * wd * c * 4 < 0x80000000ull &&
                      (uint64_t)o * k * 4 < 0x80000000ull;
    if (fast)
        hipLaunchKernelGGL((conv2d_f32_kernel<2, true>), dim3((uint32_t)nblocks), dim3(512), 0, st,
                           x, w, y, sh, tiles_n);
    else
        hipLaunchKernelGGL((conv2d_f32_kernel<2, false>), dim3((uint32_t)nblocks), dim3(512), 0, st,
                           x, w, y, sh, tiles_n);
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
                     reinterpret_cast<const void*>(&conv2d_f32_kernel<2, true>), 1});
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
