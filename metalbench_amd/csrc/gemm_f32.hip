// fp32 GEMM C[M][N] = A[M][K] @ B[K][N] (row-major), on fp32 MFMA.
//
// Spec: reference mlx/kernels/common/sqr_mm.py:10-11 (mx.matmul), registry
// mlx/kernels/common/registry.py:43-59 and :129 (A@0, B@1, C@2, M@3, N@4,
// K@5; 2*M*N*K flops, 4*(MK+KN+MN) bytes).  The reference kernel reads only N
// (metal/kernels/common/sqr_mm.metal:23); this one honours M, N and K and any
// shape, including ragged edges.
//
// gfx950 design.  fp32 MFMA peak is 256 flop/clk/CU (157.3 TFLOP/s), so at
// 1024^3 the whole problem is ~32k MFMA cycles per CU: the kernel must keep one
// 64x64 tile per CU busy from its first cycle.
//  * workgroup tile 64x64, BK = 32 per stage, LDS double buffered, one barrier
//    per stage; global loads of stage s+1 are in flight during the MFMAs of s;
//  * 4 waves own a 2x2 grid of 32x32 sub-tiles (v_mfma_f32_32x32x2f32);
//    KSPLIT=2 adds a second set of 4 waves that takes the other half of each
//    stage's K range (two waves per SIMD to hide LDS/MFMA latency) and the two
//    partial accumulators are summed through LDS at the end;
//  * A is staged K-contiguous (As[m][k], row stride 36 floats: 16 lanes reading
//    16 consecutive rows with ds_read_b128 cover all 64 banks once);
//    B is staged N-contiguous (Bs[k][n], row stride 68 floats);
//  * K order inside a stage is permuted consistently for A and B: lane l holds
//    A[i][8g + 4*(l/32) + t] for MFMA t of group g and reads the matching row
//    of Bs, so one ds_read_b128 feeds four MFMAs.  The sum over k is the same.
#include "common.h"

namespace mb {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BM = 64, BN = 64, BK = 32;
constexpr int SA = BK + 4;   // As row stride (floats)
constexpr int SB = BN + 4;   // Bs row stride (floats)

template <int KSPLIT, bool VEC>
__global__ __launch_bounds__(256 * KSPLIT)
void gemm_f32_kernel(const float* __restrict__ A, const float* __restrict__ B,
                     float* __restrict__ C, uint32_t M, uint32_t N, uint32_t K,
                     uint32_t tiles_n) {
    constexpr int NT = 256 * KSPLIT;
    constexpr int LOADS = 512 / NT;   // float4 per thread per operand per stage
    __shared__ __attribute__((aligned(16))) float As[2][BM * SA];
    __shared__ __attribute__((aligned(16))) float Bs[2][BK * SB];

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63;
    const uint32_t wave = tid >> 6;
    const uint32_t wk = wave >> 2;            // K half (KSPLIT == 2)
    const uint32_t wm = (wave >> 1) & 1;
    const uint32_t wn = wave & 1;
    const uint32_t tm = blockIdx.x / tiles_n;
    const uint32_t tn = blockIdx.x - tm * tiles_n;
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const uint32_t nstages = (K + BK - 1) / BK;

    float4 ra[LOADS], rb[LOADS];

    auto load = [&](uint32_t k0) {
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const uint32_t q = tid + i * NT;
            // A: 64 rows x 8 float4
            {
                const uint32_t row = q >> 3, kq = (q & 7) * 4;
                const uint32_t gm = m0 + row, gk = k0 + kq;
                if (VEC) {
                    ra[i] = (gm < M && gk < K)
                                ? *reinterpret_cast<const float4*>(A + (size_t)gm * K + gk)
                                : make_float4(0.f, 0.f, 0.f, 0.f);
                } else {
                    float v[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        v[e] = (gm < M && gk + e < K) ? A[(size_t)gm * K + gk + e] : 0.f;
                    ra[i] = make_float4(v[0], v[1], v[2], v[3]);
                }
            }
            // B: 32 rows x 16 float4
            {
                const uint32_t krow = q >> 4, nq = (q & 15) * 4;
                const uint32_t gk = k0 + krow, gn = n0 + nq;
                if (VEC) {
                    rb[i] = (gk < K && gn < N)
                                ? *reinterpret_cast<const float4*>(B + (size_t)gk * N + gn)
                                : make_float4(0.f, 0.f, 0.f, 0.f);
                } else {
                    float v[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        v[e] = (gk < K && gn + e < N) ? B[(size_t)gk * N + gn + e] : 0.f;
                    rb[i] = make_float4(v[0], v[1], v[2], v[3]);
                }
            }
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const uint32_t q = tid + i * NT;
            *reinterpret_cast<float4*>(&As[buf][(q >> 3) * SA + (q & 7) * 4]) = ra[i];
            *reinterpret_cast<float4*>(&Bs[buf][(q >> 4) * SB + (q & 15) * 4]) = rb[i];
        }
    };

    f32x16 acc = {};
    const uint32_t li = lane & 31;     // row (A) / column (B) inside the 32x32 sub-tile
    const uint32_t lh = lane >> 5;     // which 4-wide K quarter of a group

    if (nstages > 0) {
        load(0);
        store(0);
        __syncthreads();
    }
    for (uint32_t s = 0; s < nstages; ++s) {
        const int cur = s & 1;
        if (s + 1 < nstages) load((s + 1) * BK);
        const float* as = &As[cur][(wm * 32 + li) * SA + 4 * lh];
        const float* bs = &Bs[cur][(4 * lh) * SB + wn * 32 + li];
#pragma unroll
        for (int gg = 0; gg < 4 / KSPLIT; ++gg) {
            const int g = (int)wk * (4 / KSPLIT) + gg;
            const float4 a4 = *reinterpret_cast<const float4*>(as + 8 * g);
            const float b0 = bs[(8 * g + 0) * SB];
            const float b1 = bs[(8 * g + 1) * SB];
            const float b2 = bs[(8 * g + 2) * SB];
            const float b3 = bs[(8 * g + 3) * SB];
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a4.x, b0, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a4.y, b1, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a4.z, b2, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a4.w, b3, acc, 0, 0, 0);
        }
        if (s + 1 < nstages) store(cur ^ 1);
        __syncthreads();
    }

    if (KSPLIT == 2) {
        // Second K half hands its partial sums to the first through LDS
        // (4 waves x 64 lanes x 16 floats = 16 KB, inside As).
        float* red = &As[0][0];
        if (wk == 1) {
#pragma unroll
            for (int r = 0; r < 16; ++r) red[((wave & 3) * 16 + r) * 64 + lane] = acc[r];
        }
        __syncthreads();
        if (wk == 1) return;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] += red[((wave & 3) * 16 + r) * 64 + lane];
    }

    // 32x32 accumulator layout: lane l, register r -> row 8*(r/4) + 4*(l/32) + r%4, col l%32.
    const uint32_t gc = n0 + wn * 32 + li;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const uint32_t gr = m0 + wm * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
        if (gr < M && gc < N) C[(size_t)gr * N + gc] = acc[r];
    }
}

int launch_gemm_f32(const float* a, const float* b, float* c, uint32_t m, uint32_t n,
                    uint32_t k, hipStream_t s) {
    if (m == 0 || n == 0) return MB_OK;
    if (!a || !b || !c) return fail(MB_E_ARG, "matmul_f32: null pointer");
    const uint32_t tiles_m = cdiv(m, BM), tiles_n = cdiv(n, BN);
    const uint64_t nblocks = (uint64_t)tiles_m * tiles_n;
    if (nblocks > 0x7fffffffull) return fail(MB_E_ARG, "matmul_f32: shape too large");
    const bool vec = (k % 4 == 0) && (n % 4 == 0) &&
                     (((uintptr_t)a | (uintptr_t)b) & 15) == 0;
    if (vec)
        hipLaunchKernelGGL((gemm_f32_kernel<2, true>), dim3((uint32_t)nblocks), dim3(512), 0, s,
                           a, b, c, m, n, k, tiles_n);
    else
        hipLaunchKernelGGL((gemm_f32_kernel<2, false>), dim3((uint32_t)nblocks), dim3(512), 0, s,
                           a, b, c, m, n, k, tiles_n);
    MB_LAUNCH_CHECK("matmul_f32");
    return MB_OK;
}

// Registry launcher: A@0, B@1 (inputs f32), C@2 (output f32), M@3, N@4, K@5.
int run_gemm_f32(const Bindings& bs, hipStream_t s, PartMarks*) {
    uint32_t m, n, k;
    int rc;
    if ((rc = bs.u32(3, &m, "M")) || (rc = bs.u32(4, &n, "N")) || (rc = bs.u32(5, &k, "K")))
        return rc;
    void *a, *b, *c;
    if ((rc = bs.buffer(0, MB_DTYPE_F32, (uint64_t)m * k * 4, false, &a, "A")) ||
        (rc = bs.buffer(1, MB_DTYPE_F32, (uint64_t)k * n * 4, false, &b, "B")) ||
        (rc = bs.buffer(2, MB_DTYPE_F32, (uint64_t)m * n * 4, true, &c, "C")))
        return rc;
    return launch_gemm_f32((const float*)a, (const float*)b, (float*)c, m, n, k, s);
}

}  // namespace

void register_gemm_f32() {
    // Both names resolve to the same kernel: sqr_mm and rect_mm share the spec.
    register_kernel({"sqr_matmul_f32", run_gemm_f32,
                     reinterpret_cast<const void*>(&gemm_f32_kernel<2, true>), 1});
    register_kernel({"rect_matmul_f32", run_gemm_f32,
                     reinterpret_cast<const void*>(&gemm_f32_kernel<2, true>), 1});
}

}  // namespace mb

extern "C" int mb_launch_matmul_f32(const float* a, const float* b, float* c, uint32_t m,
                                    uint32_t n, uint32_t k, void* stream) {
    mb::clear_error();
    if (!mb::initialized()) return mb::fail(MB_E_STATE, "mb_init() has not been called");
    return mb::launch_gemm_f32(a, b, c, m, n, k, mb::stream_or_default(stream));
}
