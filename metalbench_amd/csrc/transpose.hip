// 2D fp32 transpose B[c][r] = A[r][c], bit exact.
//
// Spec: reference mlx/kernels/common/transpose_2d.py:10-11 (mx.transpose),
// registry mlx/kernels/common/registry.py:165-179 (input binding 0, output
// binding 1, scalars rows@2 and cols@3, rtol = atol = 0).
//
// gfx950 design (HBM bound, 0 flops, 2*rows*cols*4 algorithmic bytes):
//  * persistent workgroups, one per CU (256 threads), walk 128x128 tiles
//    (64 KB) in column-major tile order, so concurrently running workgroups
//    write adjacent 512-byte pieces of the same rows of B.  One workgroup per
//    CU beats two (5.7 vs 5.5 TB/s cold): fewer concurrent streams, better
//    DRAM page locality;
//  * when every tile is full, each workgroup keeps three tiles in registers:
//    two tiles' loads stay in flight while the third is transposed and
//    stored (transpose_full_kernel);
//  * global reads: 32 lanes load a 512-byte row segment of A as float4 (16
//    loads per lane), non-temporal: each byte is read once;
//  * the tile goes through LDS as float[128][129]: the +1 column of padding
//    makes both the row-wise writes and the column-wise reads conflict free
//    (bank = (row + col) mod 64);
//  * otherwise (transpose_2d_f32_kernel) the next tile's loads are issued
//    right after the LDS write of the current one, so they are in flight
//    while it is read back and stored;
//  * global writes: 32 lanes store a 512-byte row segment of B as float4,
//    non-temporal (the output is streamed, never re-read here).  Cold (working
//    set rotated past the 256 MB memory-side cache) the full-tile kernel moves
//    ~5.8 TB/s on MI355X (72 % of 8 TB/s); a plain non-temporal copy of the
//    same bytes moves 6.4 TB/s;
//  * tiles that run past the edge, rows or cols not multiples of 4, or
//    pointers that are not 16-byte aligned take a guarded scalar path, so any
//    shape (including empty and ragged ones) is handled.
#include "common.h"

#include <algorithm>

namespace mb {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int TILE = 128;
constexpr int THREADS = 256;
constexpr int LPR = TILE / 4;             // lanes per 512-byte row segment
constexpr int RPI = THREADS / LPR;        // rows per load instruction (workgroup-wide)
constexpr int NI = TILE / RPI;            // float4 per lane per tile

__global__ __launch_bounds__(THREADS)
void transpose_2d_f32_kernel(const float* __restrict__ a, float* __restrict__ b,
                             uint32_t rows, uint32_t cols, uint32_t tiles_r, uint32_t ntiles,
                             uint32_t vec_ok) {
    __shared__ float tile[TILE][TILE + 1];

    const uint32_t tx = threadIdx.x % LPR;   // float4 column within the tile
    const uint32_t ty = threadIdx.x / LPR;   // 0 .. RPI-1
    auto origin = [&](uint32_t t, uint32_t* r0, uint32_t* c0) {
        *r0 = (t % tiles_r) * TILE;
        *c0 = (t / tiles_r) * TILE;
    };
    auto full = [&](uint32_t t) {
        uint32_t r0, c0;
        origin(t, &r0, &c0);
        return vec_ok && r0 + TILE <= rows && c0 + TILE <= cols;
    };
    f32x4 v[NI];
    auto load = [&](uint32_t t) {
        uint32_t r0, c0;
        origin(t, &r0, &c0);
#pragma unroll
        for (int i = 0; i < NI; ++i)
            v[i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(
                a + (size_t)(r0 + ty + RPI * i) * cols + c0 + 4 * tx));
    };

    uint32_t t = blockIdx.x;
    if (t < ntiles && full(t)) load(t);
    for (; t < ntiles; t += gridDim.x) {
        uint32_t r0, c0;
        origin(t, &r0, &c0);
        const uint32_t tn = t + gridDim.x;
        __syncthreads();   // the previous tile's LDS reads are done
        if (full(t)) {
#pragma unroll
            for (int i = 0; i < NI; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) tile[ty + RPI * i][4 * tx + e] = v[i][e];
            __syncthreads();
            if (tn < ntiles && full(tn)) load(tn);
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const uint32_t j = ty + RPI * i;          // row of B inside the tile
                const f32x4 o = {tile[4 * tx + 0][j], tile[4 * tx + 1][j], tile[4 * tx + 2][j],
                                 tile[4 * tx + 3][j]};
                __builtin_nontemporal_store(
                    o, reinterpret_cast<f32x4*>(b + (size_t)(c0 + j) * rows + r0 + 4 * tx));
            }
        } else {
            // Edge tile: one element per lane per step, guarded.
            const uint32_t lx = threadIdx.x % TILE;
            const uint32_t ly = threadIdx.x / TILE;   // 0..1
            for (uint32_t i = ly; i < TILE; i += THREADS / TILE) {
                const uint32_t r = r0 + i, c = c0 + lx;
                if (r < rows && c < cols) tile[i][lx] = a[(size_t)r * cols + c];
            }
            __syncthreads();
            if (tn < ntiles && full(tn)) load(tn);
            for (uint32_t j = ly; j < TILE; j += THREADS / TILE) {
                const uint32_t c = c0 + j, r = r0 + lx;   // B[c][r] = A[r][c]
                if (c < cols && r < rows) b[(size_t)c * rows + r] = tile[lx][j];
            }
        }
    }
}

// Every tile full (rows, cols multiples of TILE; 16-byte aligned): three
// register tile buffers per thread, the loads of the next two tiles in flight
// while one tile goes through LDS and out.
__global__ __launch_bounds__(THREADS, 2)
void transpose_full_kernel(const float* __restrict__ a, float* __restrict__ b, uint32_t rows,
                           uint32_t cols, uint32_t tiles_r, uint32_t ntiles) {
    __shared__ float tile[TILE][TILE + 1];
    const uint32_t tx = threadIdx.x % LPR, ty = threadIdx.x / LPR;
    const uint32_t G = gridDim.x, t0 = blockIdx.x;
    const uint32_t nk = t0 < ntiles ? (ntiles - t0 + G - 1) / G : 0;   // tiles of this workgroup
    f32x4 v0[NI], v1[NI], v2[NI];
    auto load = [&](f32x4 (&v)[NI], uint32_t k) {
        const uint32_t t = t0 + k * G;
        const uint32_t r0 = (t % tiles_r) * TILE, c0 = (t / tiles_r) * TILE;
#pragma unroll
        for (int i = 0; i < NI; ++i)
            v[i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(
                a + (size_t)(r0 + ty + RPI * i) * cols + c0 + 4 * tx));
    };
    auto process = [&](f32x4 (&v)[NI], uint32_t k) {
        const uint32_t t = t0 + k * G;
        const uint32_t r0 = (t % tiles_r) * TILE, c0 = (t / tiles_r) * TILE;
        __syncthreads();   // the previous tile's LDS reads are done
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) tile[ty + RPI * i][4 * tx + e] = v[i][e];
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const uint32_t j = ty + RPI * i;   // row of B inside the tile
            const f32x4 o = {tile[4 * tx + 0][j], tile[4 * tx + 1][j], tile[4 * tx + 2][j],
                             tile[4 * tx + 3][j]};
            __builtin_nontemporal_store(
                o, reinterpret_cast<f32x4*>(b + (size_t)(c0 + j) * rows + r0 + 4 * tx));
        }
    };
    if (nk > 0) load(v0, 0);
    if (nk > 1) load(v1, 1);
    if (nk > 2) load(v2, 2);
    for (uint32_t k = 0; k < nk; k += 3) {
        process(v0, k);
        if (k + 3 < nk) load(v0, k + 3);
        if (k + 1 < nk) {
            process(v1, k + 1);
            if (k + 4 < nk) load(v1, k + 4);
        }
        if (k + 2 < nk) {
            process(v2, k + 2);
            if (k + 5 < nk) load(v2, k + 5);
        }
    }
}

int launch_transpose(const float* a, float* b, uint32_t rows, uint32_t cols, hipStream_t s) {
    if (rows == 0 || cols == 0) return MB_OK;
    if (!a || !b) return fail(MB_E_ARG, "transpose_2d_f32: null pointer");
    const uint32_t tiles_r = cdiv(rows, TILE), tiles_c = cdiv(cols, TILE);
    const uint64_t ntiles = (uint64_t)tiles_r * tiles_c;
    if (ntiles > 0x7fffffffull) return fail(MB_E_ARG, "transpose_2d_f32: shape too large");
    const uint32_t vec_ok = ((rows | cols) & 3) == 0 && (((uintptr_t)a | (uintptr_t)b) & 15) == 0;
    const uint32_t grid = (uint32_t)std::min<uint64_t>(ntiles, std::max(device_cu_count(), 1u));
    if (vec_ok && rows % TILE == 0 && cols % TILE == 0) {
        hipLaunchKernelGGL(transpose_full_kernel, dim3(grid), dim3(THREADS), 0, s, a, b, rows, cols,
                           tiles_r, (uint32_t)ntiles);
        MB_LAUNCH_CHECK("transpose_2d_f32");
        return MB_OK;
    }
    hipLaunchKernelGGL(transpose_2d_f32_kernel, dim3(grid), dim3(THREADS), 0, s, a, b, rows,
                       cols, tiles_r, (uint32_t)ntiles, vec_ok);
    MB_LAUNCH_CHECK("transpose_2d_f32");
    return MB_OK;
}

// Registry launcher: A@0 (input f32), B@1 (output f32), rows@2, cols@3.
int run_transpose(const Bindings& bs, hipStream_t s, PartMarks*) {
    uint32_t rows, cols;
    int rc;
    if ((rc = bs.u32(2, &rows, "rows")) || (rc = bs.u32(3, &cols, "cols"))) return rc;
    const uint64_t nbytes = (uint64_t)rows * cols * 4;
    void *a, *b;
    if ((rc = bs.buffer(0, MB_DTYPE_F32, nbytes, false, &a, "A")) ||
        (rc = bs.buffer(1, MB_DTYPE_F32, nbytes, true, &b, "B")))
        return rc;
    return launch_transpose((const float*)a, (float*)b, rows, cols, s);
}

}  // namespace

void register_transpose() {
    register_kernel({"transpose_2d_f32", run_transpose,
                     reinterpret_cast<const void*>(&transpose_full_kernel), 1});
}

}  // namespace mb

extern "C" int mb_launch_transpose_2d_f32(const float* a, float* b, uint32_t rows,
                                          uint32_t cols, void* stream) {
    mb::clear_error();
    if (!mb::initialized()) return mb::fail(MB_E_STATE, "mb_init() has not been called");
    return mb::launch_transpose(a, b, rows, cols, mb::stream_or_default(stream));
}
