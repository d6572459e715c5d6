// fp32 transformer sub-ops at the reference's own shapes: row RMSNorm (with an
// optional residual add), RoPE, matrix-vector product, and prefill GQA
// attention, plus the two blocks built from them and the fp32 GEMM family
// (gemm_f32.hip): llama_attention and the prefill llama_decoder_layer.
//
// Specs (reference files; registry bindings in each launcher's comment):
//   rms_norm             mlx/kernels/common/rms_norm.py:7-11 (nn.RMSNorm, unit
//                        gain at init), registry common/registry.py:135-136
//   fused_add_rms_norm   standard/fused_add_rms_norm.py:7-12, registry
//                        standard/registry.py:280-292
//   rope_embedding       standard/rope_embedding.py:15-32, registry
//                        standard/registry.py:103-117
//   matvec               common/matvec.py:9-10, registry common/registry.py:151-162
//   llama_attention      standard/llama_attention.py:18-58, registry
//                        standard/registry.py:398-413
//   llama_decoder_layer  full/llama_decoder_layer.py:17-64, registry
//                        full/registry.py:87-104
//
// gfx950 design.  These shapes are small (the reference runs each in one
// Metal threadgroup), so each op is one or a few short launches:
//  * row ops: one 64-lane wave per row, float4 loads, shuffle reductions;
//  * RoPE angles are formed in fp64 (pos * base^(-2i/D) reaches 127 rad at the
//    reference shape, where an fp32 angle would be off by ~1e-5 rad, i.e. at
//    the registry's atol);
//  * attention: one workgroup per (head, 64 queries); four lanes own a query
//    (a quarter of the head dims each), keys and values (K rotated) stream
//    through LDS 64 at a time, with an online softmax (no mask: the reference
//    attends to every position, standard/llama_attention.py:48-50);
//  * the GEMMs fuse what the blocks put around them: the RMSNorm row scale
//    (from the A operand's own loads), the residual add and SwiGLU.
#include "common.h"

#include <math.h>

namespace mb {
namespace {

constexpr float NEG_BIG = -1.0e30f;   // "no key yet": finite, so max/exp never see inf - inf

// ---- row RMSNorm ---------------------------------------------------------------------------

// y[r] = v * rsqrt(mean(v^2) + eps), v = x[r] (+ res[r]); one wave per row.
template <bool ADD, bool VEC>
__global__ __launch_bounds__(256)
void rms_norm_rows_kernel(const float* __restrict__ x, const float* __restrict__ res,
                          float* __restrict__ y, uint32_t rows, uint32_t cols, float eps) {
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63;
    if (row >= rows) return;   // whole waves only; no barriers in this kernel
    const float* xr = x + (size_t)row * cols;
    const float* rr = ADD ? res + (size_t)row * cols : nullptr;
    float* yr = y + (size_t)row * cols;
    float ss = 0.f;
    if (VEC) {
        for (uint32_t c = 4 * lane; c < cols; c += 256) {
            float4 v = *reinterpret_cast<const float4*>(xr + c);
            if (ADD) {
                const float4 r = *reinterpret_cast<const float4*>(rr + c);
                v.x += r.x; v.y += r.y; v.z += r.z; v.w += r.w;
            }
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
    } else {
        for (uint32_t c = lane; c < cols; c += 64) {
            const float v = xr[c] + (ADD ? rr[c] : 0.f);
            ss += v * v;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    const float scale = rsqrtf(ss / (float)cols + eps);
    if (VEC) {
        for (uint32_t c = 4 * lane; c < cols; c += 256) {
            float4 v = *reinterpret_cast<const float4*>(xr + c);
            if (ADD) {
                const float4 r = *reinterpret_cast<const float4*>(rr + c);
                v.x += r.x; v.y += r.y; v.z += r.z; v.w += r.w;
            }
            *reinterpret_cast<float4*>(yr + c) =
                make_float4(v.x * scale, v.y * scale, v.z * scale, v.w * scale);
        }
    } else {
        for (uint32_t c = lane; c < cols; c += 64) yr[c] = (xr[c] + (ADD ? rr[c] : 0.f)) * scale;
    }
}

template <bool ADD>
int launch_rms_norm_rows(const float* x, const float* res, float* y, uint32_t rows,
                         uint32_t cols, float eps, hipStream_t s) {
    if (rows == 0 || cols == 0) return MB_OK;
    const bool vec = cols % 4 == 0 &&
                     (((uintptr_t)x | (uintptr_t)res | (uintptr_t)y) & 15) == 0;
    const dim3 grid(cdiv(rows, 4)), block(256);
    if (vec) hipLaunchKernelGGL((rms_norm_rows_kernel<ADD, true>), grid, block, 0, s, x, res, y, rows, cols, eps);
    else hipLaunchKernelGGL((rms_norm_rows_kernel<ADD, false>), grid, block, 0, s, x, res, y, rows, cols, eps);
    MB_LAUNCH_CHECK("rms_norm");
    return MB_OK;
}

// ---- RoPE over rows (position = row index) --------------------------------------------------

// out[p][2i], out[p][2i+1] = rotation of the pair by p * base^(-2i/D).
__global__ __launch_bounds__(256)
void rope_rows_kernel(const float* __restrict__ x, float* __restrict__ y, uint32_t S, uint32_t D,
                      double base) {
    const uint32_t half = D / 2;
    const uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (uint64_t)S * half) return;
    const uint32_t p = (uint32_t)(idx / half), i = (uint32_t)(idx % half);
    const double omega = pow(base, -2.0 * (double)i / (double)D);
    double sn, cs;
    sincos((double)p * omega, &sn, &cs);
    const float2 v = *reinterpret_cast<const float2*>(x + (size_t)p * D + 2 * i);
    *reinterpret_cast<float2*>(y + (size_t)p * D + 2 * i) =
        make_float2((float)(v.x * cs - v.y * sn), (float)(v.x * sn + v.y * cs));
}

// ---- matrix-vector product -------------------------------------------------------------------

// y[m] = sum_k A[m][k] x[k]; one wave per row.
template <bool VEC>
__global__ __launch_bounds__(256)
void matvec_kernel(const float* __restrict__ A, const float* __restrict__ x, float* __restrict__ y,
                   uint32_t M, uint32_t K) {
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63;
    if (row >= M) return;   // whole waves only; no barriers in this kernel
    const float* ar = A + (size_t)row * K;
    float acc = 0.f;
    if (VEC) {
        for (uint32_t c = 4 * lane; c < K; c += 256) {
            const float4 a = *reinterpret_cast<const float4*>(ar + c);
            const float4 v = *reinterpret_cast<const float4*>(x + c);
            acc += a.x * v.x + a.y * v.y + a.z * v.z + a.w * v.w;
        }
    } else {
        for (uint32_t c = lane; c < K; c += 64) acc += ar[c] * x[c];
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
    if (lane == 0) y[row] = acc;
}

// ---- prefill GQA attention -------------------------------------------------------------------

// T is the arithmetic of the attention logits: q, k, the rotation, q.k and
// the online softmax (float, or double for the decoder layer, see
// run_llama_decoder_layer); v and the output stay fp32.
template <typename T>
struct AttnPrefillArgs {
    const T* qkv;       // [S][ldq]: q at column h*Dh, k at D + kvh*Dh, v at D + Hkv*Dh + kvh*Dh
    float* out;         // [S][ldo]: head h at column h*Dh
    uint32_t S, D, H, Hkv, ldq, ldo;
    float base, scale;  // RoPE base; 1 / sqrt(Dh)
};

constexpr int QW = 16;   // queries per workgroup
constexpr int KC = 64;   // keys per LDS chunk

template <typename T> __device__ __forceinline__ T exp_t(T v);
template <> __device__ __forceinline__ float exp_t<float>(float v) { return expf(v); }
template <> __device__ __forceinline__ double exp_t<double>(double v) { return exp(v); }

// Workgroup (head h, 16 queries); the 16 lanes 16 qq .. 16 qq + 15 of a wave
// own query qq of the block.  Per chunk of 64 keys: the keys are rotated
// into LDS (omega_j = base^(-2j/Dh) once per pair index, the angle pos *
// omega_j and its sine and cosine in fp64: an fp32 angle is off by ~pos *
// 6e-8 rad), lane kg of a query scores keys kg, kg + 16, kg + 32, kg + 48
// (a Dh-long dot product each), the query's 16 lanes fold the chunk's
// maximum and sum with shuffles (online softmax across chunks), write the
// probabilities to LDS and update their Dh / 16 output dims over the
// chunk's keys.  q and k are rotated by their positions (the row index) on
// interleaved pairs (2j, 2j+1).  (The first version gave a workgroup 64
// queries, four lanes per query and keys one at a time: at S = 64 that is
// one workgroup per head and 64 dependent steps, 21 us for llama_attention's
// registry shape.)
template <int DH, typename T>
__global__ __launch_bounds__(256)
void attention_prefill_kernel(AttnPrefillArgs<T> a) {
    constexpr int OD = DH / 16;   // output dims per lane
    __shared__ T qs[QW][DH + 1];
    __shared__ T ks[KC][DH + 1];
    __shared__ float vs[KC][DH];
    __shared__ T ps[QW][KC];
    __shared__ double omega[DH / 2];
    const uint32_t tid = threadIdx.x;
    const uint32_t h = blockIdx.x, kvh = h / (a.H / a.Hkv);
    const uint32_t q0 = blockIdx.y * QW;
    const uint32_t qq = tid >> 4, kg = tid & 15;   // query of the block, lane within the query
    const uint32_t kcol = a.D + kvh * DH, vcol = a.D + a.Hkv * DH + kvh * DH;

    if (tid < DH / 2) omega[tid] = pow((double)a.base, -2.0 * (double)tid / (double)DH);
    __syncthreads();
    for (uint32_t e = tid; e < QW * DH / 2; e += 256) {
        const uint32_t i = e / (DH / 2), pair = e % (DH / 2), pos = q0 + i;
        T x0 = 0, x1 = 0;
        if (pos < a.S) {
            const T* src = a.qkv + (size_t)pos * a.ldq + h * DH + 2 * pair;
            x0 = src[0]; x1 = src[1];
        }
        double sn, cs;
        sincos((double)pos * omega[pair], &sn, &cs);
        qs[i][2 * pair] = x0 * (T)cs - x1 * (T)sn;
        qs[i][2 * pair + 1] = x0 * (T)sn + x1 * (T)cs;
    }

    T m_run = (T)NEG_BIG, l_run = 0;
    T o[OD];
#pragma unroll
    for (int d = 0; d < OD; ++d) o[d] = 0;
    const uint32_t od = kg * OD;

    for (uint32_t kc = 0; kc < a.S; kc += KC) {
        __syncthreads();   // q is written; the previous chunk is no longer read
        for (uint32_t e = tid; e < KC * DH / 2; e += 256) {
            const uint32_t key = e / (DH / 2), pair = e % (DH / 2), kk = kc + key;
            T k0 = 0, k1 = 0, v0 = 0, v1 = 0;
            if (kk < a.S) {
                const T* kr = a.qkv + (size_t)kk * a.ldq + kcol + 2 * pair;
                const T* vr = a.qkv + (size_t)kk * a.ldq + vcol + 2 * pair;
                k0 = kr[0]; k1 = kr[1]; v0 = vr[0]; v1 = vr[1];
            }
            double sn, cs;
            sincos((double)kk * omega[pair], &sn, &cs);
            ks[key][2 * pair] = k0 * (T)cs - k1 * (T)sn;
            ks[key][2 * pair + 1] = k0 * (T)sn + k1 * (T)cs;
            vs[key][2 * pair] = (float)v0;
            vs[key][2 * pair + 1] = (float)v1;
        }
        __syncthreads();
        const uint32_t nk = min((uint32_t)KC, a.S - kc);
        T sc[4];
        T cmax = (T)NEG_BIG;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t key = kg + 16 * i;
            T dp[4] = {0, 0, 0, 0};   // four interleaved partial sums, added pairwise
#pragma unroll
            for (int d = 0; d < DH; ++d) dp[d & 3] += qs[qq][d] * ks[key][d];
            const T dot = (dp[0] + dp[1]) + (dp[2] + dp[3]);
            sc[i] = key < nk ? dot * (T)a.scale : (T)NEG_BIG;
            cmax = cmax > sc[i] ? cmax : sc[i];
        }
#pragma unroll
        for (int o2 = 1; o2 < 16; o2 <<= 1) {
            const T other = __shfl_xor(cmax, o2);
            cmax = cmax > other ? cmax : other;
        }
        const T m_new = m_run > cmax ? m_run : cmax;
        const T alpha = exp_t<T>(m_run - m_new);
        T psum = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t key = kg + 16 * i;
            const T p = key < nk ? exp_t<T>(sc[i] - m_new) : (T)0;
            ps[qq][key] = p;
            psum += p;
        }
#pragma unroll
        for (int o2 = 1; o2 < 16; o2 <<= 1) psum += __shfl_xor(psum, o2);
        l_run = l_run * alpha + psum;
        m_run = m_new;
        __syncthreads();   // the query's probabilities (written by its 16 lanes)
#pragma unroll
        for (int d = 0; d < OD; ++d) o[d] *= alpha;
        for (uint32_t j = 0; j < nk; ++j) {
            const T p = ps[qq][j];
#pragma unroll
            for (int d = 0; d < OD; ++d) o[d] += p * (T)vs[j][od + d];
        }
    }
    if (q0 + qq < a.S) {
        const T inv = (T)1 / l_run;
#pragma unroll
        for (int d = 0; d < OD; d += 2)
            *reinterpret_cast<float2*>(a.out + (size_t)(q0 + qq) * a.ldo + h * DH + od + d) =
                make_float2((float)(o[d] * inv), (float)(o[d + 1] * inv));
    }
}

template <typename T>
int launch_attention_prefill(const AttnPrefillArgs<T>& a, uint32_t dh, hipStream_t s) {
    if (a.S == 0) return MB_OK;
    const dim3 grid(a.H, cdiv(a.S, QW)), block(256);
    switch (dh) {
        case 32: hipLaunchKernelGGL((attention_prefill_kernel<32, T>), grid, block, 0, s, a); break;
        case 64: hipLaunchKernelGGL((attention_prefill_kernel<64, T>), grid, block, 0, s, a); break;
        case 128: hipLaunchKernelGGL((attention_prefill_kernel<128, T>), grid, block, 0, s, a); break;
        default: return fail(MB_E_ARG, "attention: head dim %u not 32, 64 or 128", dh);
    }
    MB_LAUNCH_CHECK("attention prefill");
    return MB_OK;
}

// ---- fp64 RMSNorm GEMM (the decoder layer's q|k|v projection) -----------------------------

// C[S][N] = rmsnorm(A) B in fp64 from fp32 A [S][K] and B [K][N]: each
// workgroup computes a (16 TR) x (16 TC) tile, thread (ty, tx) the TR x TC
// outputs of rows TR ty .. TR ty + TR - 1 and columns tx + 16 j; A and B go
// through LDS 32 k at a time, widened to fp64 on the way in, and the next
// chunk's global loads are in flight while the current one is multiplied.
// The row scale rsqrt(mean(a^2) + eps) is accumulated from the same A chunks.
// (With 64 x 64 tiles and each chunk loaded only after the previous one was
// multiplied, the decoder layer's 64 x 256 x 128 projection ran on 4
// workgroups and took 23.8 us, four load round trips in a row.)
constexpr int GK = 32;

template <int TR, int TC>   // rows and columns per thread: a (16 TR) x (16 TC) tile
__global__ __launch_bounds__(256)
void rms_gemm_f64_kernel(const float* __restrict__ A, const float* __restrict__ B,
                         double* __restrict__ C, uint32_t S, uint32_t N, uint32_t K, float eps) {
    constexpr int GR = 16 * TR, GC = 16 * TC;
    constexpr int RT = 256 / GR;      // threads per row for the sums of squares
    __shared__ double as[GR][GK + 1];
    __shared__ double bs[GK][GC + 1];
    __shared__ double rs[GR];
    const uint32_t tid = threadIdx.x, tx = tid % 16, ty = tid / 16;
    const uint32_t row0 = blockIdx.y * GR, col0 = blockIdx.x * GC;
    constexpr int LA = GR * GK / 256, LB = GK * GC / 256;   // elements per thread per chunk
    float ra[LA], rb[LB];
    auto load = [&](uint32_t k0) {
#pragma unroll
        for (int i = 0; i < LA; ++i) {
            const uint32_t e = tid + 256 * i, r = e / GK, c = e % GK;
            const uint32_t gr = row0 + r, gk = k0 + c;
            ra[i] = (gr < S && gk < K) ? A[(size_t)gr * K + gk] : 0.f;
        }
#pragma unroll
        for (int i = 0; i < LB; ++i) {
            const uint32_t e = tid + 256 * i, kr = e / GC, nc = e % GC;
            rb[i] = (k0 + kr < K && col0 + nc < N) ? B[(size_t)(k0 + kr) * N + col0 + nc] : 0.f;
        }
    };
    double acc[TR][TC] = {};
    double ss = 0;   // sum of squares of row tid / RT, k part (tid % RT) of each chunk
    load(0);
    for (uint32_t k0 = 0; k0 < K; k0 += GK) {
        __syncthreads();   // the previous chunk is no longer read
#pragma unroll
        for (int i = 0; i < LA; ++i) {
            const uint32_t e = tid + 256 * i;
            as[e / GK][e % GK] = (double)ra[i];
        }
#pragma unroll
        for (int i = 0; i < LB; ++i) {
            const uint32_t e = tid + 256 * i;
            bs[e / GC][e % GC] = (double)rb[i];
        }
        __syncthreads();
        if (k0 + GK < K) load(k0 + GK);
#pragma unroll
        for (int c = 0; c < GK / RT; ++c) {
            const double v = as[tid / RT][(tid % RT) * (GK / RT) + c];
            ss += v * v;
        }
#pragma unroll 4
        for (int kk = 0; kk < GK; ++kk) {
            double av[TR], bv[TC];
#pragma unroll
            for (int i = 0; i < TR; ++i) av[i] = as[TR * ty + i][kk];
#pragma unroll
            for (int j = 0; j < TC; ++j) bv[j] = bs[kk][tx + 16 * j];
#pragma unroll
            for (int i = 0; i < TR; ++i)
#pragma unroll
                for (int j = 0; j < TC; ++j) acc[i][j] += av[i] * bv[j];
        }
    }
#pragma unroll
    for (int o2 = 1; o2 < RT; o2 <<= 1) ss += __shfl_xor(ss, o2);
    if (tid % RT == 0) rs[tid / RT] = 1.0 / sqrt(ss / (double)K + (double)eps);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TR; ++i) {
        const uint32_t r = row0 + TR * ty + i;
        if (r >= S) continue;
#pragma unroll
        for (int j = 0; j < TC; ++j) {
            const uint32_t c = col0 + tx + 16 * j;
            if (c < N) C[(size_t)r * N + c] = acc[i][j] * rs[TR * ty + i];
        }
    }
}

int launch_rms_gemm_f64(const float* a, const float* b, double* c, uint32_t S, uint32_t N,
                        uint32_t K, float eps, hipStream_t s) {
    if (S == 0 || N == 0) return MB_OK;
    if (K == 0) return fail(MB_E_ARG, "rms gemm: K must be positive");
    // 16 x 32 tiles: 32 workgroups at the registry's 64 x 256 (34 us for the
    // layer, against 35-36 us with 32 x 32 or 32 x 64 tiles and 16 x 64)
    hipLaunchKernelGGL((rms_gemm_f64_kernel<1, 2>), dim3(cdiv(N, 32), cdiv(S, 16)), dim3(256), 0,
                       s, a, b, c, S, N, K, eps);
    MB_LAUNCH_CHECK("rms_gemm_f64");
    return MB_OK;
}

// Shape checks shared by llama_attention and llama_decoder_layer.
int check_heads(uint32_t S, uint32_t D, uint32_t H, uint32_t HKV, uint32_t* dh) {
    if (S == 0 || D == 0 || H == 0 || HKV == 0 || D % H || H % HKV)
        return fail(MB_E_ARG, "attention: S %u, D %u, H %u, H_kv %u: need D %% H == 0 and "
                    "H %% H_kv == 0", S, D, H, HKV);
    *dh = D / H;
    if (*dh != 32 && *dh != 64 && *dh != 128)
        return fail(MB_E_ARG, "attention: head dim %u not 32, 64 or 128", *dh);
    if (S > 65535u * QW) return fail(MB_E_ARG, "attention: S %u too large", S);
    return MB_OK;
}

// ---- registry launchers ----------------------------------------------------------------------

// rms_norm: x@0 [rows][cols], y@1, cols@2, eps@3 (rows = x's size / cols).
int run_rms_norm(const Bindings& bs, hipStream_t s, PartMarks*) {
    uint32_t cols;
    float eps;
    int rc;
    if ((rc = bs.u32(2, &cols, "cols")) || (rc = bs.f32(3, &eps, "eps"))) return rc;
    if (cols == 0) return fail(MB_E_ARG, "rms_norm: cols must be positive");
    const uint64_t rows = bs.nbytes(0) / ((uint64_t)cols * 4);
    void *x, *y;
    if ((rc = bs.buffer(0, MB_DTYPE_F32, rows * cols * 4, false, &x, "x")) ||
        (rc = bs.buffer(1, MB_DTYPE_F32, rows * cols * 4, true, &y, "y")))
        return rc;
    return launch_rms_norm_rows<false>((const float*)x, nullptr, (float*)y, (uint32_t)rows, cols,
                                       eps, s);
}

// fused_add_rms_norm: x@0, residual@1 [rows][cols], y@2, cols@3, eps@4.
int run_fused_add_rms_norm(const Bindings& bs, hipStream_t s, PartMarks*) {
    uint32_t cols;
    float eps;
    int rc;
    if ((rc = bs.u32(3, &cols, "cols")) || (rc = bs.f32(4, &eps, "eps"))) return rc;
    if (cols == 0) return fail(MB_E_ARG, "fused_add_rms_norm: cols must be positive");
    const uint64_t rows = bs.nbytes(0) / ((uint64_t)cols * 4);
    void *x, *r, *y;
    if ((rc = bs.buffer(0, MB_DTYPE_F32, rows * cols * 4, false, &x, "x")) ||
        (rc = bs.buffer(1, MB_DTYPE_F32, rows * cols * 4, false, &r, "residual")) ||
        (rc = bs.buffer(2, MB_DTYPE_F32, rows * cols * 4, true, &y, "y")))
        return rc;
    return launch_rms_norm_rows<true>((const float*)x, (const float*)r, (float*)y,
                                      (uint32_t)rows, cols, eps, s);
}

// rope_embedding: x@0 [S][D], y@1, S@2, D@3, base@4.
int run_rope(const Bindings& bs, hipStream_t s, PartMarks*) {
    uint32_t S, D;
    float base;
    int rc;
    if ((rc = bs.u32(2, &S, "S")) || (rc = bs.u32(3, &D, "D")) || (rc = bs.f32(4, &base, "base")))
        return rc;
    if (D % 2) return fail(MB_E_ARG, "rope_embedding: D %u must be even", D);
    if (!(base > 0.f)) return fail(MB_E_ARG, "rope_embedding: base must be > 0");
    void *x, *y;
    if ((rc = bs.buffer(0, MB_DTYPE_F32, (uint64_t)S * D * 4, false, &x, "x")) ||
        (rc = bs.buffer(1, MB_DTYPE_F32, (uint64_t)S * D * 4, true, &y, "y")))
        return rc;
    const uint64_t pairs = (uint64_t)S * (D / 2);
    if (pairs == 0) return MB_OK;
    if (pairs > 0xffffffffull) return fail(MB_E_ARG, "rope_embedding: shape too large");
    if (((uintptr_t)x | (uintptr_t)y) & 7) return fail(MB_E_ARG, "rope_embedding: unaligned buffers");
    hipLaunchKernelGGL(rope_rows_kernel, dim3((uint32_t)((pairs + 255) / 256)), dim3(256), 0, s,
                       (const float*)x, (float*)y, S, D, (double)base);
    MB_LAUNCH_CHECK("rope_embedding");
    return MB_OK;
}

// matvec: A@0 [M][K], x@1 [K], y@2 [M], K@3 (M = y's size).
int run_matvec(const Bindings& bs, hipStream_t s, PartMarks*) {
    uint32_t K;
    int rc;
    if ((rc = bs.u32(3, &K, "K"))) return rc;
    const uint64_t M = bs.nbytes(2) / 4;
    void *A, *x, *y;
    if ((rc = bs.buffer(0, MB_DTYPE_F32, M * K * 4, false, &A, "A")) ||
        (rc = bs.buffer(1, MB_DTYPE_F32, (uint64_t)K * 4, false, &x, "x")) ||
        (rc = bs.buffer(2, MB_DTYPE_F32, M * 4, true, &y, "y")))
        return rc;
    if (M == 0) return MB_OK;
    if (M > 0x7ffffffcull) return fail(MB_E_ARG, "matvec: M too large");
    const bool vec = K % 4 == 0 && (((uintptr_t)A | (uintptr_t)x) & 15) == 0;
    const dim3 grid(cdiv((uint32_t)M, 4)), block(256);
    if (vec) hipLaunchKernelGGL(matvec_kernel<true>, grid, block, 0, s, (const float*)A, (const float*)x, (float*)y, (uint32_t)M, K);
    else hipLaunchKernelGGL(matvec_kernel<false>, grid, block, 0, s, (const float*)A, (const float*)x, (float*)y, (uint32_t)M, K);
    MB_LAUNCH_CHECK("matvec");
    return MB_OK;
}

// llama_attention: x@0 [S][D], W_qkv@1 [D][D + 2 Hkv Dh], W_o@2 [D][D], y@3
// [S][D], S@4, D@5, H@6, H_kv@7, base@8.  y = attention(x W_qkv) W_o (no
// norm, no residual: standard/llama_attention.py:30-52).
int run_llama_attention(const Bindings& bs, hipStream_t s, PartMarks*) {
    uint32_t S, D, H, HKV, dh;
    float base;
    int rc;
    if ((rc = bs.u32(4, &S, "S")) || (rc = bs.u32(5, &D, "D")) || (rc = bs.u32(6, &H, "H")) ||
        (rc = bs.u32(7, &HKV, "H_kv")) || (rc = bs.f32(8, &base, "base")))
        return rc;
    if ((rc = check_heads(S, D, H, HKV, &dh))) return rc;
    const uint32_t nqkv = D + 2 * HKV * dh;
    void *x, *wqkv, *wo, *y;
    if ((rc = bs.buffer(0, MB_DTYPE_F32, (uint64_t)S * D * 4, false, &x, "x")) ||
        (rc = bs.buffer(1, MB_DTYPE_F32, (uint64_t)D * nqkv * 4, false, &wqkv, "W_qkv")) ||
        (rc = bs.buffer(2, MB_DTYPE_F32, (uint64_t)D * D * 4, false, &wo, "W_o")) ||
        (rc = bs.buffer(3, MB_DTYPE_F32, (uint64_t)S * D * 4, true, &y, "y")))
        return rc;
    const size_t qkv_bytes = ((size_t)S * nqkv * 4 + 255) & ~(size_t)255;
    uint8_t* ws = static_cast<uint8_t*>(library_workspace(qkv_bytes + (size_t)S * D * 4));
    if (!ws) return MB_E_HIP;
    float* qkv = reinterpret_cast<float*>(ws);
    float* attn = reinterpret_cast<float*>(ws + qkv_bytes);
    if ((rc = launch_gemm_f32_ex(gemm_f32_args((const float*)x, (const float*)wqkv, qkv, S, nqkv, D),
                                 GEMM_F32_PLAIN, 1, s)))
        return rc;
    AttnPrefillArgs<float> a{qkv, attn, S, D, H, HKV, nqkv, D, base, 1.0f / sqrtf((float)dh)};
    if ((rc = launch_attention_prefill(a, dh, s))) return rc;
    return launch_gemm_f32_ex(gemm_f32_args(attn, (const float*)wo, (float*)y, S, D, D),
                              GEMM_F32_PLAIN, 1, s);
}

// llama_decoder_layer (prefill): x@0 [S][D], W_qkv@1, W_o@2, W_gu@3 [D][2 FF]
// ([gate | up]), W_down@4 [FF][D], y@5 [S][D], S@6, D@7, H@8, H_kv@9, FF@10,
// base@11, eps@12.  Five launches:
//   qkv  = rmsnorm(x) W_qkv                    (fp64, RMS row scale in the GEMM)
//   attn = attention(RoPE(q), RoPE(k), v)      (fp64 logits and softmax)
// The attention logits are the ill-conditioned part of this entry: with the
// reference's normal(0, 1) weights q.k / sqrt(Dh) reaches the hundreds, so
// fp32 rounding of q, k and the dot products moves the softmax weights of
// near-tied keys, and the FFN amplifies it; an all-fp32 evaluation of the
// layer lands ~0.15 from float64 on outputs of up to ~6000, one with fp64 q|k|v
// and logits ~0.004.  At S = 64, D = 128 the fp64 work is a few hundred
// thousand multiply-adds.
//   x1   = x + attn W_o                        (residual in the epilogue)
//   act  = silu(rmsnorm(x1) W_gate) * (rmsnorm(x1) W_up)
//   y    = x1 + act W_down
int run_llama_decoder_layer(const Bindings& bs, hipStream_t s, PartMarks* pm) {
    uint32_t S, D, H, HKV, FF, dh;
    float base, eps;
    int rc;
    if ((rc = bs.u32(6, &S, "S")) || (rc = bs.u32(7, &D, "D")) || (rc = bs.u32(8, &H, "H")) ||
        (rc = bs.u32(9, &HKV, "H_kv")) || (rc = bs.u32(10, &FF, "FF")) ||
        (rc = bs.f32(11, &base, "base")) || (rc = bs.f32(12, &eps, "eps")))
        return rc;
    if ((rc = check_heads(S, D, H, HKV, &dh))) return rc;
    if (FF == 0) return fail(MB_E_ARG, "llama_decoder_layer: FF must be positive");
    const uint32_t nqkv = D + 2 * HKV * dh;
    void *x, *wqkv, *wo, *wgu, *wdown, *y;
    if ((rc = bs.buffer(0, MB_DTYPE_F32, (uint64_t)S * D * 4, false, &x, "x")) ||
        (rc = bs.buffer(1, MB_DTYPE_F32, (uint64_t)D * nqkv * 4, false, &wqkv, "W_qkv")) ||
        (rc = bs.buffer(2, MB_DTYPE_F32, (uint64_t)D * D * 4, false, &wo, "W_o")) ||
        (rc = bs.buffer(3, MB_DTYPE_F32, (uint64_t)D * 2 * FF * 4, false, &wgu, "W_gu")) ||
        (rc = bs.buffer(4, MB_DTYPE_F32, (uint64_t)FF * D * 4, false, &wdown, "W_down")) ||
        (rc = bs.buffer(5, MB_DTYPE_F32, (uint64_t)S * D * 4, true, &y, "y")))
        return rc;
    auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
    const size_t o_qkv = 0, o_attn = al((size_t)S * nqkv * 8),
                 o_x1 = o_attn + al((size_t)S * D * 4), o_act = o_x1 + al((size_t)S * D * 4),
                 total = o_act + al((size_t)S * FF * 4);
    uint8_t* ws = static_cast<uint8_t*>(library_workspace(total));
    if (!ws) return MB_E_HIP;
    double* qkv = reinterpret_cast<double*>(ws + o_qkv);
    float* attn = reinterpret_cast<float*>(ws + o_attn);
    float* x1 = reinterpret_cast<float*>(ws + o_x1);
    float* act = reinterpret_cast<float*>(ws + o_act);
    auto mark = [&](const char* n) { if (pm) pm->mark(s, n); };

    mark("qkv_rmsnorm");
    if ((rc = launch_rms_gemm_f64((const float*)x, (const float*)wqkv, qkv, S, nqkv, D, eps, s)))
        return rc;
    mark("attention");
    AttnPrefillArgs<double> a{qkv, attn, S, D, H, HKV, nqkv, D, base, 1.0f / sqrtf((float)dh)};
    if ((rc = launch_attention_prefill(a, dh, s))) return rc;
    mark("wo_residual");
    GemmF32Args g = gemm_f32_args(attn, (const float*)wo, x1, S, D, D);
    g.r = (const float*)x;
    if ((rc = launch_gemm_f32_ex(g, GEMM_F32_RESID, 1, s))) return rc;
    mark("gate_up_swiglu");
    g = gemm_f32_args(x1, (const float*)wgu, act, S, FF, D);
    g.b2 = (const float*)wgu + FF;
    g.ldb = 2 * FF;
    g.eps = eps;
    if ((rc = launch_gemm_f32_ex(g, GEMM_F32_RMS_SWIGLU, 1, s))) return rc;
    mark("down_residual");
    g = gemm_f32_args(act, (const float*)wdown, (float*)y, S, D, FF);
    g.r = x1;
    return launch_gemm_f32_ex(g, GEMM_F32_RESID, 1, s);
}

}  // namespace

void register_transformer_f32() {
    register_kernel({"rms_norm_f32", run_rms_norm,
                     reinterpret_cast<const void*>(&rms_norm_rows_kernel<false, true>), 1});
    register_kernel({"fused_add_rms_norm_f32", run_fused_add_rms_norm,
                     reinterpret_cast<const void*>(&rms_norm_rows_kernel<true, true>), 1});
    register_kernel({"rope_embedding_f32", run_rope,
                     reinterpret_cast<const void*>(&rope_rows_kernel), 1});
    register_kernel({"matvec_f32", run_matvec,
                     reinterpret_cast<const void*>(&matvec_kernel<true>), 1});
    register_kernel({"llama_attention_f32", run_llama_attention,
                     reinterpret_cast<const void*>(&attention_prefill_kernel<32, float>), 1});
    register_kernel({"llama_decoder_layer_f32", run_llama_decoder_layer,
                     reinterpret_cast<const void*>(&attention_prefill_kernel<32, double>), 5});
}

}  // namespace mb
