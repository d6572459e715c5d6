"""Kernel registry (common set): name -> dispatch metadata, one entry per kernel.

Same layout and keys as the reference's registry (reference
mlx/kernels/common/registry.py:1-59): `metal_function` names the kernel in the
native library (libmbhip.so here), inputs sit at `input_bindings`, the single
output at binding len(input_shapes), then the scalars.  `grid` and
`threadgroup` are advisory on gfx950: each HIP kernel derives its launch from
the scalars.

Optional keys added on top of the reference's (all backward compatible; a
reference-style entry without them means f32 normal(0,1) inputs):
  input_dtypes   per-input dtype tag, "f32" or "bf16"
  input_init     per-input initialiser: ("normal", mean, std),
                 ("uniform", lo, hi) or ("kaiming_normal", fan_in)
  output_dtype   dtype tag of the output (default "f32")
  compute_dtype  arithmetic the roofline is priced in ("f32" or "bf16")
  cpu_iters      iterations for the CPU baseline timing (heavy configs)

This file is exec'd on its own by tools and tests, so it imports nothing.
"""

REGISTRY = {}


def matmul(name, metal_func, M, N, K, BM=64, BN=64, TG=512, rtol=1e-3, atol=1e-3,
           dtype="f32", init=("normal", 0.0, 1.0), cpu_iters=None):
    """Matrix multiply C[M,N] = A[M,K] @ B[K,N] (reference registry.py:43-59)."""
    esize = 2 if dtype == "bf16" else 4
    REGISTRY[name] = dict(
        metal_function=metal_func,
        threadgroup=(TG, 1, 1),
        input_bindings=(0, 1),
        input_shapes=[(M, K), (K, N)],
        output_shape=(M, N),
        rtol=rtol, atol=atol,
        grid=((N // BN) * TG, M // BM, 1),
        scalars=[dict(binding=3, dtype="u32", value=M),
                 dict(binding=4, dtype="u32", value=N),
                 dict(binding=5, dtype="u32", value=K)],
        flops=2 * M * N * K,
        bytes=esize * (M * K + K * N + M * N),
        input_dtypes=[dtype, dtype],
        input_init=[init, init],
        output_dtype=dtype,
        compute_dtype=dtype,
    )
    if cpu_iters:
        REGISTRY[name]["cpu_iters"] = cpu_iters


# Square fp32 GEMM, 1024^3, inputs iid uniform[-1,1]; rtol = atol = 1e-4.
matmul("sqr_mm", "sqr_matmul_f32", 1024, 1024, 1024, rtol=1e-4, atol=1e-4,
       init=("uniform", -1.0, 1.0))

# The reference's rectangular GEMM shape (reference registry.py:130), same kernel.
matmul("rect_mm", "rect_matmul_f32", 1024, 2048, 4096)

# Large bf16 GEMM 8192^3, fp32 accumulate, bf16 output, inputs iid normal(0, 0.02).
# The gate compares against the fp32-accumulated product: rtol 1e-2, and atol
# 1e-4 for outputs near zero (their std is 0.02^2 * sqrt(8192) ~ 0.036).
matmul("large_mm", "large_matmul_bf16", 8192, 8192, 8192, BM=256, BN=256, TG=256,
       rtol=1e-2, atol=1e-4, dtype="bf16", init=("normal", 0.0, 0.02), cpu_iters=2)

# Transpose 8192 x 8192 fp32, iid normal(0,1): bit exact.
# (The reference's entry is 1024 x 2048 — see transpose_2d_ref below.)
REGISTRY["transpose_2d"] = dict(
    metal_function="transpose_2d_f32",
    threadgroup=(256, 1, 1),
    input_bindings=(0,),
    input_shapes=[(8192, 8192)],
    output_shape=(8192, 8192),
    rtol=0, atol=0,
    grid=(128 * 128 * 256, 1, 1),
    scalars=[dict(binding=2, dtype="u32", value=8192),
             dict(binding=3, dtype="u32", value=8192)],
    flops=0,
    bytes=8192 * 8192 * 4 * 2,
    cpu_iters=5,
)

# The reference's own transpose shape (reference registry.py:165-179).
REGISTRY["transpose_2d_ref"] = dict(
    metal_function="transpose_2d_f32",
    threadgroup=(256, 1, 1),
    input_bindings=(0,),
    input_shapes=[(1024, 2048)],
    output_shape=(2048, 1024),
    rtol=0, atol=0,
    grid=(512 * 256, 1, 1),
    scalars=[dict(binding=2, dtype="u32", value=1024),
             dict(binding=3, dtype="u32", value=2048)],
    flops=0,
    bytes=1024 * 2048 * 4 * 2,
)


def conv2d(name, N, H, W, C, O, R, S, stride, pad, rtol=1e-3, atol=1e-3,
           init_x=("normal", 0.0, 1.0), init_w=None, cpu_iters=None):
    """NHWC x OHWI cross-correlation (reference registry.py:469-477), plus a
    `pad` scalar at binding 11 (the reference kernel has valid padding only)."""
    P = (H + 2 * pad - R) // stride + 1
    Q = (W + 2 * pad - S) // stride + 1
    REGISTRY[name] = dict(
        metal_function="conv2d_f32", threadgroup=(256, 1, 1), input_bindings=(0, 1),
        input_shapes=[(N, H, W, C), (O, R, S, C)], output_shape=(N, P, Q, O),
        rtol=rtol, atol=atol, grid=(((N * P * Q + 127) // 128) * 256, 1, 1),
        scalars=[dict(binding=3, dtype="u32", value=N), dict(binding=4, dtype="u32", value=H),
                 dict(binding=5, dtype="u32", value=W), dict(binding=6, dtype="u32", value=C),
                 dict(binding=7, dtype="u32", value=O), dict(binding=8, dtype="u32", value=R),
                 dict(binding=9, dtype="u32", value=S),
                 dict(binding=10, dtype="u32", value=stride),
                 dict(binding=11, dtype="u32", value=pad)],
        flops=2 * N * P * Q * O * R * S * C,
        bytes=4 * (N * H * W * C + O * R * S * C + N * P * Q * O),
        input_init=[init_x, init_w or ("kaiming_normal", R * S * C)],
        compute_dtype="f32",
        model_kwargs=dict(in_channels=C, out_channels=O, kernel_size=R, stride=stride,
                          padding=pad),
    )
    if cpu_iters:
        REGISTRY[name]["cpu_iters"] = cpu_iters


# NHWC fp32 conv: batch 32, 56x56, 64 -> 64 channels, 3x3, stride 1, pad 1,
# Kaiming-normal weights (std sqrt(2/576)); rtol 1e-3 (atol 1e-3 as the reference).
conv2d("conv2d", 32, 56, 56, 64, 64, 3, 3, stride=1, pad=1, cpu_iters=20)

# The reference's own conv shape: 8x64x64x64 -> 128, 3x3, valid, normal(0,1)
# weights (reference registry.py:469-477).
conv2d("conv2d_ref", 8, 64, 64, 64, 128, 3, 3, stride=1, pad=0,
       init_w=("normal", 0.0, 1.0))


# ---- decoder sub-ops and adjacent GEMMs at the reference's own shapes --------

# RMSNorm over rows of 1024 (reference registry.py:135-136, `reduction`
# helper :79-98): x@0, y@1, cols@2, eps@3.  nn.RMSNorm's gain is all ones at
# init, so y = x * rsqrt(mean(x^2) + eps).
REGISTRY["rms_norm"] = dict(
    metal_function="rms_norm_f32",
    threadgroup=(1024, 1, 1),
    input_bindings=(0,),
    input_shapes=[(1024, 1024)],
    output_shape=(1024, 1024),
    rtol=1e-3, atol=1e-3,
    grid=(1024, 1024, 1),
    scalars=[dict(binding=2, dtype="u32", value=1024),
             dict(binding=3, dtype="f32", value=1e-5)],
    flops=1024 * 1024 * 5,
    bytes=2 * 1024 * 1024 * 4,
    model_kwargs=dict(dims=1024, eps=1e-5),
)

# Matrix-vector product y = A @ x, 1024 x 1024 (reference registry.py:151-162).
REGISTRY["matvec"] = dict(
    metal_function="matvec_f32",
    threadgroup=(1024, 1, 1),
    input_bindings=(0, 1),
    input_shapes=[(1024, 1024), (1024,)],
    output_shape=(1024,),
    rtol=1e-3, atol=1e-3,
    grid=(1024, 1024, 1),
    scalars=[dict(binding=3, dtype="u32", value=1024)],
    flops=2 * 1024 * 1024,
    bytes=4 * (1024 * 1024 + 1024 + 1024),
)

# Batched GEMM C[b] = A[b] @ B[b]: 128 batches of 128 x 256 @ 256 x 512
# (reference registry.py:61-77, 131): A@0, B@1, C@2, M@3, N@4, K@5.
_BB, _BM, _BN, _BK = 128, 128, 512, 256
REGISTRY["batch_mm"] = dict(
    metal_function="batch_matmul_f32",
    threadgroup=(512, 1, 1),
    input_bindings=(0, 1),
    input_shapes=[(_BB, _BM, _BK), (_BB, _BK, _BN)],
    output_shape=(_BB, _BM, _BN),
    rtol=1e-3, atol=1e-3,
    grid=((_BN // 64) * 512, (_BM // 64) * _BB, 1),
    scalars=[dict(binding=3, dtype="u32", value=_BM),
             dict(binding=4, dtype="u32", value=_BN),
             dict(binding=5, dtype="u32", value=_BK)],
    flops=_BB * 2 * _BM * _BN * _BK,
    bytes=_BB * 4 * (_BM * _BK + _BK * _BN + _BM * _BN),
    compute_dtype="f32",
)
