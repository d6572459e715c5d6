"""CPU oracle — test infrastructure only (see oracle/oracle.py).

Import from tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg only.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

from .oracle import *  # noqa: F401,F403
from .oracle import (as_f64, bf16_bits_to_f64, conv2d_nhwc, f32_to_bf16_bits,  # noqa: F401
                     gqa_decode_attention, llama_decoder_layer, llama_decoder_step, matmul,
                     rms_norm, rope_interleaved, silu, softmax, transpose)

LIB_PATH = Path(__file__).resolve().parent / "lib" / "liboracle.so"
_cref = None


def cref() -> ctypes.CDLL:
    """The C restatements in oracle/cref.c (built by `make oracle`)."""
    global _cref
    if _cref is None:
        if not LIB_PATH.is_file():
            raise FileNotFoundError(f"{LIB_PATH} missing: run `make oracle`")
        lib = ctypes.CDLL(str(LIB_PATH))
        p = ctypes.c_void_p
        i64 = ctypes.c_int64
        lib.oracle_gemm_f64.argtypes = [p, p, p, i64, i64, i64]
        lib.oracle_conv2d_nhwc_f64.argtypes = [p, p, p] + [i64] * 9
        lib.oracle_transpose_f32.argtypes = [p, p, i64, i64]
        for f in (lib.oracle_gemm_f64, lib.oracle_conv2d_nhwc_f64, lib.oracle_transpose_f32):
            f.restype = None
        _cref = lib
    return _cref
