"""libmbhip.so loads, exports every symbol include/mbhip.h declares, and its
error paths work without a GPU (reference main.mm:28-32 die() semantics)."""
import ctypes
import re

import pytest

from metalbench_amd import helpers as H
from metalbench_amd import native

HEADER = (H.REPO_ROOT / "include" / "mbhip.h").read_text()
DECLARED = sorted(set(re.findall(r"^\s*[A-Za-z_][\w\s\*]*?\b(mb_\w+)\s*\(", HEADER, re.M)))


def _gpu():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def test_header_declares_the_expected_entry_points():
    for fn in ("mb_init", "mb_run", "mb_kernel_find", "mb_last_error",
               "mb_launch_llama_decoder_step_bf16"):
        assert fn in DECLARED


def test_library_exports_every_declared_symbol():
    lib = native.load()
    missing = [fn for fn in DECLARED if not hasattr(lib, fn)]
    assert not missing, missing
    assert set(DECLARED) == set(native.SIGNATURES), "ctypes signatures out of sync with header"


def test_struct_layouts_match():
    lib = native.load()
    assert lib.mb_abi_version() == 2
    for which, S in native.STRUCTS.items():
        assert lib.mb_abi_struct_size(which) == ctypes.sizeof(S), S.__name__
    assert lib.mb_abi_struct_size(99) == -1


def test_every_registry_function_is_registered():
    names = native.kernel_names()
    for _, name in H.all_kernels():
        assert H.load_baseline(name).metal_function in names


def test_unknown_kernel_is_reported():
    with pytest.raises(native.NativeError) as e:
        native.kernel_find("no_such_kernel_f32")
    assert e.value.code == -2 and "function no_such_kernel_f32 not found" in str(e.value)


@pytest.mark.skipif(_gpu(), reason="checks the no-GPU path")
def test_no_device_and_uninitialised_paths():
    lib = native.load()
    assert lib.mb_init(0) == -1 and "no HIP device" in native.last_error()
    t = native.MbTiming()
    assert lib.mb_run(0, None, 0, 0, 1, 0, ctypes.byref(t)) == -6
    assert lib.mb_launch_transpose_2d_f32(None, None, 4, 4, None) == -6
    assert lib.mb_launch_matmul_f32(None, None, None, 4, 4, 4, None) == -6
    assert lib.mb_launch_copy_f32(None, None, 4, None) == -6
    assert lib.mb_set_stream(None) == -6
    info = native.MbDeviceInfo()
    assert lib.mb_device_info_get(ctypes.byref(info)) == -6
    assert lib.mb_shutdown() == 0 and lib.mb_shutdown() == 0


def test_decoder_workspace_size_without_gpu():
    a = native.MbDecoderStepArgs(batch=16, d_model=4096, n_heads=32, n_kv_heads=8, head_dim=128,
                                 d_ff=14336, cache_len=2048, cache_stride=2048,
                                 rope_base=500000.0, eps=1e-5)
    n = native.load().mb_decoder_step_workspace_bytes(ctypes.byref(a))
    assert 0 < n < (1 << 30), native.last_error()
    # The plan does not depend on mb_init(): without a device the size already
    # holds the split-K partials of the whole-device grid, e.g. gate/up's 56
    # tiles x 4 splits of 16 x 512 fp32 (a plan for one CU would need 1 split).
    assert n >= 56 * 4 * 16 * 512 * 4
    a.head_dim = 64
    assert native.load().mb_decoder_step_workspace_bytes(ctypes.byref(a)) == 0
    # One 8-way tensor-parallel shard (attention width 4 x 128 < d_model) is a
    # supported shape; a residual width that is not a multiple of 128 is not.
    a.head_dim, a.n_heads, a.n_kv_heads, a.d_ff = 128, 4, 1, 1792
    assert native.load().mb_decoder_step_workspace_bytes(ctypes.byref(a)) > 0, native.last_error()
    a.d_model = 4000
    assert native.load().mb_decoder_step_workspace_bytes(ctypes.byref(a)) == 0
