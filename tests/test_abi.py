"""The C-ABI library loads and exports every entry point declared in
include/spira_hip.h (no compute calls: this runs without a GPU)."""
import ctypes
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "spira_hip.h")
LIB = os.path.join(ROOT, "spira_amd", "libspira_hip.so")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(spira_hip_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared()
    assert "spira_hip_kmap_search" in names and "spira_hip_conv_os" in names
    assert len(names) >= 20


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(LIB)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_last_error_callable_without_gpu():
    lib = ctypes.CDLL(LIB)
    lib.spira_hip_last_error.restype = ctypes.c_char_p
    assert isinstance(lib.spira_hip_last_error(), bytes)
    # argument validation runs on the host: a bad key width is rejected
    rc = lib.spira_hip_pack(None, ctypes.c_int64(1), 48, None, None)
    assert rc != 0
    assert b"key_bits" in lib.spira_hip_last_error()


def test_extension_exports_reference_names():
    from spira_amd.nn.functional import _native
    expected = {
        "cuda_flatten_sort", "cuda_unflatten", "cuda_downsample", "cuda_streamed_output_generate",
        "cuda_binary_search", "cuda_binary_search_streamed", "cuda_binary_search_no_small_z",
        "cuda_convert_transposed_os", "cuda_sparse_convolution_forward_os", "cuda_sparse_convolution_forward_ws",
        "cuda_sparse_convolution_forward_ws_merged", "cuda_sparse_convolution_forward_hs",
        "cuda_sparse_convolution_forward_hs_merged", "cuda_time_gemm", "cuda_time_gather", "cuda_time_scatter",
        "cuda_free_buffers", "cuda_reset_error",
    }
    assert expected <= set(dir(_native._C))


def test_spira_alias_resolves_to_spira_amd():
    """`import spira` (the reference's package name) is this implementation."""
    import spira
    import spira_amd
    assert spira is spira_amd
    import spira.nn
    assert spira.nn.SparseConv is spira_amd.nn.SparseConv
    assert hasattr(spira, "SparseTensor") and hasattr(spira, "tune") and hasattr(spira, "set_kernel_map_cache")


def test_noalloc_scratch_holds_the_maximum_workspace():
    """The allocation-free flatten_sort's fixed 32 MiB scratch holds the
    workspace of its maximum input (1048576 points) for both key widths (a
    host-side size query: no GPU needed)."""
    lib = ctypes.CDLL(LIB)
    lib.spira_hip_flatten_sort_workspace.argtypes = [ctypes.c_int64, ctypes.c_int, ctypes.POINTER(ctypes.c_size_t)]
    for bits in (32, 64):
        wsb = ctypes.c_size_t(0)
        assert lib.spira_hip_flatten_sort_workspace(1 << 20, bits, ctypes.byref(wsb)) == 0
        assert 0 < wsb.value <= 32 << 20, (bits, wsb.value)
