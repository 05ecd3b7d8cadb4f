"""The C-ABI library loads like the reference's Rust seam loads its backend and
exports every symbol include/volta_cuda_abi.h declares.  CPU only: no call
here touches a GPU except context creation, which must fail cleanly when no
device exists."""
import ctypes
import pathlib
import re
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent


def test_header_declares_the_reference_symbol_set():
    from volta_mi355x import abi_symbols
    syms = abi_symbols()
    # rust/volta-accel/src/cuda.rs:1159-1449 loads 123 symbols plus the
    # version query; the test-only injector is among them under cfg(test).
    assert len(syms) == 124
    rust = (pathlib.Path("/root/reference/rust/volta-accel/src/cuda.rs"))
    if rust.exists():  # only in the build container
        ref = set(re.findall(r'b"(volta_cuda_\w+)\\0"', rust.read_text()))
        assert ref == set(syms)


def test_library_exports_every_declared_symbol():
    from volta_mi355x import abi_symbols, extension_symbols
    from volta_mi355x.accel import DEFAULT_LIBRARY
    out = subprocess.run(["nm", "-D", "--defined-only", str(DEFAULT_LIBRARY)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r" T (volta_\w+)$", out, flags=re.M))
    assert set(abi_symbols()) <= exported
    assert set(extension_symbols()) <= exported
    # nothing else leaks from the library's C++ internals
    assert all(s.startswith(("volta_cuda_", "volta_mi355x_")) for s in exported)


def test_load_checks_abi_version():
    from volta_mi355x import ABI_VERSION, load_library
    lib = load_library()
    assert lib.volta_cuda_abi_version() == ABI_VERSION == 37


def test_load_rejects_missing_library(tmp_path):
    from volta_mi355x import LibraryLoad, load_library
    with pytest.raises(LibraryLoad):
        load_library(tmp_path / "nope.so")


def test_raw_stats_layout_matches_reference():
    from volta_mi355x.accel import RawStats
    assert ctypes.sizeof(RawStats) == 504  # cuda.rs:78
    assert RawStats.timing_mode.offset == 496


def test_create_fails_cleanly_without_gpu():
    import os
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU driver is present; context creation is covered by the gpu tests")
    from volta_mi355x import GpuError, Backend
    with pytest.raises(GpuError):
        Backend()


def test_out_of_scope_symbols_fail_explicitly_on_null_context():
    from volta_mi355x import load_library
    lib = load_library()
    # a null context is rejected before anything else
    assert lib.volta_cuda_gemm_i64(None, None, None, None, 0, 0, 0) != 0
