"""volta_mi355x: MI355X (gfx950) backend for VOLTA-ZK's Ligero commit arithmetic.

The product is libvolta_mi355x_backend.so, a drop-in for the reference's
volta_cuda_* C ABI (v37).  This package is its host-side mirror: `accel`
(the seam's Backend over ctypes), `ligero` (commit/combination orchestration)
and `workloads` (synthetic benchmark inputs).
"""
from .accel import (ABI_VERSION, FP2, P, AbiMismatch, AccelError, Backend, DeviceBuffer, DeviceMerkleTree, GpuError,
                    InvalidInput, LibraryLoad, MissingSymbol, abi_symbols, extension_symbols, fp2_as_u64,
                    load_library)

__all__ = ["ABI_VERSION", "FP2", "P", "AbiMismatch", "AccelError", "Backend", "DeviceBuffer", "DeviceMerkleTree", "GpuError",
           "InvalidInput", "LibraryLoad", "MissingSymbol", "abi_symbols", "extension_symbols", "fp2_as_u64",
           "load_library"]
