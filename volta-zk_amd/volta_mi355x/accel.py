"""Host-side mirror of the reference's accelerator seam for the Ligero path.

`Backend` mirrors the PCS subset of rust/volta-accel's `Backend` (resident
kind): same method names, argument meaning, allocation-returning style and
error behaviour (geometry errors raise `InvalidInput`, backend failures raise
`GpuError` carrying volta_cuda_last_error).  It drives
libvolta_mi355x_backend.so through the same C ABI the Rust seam loads
(rust/volta-accel/src/cuda.rs:1119-1449): dlopen, ABI check (37), eager
resolution of every volta_cuda_* symbol, create/destroy.

There is no CPU fallback: if the library or a GPU is missing, construction
raises.
"""
from __future__ import annotations

import ctypes
import os
import pathlib
import re
from dataclasses import dataclass

import numpy as np

ABI_VERSION = 37
P = 0xFFFF_FFFF_0000_0001
FP2 = np.dtype([("c0", "<u8"), ("c1", "<u8")])

_PKG = pathlib.Path(__file__).resolve().parent.parent
DEFAULT_LIBRARY = _PKG / "libvolta_mi355x_backend.so"
HEADER = _PKG.parent / "include" / "volta_cuda_abi.h"

# Operation indices of RawStats.calls / kernel_ns (reference .cu:25-32;
# rust/volta-accel/src/lib.rs:25-59).
OPERATIONS = ("gemm", "logup", "pcs_rows", "pcs_ntt", "pcs_merkle", "auth_masks", "mailbox")


class AccelError(Exception):
    """Base of the seam's errors (rust/volta-accel/src/lib.rs AccelError)."""


class LibraryLoad(AccelError):
    pass


class MissingSymbol(AccelError):
    pass


class AbiMismatch(AccelError):
    pass


class InvalidInput(AccelError):
    pass


class GpuError(AccelError):
    """A backend call returned non-zero (the reference's AccelError::Cuda)."""


class RawStats(ctypes.Structure):
    _fields_ = [
        ("calls", ctypes.c_uint64 * 7),
        ("kernel_ns", ctypes.c_uint64 * 7),
    ] + [(n, ctypes.c_uint64) for n in (
        "h2d_bytes d2h_bytes d2d_bytes device_zeroed_bytes device_generated_bytes h2d_ns d2h_ns "
        "resident_h2d_host_calls resident_d2h_host_calls resident_h2d_host_call_ns resident_d2h_host_call_ns "
        "synchronizations synchronization_ns sync_host_output sync_upload_lifetime sync_timing_flush "
        "sync_profiling_legacy sync_allocator_flush allocation_calls resident_alloc_requests resident_reuse_hits "
        "resident_free_requests physical_free_calls live_device_bytes peak_device_bytes pinned_allocation_calls "
        "pinned_alloc_requests pinned_reuse_hits pinned_free_requests pinned_physical_free_calls "
        "pinned_host_write_calls pinned_host_write_bytes live_pinned_bytes peak_pinned_bytes x4c_arena_reset_calls "
        "x4c_arena_reset_bytes x4c_kernel_launches x4c_control_peek_calls x4c_control_peek_pending timing_records "
        "timing_elapsed_query_attempts timing_elapsed_no_write timing_event_queries timing_event_api_calls "
        "timing_pending_high_water timing_flush_count coarse_timing_scopes coarse_timing_ns").split()
    ] + [("timing_mode", ctypes.c_uint32), ("reserved", ctypes.c_uint32)]


assert ctypes.sizeof(RawStats) == 504


class Fp2C(ctypes.Structure):
    _fields_ = [("c0", ctypes.c_uint64), ("c1", ctypes.c_uint64)]


def abi_symbols(header: pathlib.Path = HEADER) -> list[str]:
    """The reference-ABI symbol names declared in include/volta_cuda_abi.h."""
    text = header.read_text()
    return sorted(set(re.findall(r"^[\w \*]+?\b(volta_cuda_\w+)\(", text, flags=re.M)))


def extension_symbols(header: pathlib.Path = HEADER) -> list[str]:
    text = header.read_text()
    return sorted(set(re.findall(r"^[\w \*]+?\b(volta_mi355x_\w+)\(", text, flags=re.M)))


_u64, _sz, _int, _vp = ctypes.c_uint64, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p
_SIGS = {
    "volta_cuda_abi_version": (ctypes.c_uint32, []),
    "volta_cuda_create": (_int, [ctypes.POINTER(_vp)]),
    "volta_cuda_destroy": (None, [_vp]),
    "volta_cuda_last_error": (ctypes.c_char_p, [_vp]),
    "volta_cuda_set_resident_timing_policy": (_int, [_vp, _int]),
    "volta_cuda_begin_coarse_timing": (_int, [_vp, _int]),
    "volta_cuda_end_coarse_timing": (_int, [_vp]),
    "volta_cuda_abort_coarse_timing": (_int, [_vp]),
    "volta_cuda_flush_profiling": (_int, [_vp]),
    "volta_cuda_reset_stats": (_int, [_vp]),
    "volta_cuda_get_stats": (_int, [_vp, ctypes.POINTER(RawStats)]),
    "volta_cuda_memory_breakdown": (_int, [_vp, ctypes.POINTER(_u64), ctypes.POINTER(_u64), ctypes.POINTER(_u64)]),
    "volta_cuda_trim_resident_cache": (_int, [_vp]),
    "volta_cuda_resident_alloc": (_int, [_vp, _sz, ctypes.POINTER(_u64)]),
    "volta_cuda_resident_free": (_int, [_vp, _u64]),
    "volta_cuda_resident_upload": (_int, [_vp, _u64, _sz, _vp, _sz]),
    "volta_cuda_resident_download": (_int, [_vp, _u64, _sz, _vp, _sz]),
    "volta_cuda_resident_zero": (_int, [_vp, _u64, _sz, _sz]),
    "volta_cuda_resident_copy_rows": (_int, [_vp, _u64, _sz, _sz, _u64, _sz, _sz, _sz, _sz]),
    "volta_cuda_ntt_fp": (_int, [_vp, _vp, _sz, _sz, _vp]),
    "volta_cuda_ntt_fp_batch": (_int, [_vp, _vp, _sz, _sz, _sz, _vp]),
    "volta_cuda_ntt_fp2": (_int, [_vp, _vp, _sz, _sz, _vp]),
    "volta_cuda_ntt_fp_batch_device": (_int, [_vp, _u64, _sz, _sz, _sz, _u64, _sz]),
    "volta_cuda_ntt_fp2_batch_device": (_int, [_vp, _u64, _sz, _sz, _sz, _u64, _sz]),
    "volta_cuda_pcs_messages_device": (_int, [_vp, _u64, _sz, _u64, _sz, _sz, _sz, _sz, _sz, _u64, _sz]),
    "volta_cuda_pcs_combine_rows_device": (_int, [_vp, _u64, _sz, _u64, _sz, _u64, _sz, _sz, _sz, _sz, _sz, _u64, _sz]),
    "volta_cuda_pcs_combine_rows": (_int, [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _vp]),
    "volta_cuda_fp2_powers_device": (_int, [_vp, _u64, _u64, _u64, _sz, _sz]),
    "volta_cuda_fp2_add_inplace_device": (_int, [_vp, _u64, _sz, _u64, _sz, _sz]),
    "volta_cuda_logup_eq_rows_device": (_int, [_vp, _u64, _sz, _sz, _sz, _u64, _sz]),
    "volta_cuda_fp2_row_dots_device": (_int, [_vp, _u64, _sz, _sz, _u64, _sz, _sz, _u64, _sz, _sz, _sz]),
    "volta_cuda_pcs_gather_columns_device": (_int, [_vp, _u64, _sz, _sz, _sz, _u64, _sz, _sz, _u64, _sz, _int]),
    "volta_cuda_pcs_gather_columns": (_int, [_vp, _vp, _sz, _sz, _vp, _sz, _vp]),
    "volta_cuda_chacha8_prover_secret_fp_rows_device": (_int, [_vp, _u64, _sz, _vp, _u64, _sz, _sz]),
    "volta_cuda_chacha8_prover_secret_fp2_rows_padded_device": (_int, [_vp, _u64, _sz, _vp, _u64, _sz, _sz, _sz]),
    "volta_cuda_mock_correlation_sub_masks_device": (_int, [_vp, _u64, _sz, _vp, _u64, _sz, _sz]),
    "volta_cuda_hash_fp_tree_device": (_int, [_vp, _u64, _sz, _sz, _sz, _u64, _sz]),
    "volta_cuda_hash_fp2_tree_device": (_int, [_vp, _u64, _sz, _sz, _sz, _u64, _sz]),
    "volta_cuda_merkle_paths_device": (_int, [_vp, _u64, _sz, _sz, _u64, _sz, _sz, _u64, _sz]),
    "volta_cuda_hash_fp_columns": (_int, [_vp, _vp, _sz, _sz, _vp]),
    "volta_cuda_x4b_ntt_fp2": (_int, [_vp, _vp, _sz, _sz, _vp]),
    "volta_cuda_pinned_alloc": (_int, [_vp, _sz, ctypes.POINTER(_u64)]),
    "volta_cuda_pinned_write": (_int, [_vp, _u64, _sz, _vp, _sz]),
    "volta_cuda_pinned_wait_ready": (_int, [_vp, _u64]),
    "volta_cuda_pinned_free": (_int, [_vp, _u64]),
    "volta_cuda_x4c_upload_pinned": (_int, [_vp, _u64, _sz, _u64, _sz, _sz]),
    "volta_cuda_x4c_direct_fold_pinned_tile": (_int, [_vp, _u64, _sz, _u64, _sz, _sz, _sz, _sz, _sz, _u64, _u64]),
    "volta_cuda_x4c_direct_fold_arena": (_int, [_vp, _u64, _sz, _sz, _sz, _u64, _u64]),
    "volta_cuda_fp2_mobius_inverse_inplace_device": (_int, [_vp, _u64, _sz, _sz]),
    "volta_mi355x_x4_ntt_fp2_device": (_int, [_vp, _u64, _sz, _sz, _sz, _u64, _sz]),
    "volta_mi355x_ntt_fp_inverse_batch_device": (_int, [_vp, _u64, _sz, _sz, _sz, _u64, _sz]),
    "volta_mi355x_ntt_fp_encode_device": (_int, [_vp, _u64, _sz, _sz, _sz, _sz, _u64, _sz]),
    "volta_mi355x_pcs_encode_device": (_int, [_vp, _u64, _sz, _u64, _sz, _sz, _sz, _sz, _sz, _u64, _sz]),
    "volta_mi355x_combine_rows_fp_device": (_int, [_vp, _u64, _sz, _sz, _sz, _u64, _sz, _sz, _u64, _sz]),
    "volta_mi355x_pcs_combine_rows_device_noalloc": (_int, [_vp, _u64, _sz, _u64, _sz, _u64, _sz, _sz, _sz, _sz, _sz,
                                                            _u64, _sz]),
    "volta_mi355x_resident_device_ptr": (_int, [_vp, _u64, _sz, _sz, ctypes.POINTER(_vp)]),
    "volta_mi355x_stream": (_int, [_vp, ctypes.POINTER(_vp)]),
    "volta_mi355x_synchronize": (_int, [_vp]),
    "volta_mi355x_probe_copy_device": (_int, [_vp, _u64, _u64, _sz]),
    "volta_mi355x_probe_expand_device": (_int, [_vp, _u64, _u64, _sz]),
    "volta_mi355x_probe_fp2_device": (_int, [_vp, _u64, _u64, _u64, _sz, _int]),
    "volta_mi355x_fnv64_host": (_u64, [_vp, _sz, _u64]),
}


def load_library(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """dlopen the backend like CudaContext::load (cuda.rs:1119-1157): resolve
    every reference symbol eagerly and check the ABI version first."""
    path = str(path or os.environ.get("VOLTA_CUDA_LIBRARY") or DEFAULT_LIBRARY)
    if not os.path.exists(path):
        raise LibraryLoad(f"{path}: not found (build it with volta-zk_amd/build.py)")
    try:
        lib = ctypes.CDLL(path, mode=os.RTLD_NOW | os.RTLD_LOCAL)
    except OSError as e:
        raise LibraryLoad(f"{path}: {e}") from e
    try:
        abi = lib.volta_cuda_abi_version
    except AttributeError as e:
        raise MissingSymbol("volta_cuda_abi_version") from e
    abi.restype = ctypes.c_uint32
    found = abi()
    if found != ABI_VERSION:
        raise AbiMismatch(f"expected ABI {ABI_VERSION}, found {found}")
    for name in abi_symbols() + extension_symbols():
        if not hasattr(lib, name):
            raise MissingSymbol(name)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


@dataclass
class DeviceBuffer:
    """A resident allocation owned by one Backend (rust DeviceBuffer<T>)."""
    id: int
    len: int
    dtype: np.dtype
    owner: int  # id() of the owning backend

    @property
    def nbytes(self) -> int:
        return self.len * self.dtype.itemsize


@dataclass
class DeviceMerkleTree:
    """A resident BLAKE3 column tree (rust DeviceMerkleTree, lib.rs:6700-6725):
    storage holds (2 leaves - 1) 32-byte hashes, leaves first, root last."""
    storage: DeviceBuffer
    leaves: int


def _as_fp2(a) -> np.ndarray:
    a = np.ascontiguousarray(a)
    if a.dtype == FP2:
        return a.reshape(-1)
    a = np.ascontiguousarray(a, dtype=np.uint64)
    if a.shape[-1] != 2:
        raise InvalidInput("Fp2 arrays must have a trailing dimension of 2 (c0, c1)")
    return a.reshape(-1, 2).view(FP2).reshape(-1)


def fp2_as_u64(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a).view(np.uint64).reshape(a.shape + (2,))


class Backend:
    """Resident backend over one context (rust Backend::cuda_resident)."""

    def __init__(self, library: str | os.PathLike | None = None, timing_policy: int | None = 0):
        self.lib = load_library(library)
        raw = ctypes.c_void_p()
        rc = self.lib.volta_cuda_create(ctypes.byref(raw))
        if rc != 0 or not raw.value:
            msg = self.lib.volta_cuda_last_error(raw).decode() if raw.value else f"status {rc}"
            if raw.value:
                self.lib.volta_cuda_destroy(raw)
            raise GpuError(f"context creation failed: {msg}")
        self.raw = raw
        self._live: dict[int, DeviceBuffer] = {}
        if timing_policy is not None:
            self._check(self.lib.volta_cuda_set_resident_timing_policy(self.raw, timing_policy))

    # ---- lifecycle ----------------------------------------------------------
    def close(self) -> None:
        if getattr(self, "raw", None) is not None and self.raw.value:
            self.lib.volta_cuda_destroy(self.raw)
            self.raw = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):  # pragma: no cover - best effort
        try:
            self.close()
        except Exception:
            pass

    def last_error(self) -> str:
        return self.lib.volta_cuda_last_error(self.raw).decode()

    def _check(self, rc: int) -> None:
        if rc != 0:
            raise GpuError(self.last_error() or f"status {rc}")

    def _own(self, buf: DeviceBuffer) -> None:
        if buf.owner != id(self) or buf.id not in self._live:
            raise InvalidInput("device buffer belongs to another backend or was freed")

    # ---- resident memory (lib.rs:1372-1640) ---------------------------------------
    def alloc_device(self, n: int, dtype) -> DeviceBuffer:
        dtype = np.dtype(dtype)
        if n <= 0:
            raise InvalidInput("device allocations must be non-empty")
        out = ctypes.c_uint64()
        self._check(self.lib.volta_cuda_resident_alloc(self.raw, n * dtype.itemsize, ctypes.byref(out)))
        buf = DeviceBuffer(out.value, n, dtype, id(self))
        self._live[buf.id] = buf
        return buf

    def free_device(self, buf: DeviceBuffer) -> None:
        self._own(buf)
        self._check(self.lib.volta_cuda_resident_free(self.raw, buf.id))
        del self._live[buf.id]

    def upload_device(self, host: np.ndarray, dtype=None) -> DeviceBuffer:
        arr = _as_fp2(host) if dtype is not None and np.dtype(dtype) == FP2 else np.ascontiguousarray(host, dtype=dtype)
        buf = self.alloc_device(max(arr.size, 1), arr.dtype)
        if arr.size:
            self.upload_into(buf, 0, arr)
        return buf

    def upload_into(self, buf: DeviceBuffer, offset: int, host: np.ndarray) -> None:
        self._own(buf)
        arr = np.ascontiguousarray(host)
        self._check(self.lib.volta_cuda_resident_upload(self.raw, buf.id, offset * buf.dtype.itemsize,
                                                        arr.ctypes.data, arr.nbytes))

    def download_device(self, buf: DeviceBuffer, offset: int = 0, count: int | None = None) -> np.ndarray:
        self._own(buf)
        count = buf.len - offset if count is None else count
        out = np.empty(count, dtype=buf.dtype)
        if count:
            self._check(self.lib.volta_cuda_resident_download(self.raw, buf.id, offset * buf.dtype.itemsize,
                                                              out.ctypes.data, out.nbytes))
        return out

    def zero_device(self, buf: DeviceBuffer, offset: int, count: int) -> None:
        self._own(buf)
        sz = buf.dtype.itemsize
        self._check(self.lib.volta_cuda_resident_zero(self.raw, buf.id, offset * sz, count * sz))

    def copy_device_rows(self, src: DeviceBuffer, src_offset: int, src_stride: int, dst: DeviceBuffer,
                         dst_offset: int, dst_stride: int, rows: int, row_len: int) -> None:
        """Strided D2D copy in elements of the buffers' dtype (lib.rs:1613)."""
        self._own(src)
        self._own(dst)
        sz = src.dtype.itemsize
        self._check(self.lib.volta_cuda_resident_copy_rows(self.raw, src.id, src_offset * sz, src_stride * sz,
                                                           dst.id, dst_offset * sz, dst_stride * sz, rows,
                                                           row_len * sz))

    def device_ptr(self, buf: DeviceBuffer, offset: int = 0) -> int:
        self._own(buf)
        out = ctypes.c_void_p()
        sz = buf.dtype.itemsize
        self._check(self.lib.volta_mi355x_resident_device_ptr(self.raw, buf.id, offset * sz,
                                                              (buf.len - offset) * sz, ctypes.byref(out)))
        return out.value

    def stream(self) -> int:
        out = ctypes.c_void_p()
        self._check(self.lib.volta_mi355x_stream(self.raw, ctypes.byref(out)))
        return out.value or 0

    def synchronize(self) -> None:
        self._check(self.lib.volta_mi355x_synchronize(self.raw))

    # ---- measurement (lib.rs:1106-1171) ---------------------------------------------
    def reset_stats(self) -> None:
        self._check(self.lib.volta_cuda_reset_stats(self.raw))

    def get_stats(self) -> dict:
        s = RawStats()
        self._check(self.lib.volta_cuda_get_stats(self.raw, ctypes.byref(s)))
        out = {name: getattr(s, name) for name, _ in RawStats._fields_ if name not in ("calls", "kernel_ns")}
        out["calls"] = dict(zip(OPERATIONS, list(s.calls)))
        out["kernel_ns"] = dict(zip(OPERATIONS, list(s.kernel_ns)))
        return out

    begin_measurement = reset_stats
    finish_measurement = get_stats

    def memory_breakdown(self) -> tuple[int, int, int]:
        a, b, c = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
        self._check(self.lib.volta_cuda_memory_breakdown(self.raw, ctypes.byref(a), ctypes.byref(b), ctypes.byref(c)))
        return a.value, b.value, c.value

    # ---- PCS primitives -------------------------------------------------------------
    @staticmethod
    def _pow2(n: int) -> bool:
        return n >= 2 and (n & (n - 1)) == 0

    def _region(self, buf: DeviceBuffer, offset: int, count: int) -> None:
        self._own(buf)
        if offset < 0 or count < 0 or offset + count > buf.len:
            raise InvalidInput("device region is out of bounds")

    def ntt_fp_batch_device(self, inp: DeviceBuffer, rows: int, n: int) -> DeviceBuffer:
        """Batched forward NTT of pre-padded rows x n (lib.rs:5419-5448)."""
        if rows == 0 or not self._pow2(n):
            raise InvalidInput("invalid resident Fp NTT geometry")
        self._region(inp, 0, rows * n)
        out = self.alloc_device(rows * n, np.uint64)
        self._call_or_free(out, self.lib.volta_cuda_ntt_fp_batch_device, inp.id, 0, rows, n, out.id, 0)
        return out

    def ntt_fp2_batch_device(self, inp: DeviceBuffer, rows: int, n: int) -> DeviceBuffer:
        if rows == 0 or not self._pow2(n):
            raise InvalidInput("invalid resident Fp2 NTT geometry")
        self._region(inp, 0, rows * n)
        out = self.alloc_device(rows * n, FP2)
        self._call_or_free(out, self.lib.volta_cuda_ntt_fp2_batch_device, inp.id, 0, rows, n, out.id, 0)
        return out

    def ntt_fp_inverse_batch_device(self, inp: DeviceBuffer, rows: int, n: int) -> DeviceBuffer:
        if rows == 0 or not self._pow2(n):
            raise InvalidInput("invalid resident inverse Fp NTT geometry")
        self._region(inp, 0, rows * n)
        out = self.alloc_device(rows * n, np.uint64)
        self._call_or_free(out, self.lib.volta_mi355x_ntt_fp_inverse_batch_device, inp.id, 0, rows, n, out.id, 0)
        return out

    def ntt_fp_encode_device(self, msgs: DeviceBuffer, rows: int, msg_len: int, n: int) -> DeviceBuffer:
        if rows == 0 or not self._pow2(n) or msg_len > n:
            raise InvalidInput("invalid resident Fp encode geometry")
        self._region(msgs, 0, rows * msg_len)
        out = self.alloc_device(rows * n, np.uint64)
        self._call_or_free(out, self.lib.volta_mi355x_ntt_fp_encode_device, msgs.id, 0, rows, msg_len, n, out.id, 0)
        return out

    def ntt_fp_batch(self, messages: np.ndarray, rows: int, msg_len: int, n: int) -> np.ndarray:
        """Hybrid form: compact host rows in, rows x n codewords out (lib.rs:4722-4746)."""
        m = np.ascontiguousarray(messages, dtype=np.uint64).reshape(-1)
        if rows == 0 or not self._pow2(n) or msg_len > n or m.size != rows * msg_len:
            raise InvalidInput("invalid Fp NTT batch geometry")
        out = np.empty(rows * n, dtype=np.uint64)
        self._check(self.lib.volta_cuda_ntt_fp_batch(self.raw, m.ctypes.data, rows, msg_len, n, out.ctypes.data))
        return out.reshape(rows, n)

    def ntt_fp(self, msg: np.ndarray, n: int) -> np.ndarray:
        m = np.ascontiguousarray(msg, dtype=np.uint64).reshape(-1)
        if not self._pow2(n) or m.size > n:
            raise InvalidInput("invalid Fp NTT geometry")
        out = np.empty(n, dtype=np.uint64)
        self._check(self.lib.volta_cuda_ntt_fp(self.raw, m.ctypes.data, m.size, n, out.ctypes.data))
        return out

    def ntt_fp2(self, msg, n: int) -> np.ndarray:
        m = _as_fp2(msg)
        if not self._pow2(n) or m.size > n:
            raise InvalidInput("invalid Fp2 NTT geometry")
        out = np.empty(n, dtype=FP2)
        self._check(self.lib.volta_cuda_ntt_fp2(self.raw, m.ctypes.data, m.size, n, out.ctypes.data))
        return fp2_as_u64(out)

    def pcs_messages_device(self, weights: DeviceBuffer, weights_offset: int, pads: DeviceBuffer, pads_offset: int,
                            rows: int, cols: int, pad: int, code_len: int) -> DeviceBuffer:
        """msg = lift(w) || pads || 0 (lib.rs:6478-6520)."""
        if rows == 0 or cols == 0 or cols + pad > code_len:
            raise InvalidInput("invalid resident PCS message geometry")
        self._region(weights, weights_offset, rows * cols)
        self._region(pads, pads_offset, rows * pad)
        out = self.alloc_device(rows * code_len, np.uint64)
        self._call_or_free(out, self.lib.volta_cuda_pcs_messages_device, weights.id, weights_offset, pads.id,
                           pads_offset, rows, cols, pad, code_len, out.id, 0)
        return out

    def pcs_encode_device(self, weights: DeviceBuffer, weights_offset: int, pads: DeviceBuffer, pads_offset: int,
                          rows: int, cols: int, pad: int, code_len: int) -> DeviceBuffer:
        """Fused messages + NTT (extension): same codewords, no message buffer."""
        if rows == 0 or cols == 0 or cols + pad > code_len or not self._pow2(code_len):
            raise InvalidInput("invalid resident PCS encode geometry")
        self._region(weights, weights_offset, rows * cols)
        self._region(pads, pads_offset, rows * pad)
        out = self.alloc_device(rows * code_len, np.uint64)
        self._call_or_free(out, self.lib.volta_mi355x_pcs_encode_device, weights.id, weights_offset, pads.id,
                           pads_offset, rows, cols, pad, code_len, out.id, 0)
        return out

    def pcs_combine_rows_device(self, weights: DeviceBuffer, weights_offset: int, pads: DeviceBuffer,
                                pads_offset: int, coeffs: DeviceBuffer, coeffs_offset: int, rows: int, cols: int,
                                pad: int, combinations: int) -> DeviceBuffer:
        """u[c][j] = sum_i coeffs[c*rows+i] * msg_i[j] (lib.rs:6522-6569)."""
        if rows == 0 or cols == 0 or combinations == 0:
            raise InvalidInput("invalid resident PCS combination geometry")
        self._region(weights, weights_offset, rows * cols)
        self._region(pads, pads_offset, rows * pad)
        self._region(coeffs, coeffs_offset, combinations * rows)
        out = self.alloc_device(combinations * (cols + pad), FP2)
        self._call_or_free(out, self.lib.volta_cuda_pcs_combine_rows_device, weights.id, weights_offset, pads.id,
                           pads_offset, coeffs.id, coeffs_offset, rows, cols, pad, combinations, out.id, 0)
        return out

    def combine_rows_fp_device(self, matrix: DeviceBuffer, rows: int, cols: int, coeffs: DeviceBuffer,
                               combinations: int) -> DeviceBuffer:
        if rows == 0 or cols == 0 or combinations == 0:
            raise InvalidInput("invalid resident Fp combination geometry")
        self._region(matrix, 0, rows * cols)
        self._region(coeffs, 0, combinations * rows)
        out = self.alloc_device(combinations * cols, FP2)
        self._call_or_free(out, self.lib.volta_mi355x_combine_rows_fp_device, matrix.id, 0, rows, cols, coeffs.id, 0,
                           combinations, out.id, 0)
        return out

    def pcs_combine_rows(self, weights: np.ndarray, pads: np.ndarray, coeffs, rows: int, cols: int, pad: int,
                         combinations: int) -> np.ndarray:
        """Hybrid form (lib.rs:6407-6445); returns (combinations, cols+pad, 2) u64."""
        w = np.ascontiguousarray(weights, dtype=np.int16).reshape(-1)
        p = np.ascontiguousarray(pads, dtype=np.uint64).reshape(-1)
        c = _as_fp2(coeffs)
        if rows == 0 or cols == 0 or combinations == 0 or w.size != rows * cols or p.size != rows * pad \
                or c.size != combinations * rows:
            raise InvalidInput("invalid PCS row-combination geometry")
        out = np.empty(combinations * (cols + pad), dtype=FP2)
        pp = p.ctypes.data if p.size else None
        self._check(self.lib.volta_cuda_pcs_combine_rows(self.raw, w.ctypes.data, pp, c.ctypes.data, rows, cols, pad,
                                                         combinations, out.ctypes.data))
        return fp2_as_u64(out.reshape(combinations, cols + pad))

    def fp2_powers_device(self, c, count: int) -> DeviceBuffer:
        """[c^1 .. c^count] (lib.rs:1912-1937)."""
        c0, c1 = int(c[0]), int(c[1])
        if count == 0 or c0 >= P or c1 >= P:
            raise InvalidInput("invalid Fp2 powers input")
        out = self.alloc_device(count, FP2)
        self._call_or_free(out, self.lib.volta_cuda_fp2_powers_device, c0, c1, out.id, 0, count)
        return out

    def fp2_add_inplace_device(self, target: DeviceBuffer, target_offset: int, add: DeviceBuffer, add_offset: int,
                               length: int) -> None:
        self._region(target, target_offset, length)
        self._region(add, add_offset, length)
        self._check(self.lib.volta_cuda_fp2_add_inplace_device(self.raw, target.id, target_offset, add.id, add_offset,
                                                               length))

    def pcs_gather_columns_device(self, matrix: DeviceBuffer, rows: int, cols: int, indices: np.ndarray,
                                  fp2: bool = False) -> DeviceBuffer:
        """out[q*rows + i] = M[i*cols + idx[q]] (lib.rs:6773-6827)."""
        idx = np.ascontiguousarray(indices, dtype=np.uint32).reshape(-1)
        if rows == 0 or cols == 0 or idx.size == 0 or (idx >= cols).any():
            raise InvalidInput("invalid PCS column-gather geometry")
        self._region(matrix, 0, rows * cols)
        ib = self.upload_device(idx)
        try:
            out = self.alloc_device(rows * idx.size, FP2 if fp2 else np.uint64)
            self._call_or_free(out, self.lib.volta_cuda_pcs_gather_columns_device, matrix.id, 0, rows, cols, ib.id, 0,
                               idx.size, out.id, 0, 1 if fp2 else 0)
        finally:
            self.free_device(ib)
        return out

    def pcs_gather_columns(self, matrix: np.ndarray, indices: np.ndarray) -> np.ndarray:
        m = np.ascontiguousarray(matrix, dtype=np.uint64)
        rows, cols = m.shape
        idx = np.ascontiguousarray(indices, dtype=np.uint32).reshape(-1)
        if idx.size == 0 or (idx >= cols).any():
            raise InvalidInput("invalid PCS column-gather geometry")
        out = np.empty(rows * idx.size, dtype=np.uint64)
        self._check(self.lib.volta_cuda_pcs_gather_columns(self.raw, m.ctypes.data, rows, cols, idx.ctypes.data,
                                                           idx.size, out.ctypes.data))
        return out.reshape(idx.size, rows)

    def chacha8_prover_secret_fp_rows_device(self, seed: bytes, base_domain: int, rows: int,
                                             count: int) -> DeviceBuffer:
        """Row r = FpStream::domain_separated(seed, base+r), count draws (lib.rs:1748-1757)."""
        seed = bytes(seed)
        if len(seed) != 32 or rows == 0 or count == 0:
            raise InvalidInput("ChaCha8 row generation needs a 32-byte seed and non-zero rows and count")
        out = self.alloc_device(rows * count, np.uint64)
        buf = (ctypes.c_uint8 * 32).from_buffer_copy(seed)
        self._call_or_free(out, self.lib.volta_cuda_chacha8_prover_secret_fp_rows_device, out.id, 0, buf,
                           base_domain, rows, count)
        return out

    def chacha8_prover_secret_fp2_rows_padded_device(self, seed: bytes, base_domain: int, rows: int, count: int,
                                                     padded: int) -> DeviceBuffer:
        seed = bytes(seed)
        if len(seed) != 32 or rows == 0 or count == 0 or count > padded:
            raise InvalidInput("invalid prover-secret padded Fp2 row generation")
        out = self.alloc_device(rows * padded, FP2)
        buf = (ctypes.c_uint8 * 32).from_buffer_copy(seed)
        self._call_or_free(out, self.lib.volta_cuda_chacha8_prover_secret_fp2_rows_padded_device, out.id, 0, buf,
                           base_domain, rows, count, padded)
        return out

    # ---- helpers ---------------------------------------------------------------------------
    # ---- opening-path helpers (lib.rs:1873-1908, 3037-3053, 6167-6205) -------------------
    def logup_eq_rows_device(self, points: DeviceBuffer | None, rows: int, dims: int) -> DeviceBuffer:
        """rows x 2^dims Fp2: row r is the LSB-first equality table of point r."""
        if rows == 0 or dims >= 64:
            raise InvalidInput("invalid resident eq-row geometry")
        if dims and points is None:
            raise InvalidInput("non-empty equality rows require resident points")
        if points is not None:
            self._region(points, 0, rows * dims)
        out = self.alloc_device(rows << dims, FP2)
        self._call_or_free(out, self.lib.volta_cuda_logup_eq_rows_device, points.id if points is not None else 0, 0,
                           rows, dims, out.id, 0)
        return out

    def equality_weights_device(self, point) -> DeviceBuffer:
        """The 2^len(point) equality weights of one Fp2 point (lib.rs:3037-3053)."""
        pts = np.ascontiguousarray(point, dtype=np.uint64).reshape(-1, 2)
        buf = self.upload_device(pts, FP2) if len(pts) else None
        try:
            return self.logup_eq_rows_device(buf, 1, len(pts))
        finally:
            if buf is not None:
                self.free_device(buf)

    def fp2_row_dots_device(self, a: DeviceBuffer, a_offset: int, a_stride: int, b: DeviceBuffer, b_offset: int,
                            b_stride: int, rows: int, length: int) -> DeviceBuffer:
        """rows Fp2: sum_j a[r a_stride + j] b[r b_stride + j] (element offsets)."""
        if rows == 0 or length == 0 or a_stride < length or b_stride < length:
            raise InvalidInput("invalid Fp2 row-dot geometry")
        self._region(a, a_offset, (rows - 1) * a_stride + length)
        self._region(b, b_offset, (rows - 1) * b_stride + length)
        out = self.alloc_device(rows, FP2)
        self._call_or_free(out, self.lib.volta_cuda_fp2_row_dots_device, a.id, a_offset, a_stride, b.id, b_offset,
                           b_stride, out.id, 0, rows, length)
        return out

    # ---- BLAKE3 column leaves and Merkle tree (lib.rs:6380-6405, 6677-6770) ------------
    def _hash_tree_device(self, matrix: DeviceBuffer, rows: int, cols: int, fp2: bool) -> DeviceMerkleTree:
        if rows == 0 or cols == 0 or cols & (cols - 1):
            raise InvalidInput("invalid resident Merkle matrix geometry")
        self._region(matrix, 0, rows * cols)
        storage = self.alloc_device((2 * cols - 1) * 32, np.uint8)
        fn = self.lib.volta_cuda_hash_fp2_tree_device if fp2 else self.lib.volta_cuda_hash_fp_tree_device
        self._call_or_free(storage, fn, matrix.id, 0, rows, cols, storage.id, 0)
        return DeviceMerkleTree(storage, cols)

    def hash_fp_tree_device(self, matrix: DeviceBuffer, rows: int, cols: int) -> DeviceMerkleTree:
        """Leaves = blake3 of each column of the rows x cols Fp matrix, then the tree."""
        return self._hash_tree_device(matrix, rows, cols, False)

    def hash_fp2_tree_device(self, matrix: DeviceBuffer, rows: int, cols: int) -> DeviceMerkleTree:
        """The same over an Fp2 matrix, each element hashed as c0 then c1."""
        return self._hash_tree_device(matrix, rows, cols, True)

    def merkle_root_device(self, tree: DeviceMerkleTree) -> bytes:
        self._own(tree.storage)
        return self.download_device(tree.storage, (2 * tree.leaves - 2) * 32, 32).tobytes()

    def merkle_paths_device(self, tree: DeviceMerkleTree, indices: DeviceBuffer, queries: int) -> DeviceBuffer:
        """queries x log2(leaves) sibling hashes (32 bytes each), leaf level first."""
        self._own(tree.storage)
        self._region(indices, 0, queries)
        if queries == 0:
            raise InvalidInput("empty resident Merkle query set")
        bits = tree.leaves.bit_length() - 1
        paths = self.alloc_device(max(queries * bits * 32, 1), np.uint8)
        self._call_or_free(paths, self.lib.volta_cuda_merkle_paths_device, tree.storage.id, 0, tree.leaves,
                           indices.id, 0, queries, paths.id, 0)
        return paths

    def free_device_merkle_tree(self, tree: DeviceMerkleTree) -> None:
        self.free_device(tree.storage)

    def hash_fp_columns(self, matrix: np.ndarray, rows: int, cols: int) -> np.ndarray:
        """Host form: cols x 32 leaf bytes (lib.rs:6380-6405, same geometry rule)."""
        m = np.ascontiguousarray(matrix, dtype=np.uint64).reshape(-1)
        if rows < 8 or rows % 8 or cols == 0 or cols & (cols - 1) or m.size != rows * cols:
            raise InvalidInput("invalid PCS hash matrix geometry")
        out = np.empty((cols, 32), np.uint8)
        self._check(self.lib.volta_cuda_hash_fp_columns(self.raw, m.ctypes.data, rows, cols, out.ctypes.data))
        return out

    # ---- X4 extension-field transforms (lib.rs:4761-4780, 5028-5075, 6601-6620) ---------
    def x4b_ntt_fp2(self, coefficients, size: int) -> np.ndarray:
        """size x 2: the X4 Fp2 NTT of the coefficients (x4/ntt.rs:66-122), host form."""
        cf = _as_fp2(coefficients)
        if cf.size == 0 or cf.size > size or not self._pow2(size) or size > 1 << 33:
            raise InvalidInput("invalid X4b Fp2 NTT geometry")
        out = np.empty(size, dtype=FP2)
        self._check(self.lib.volta_cuda_x4b_ntt_fp2(self.raw, cf.ctypes.data, cf.size, size, out.ctypes.data))
        return fp2_as_u64(out)

    def x4_ntt_fp2_device(self, inp: DeviceBuffer, length: int, size: int, out: DeviceBuffer | None = None,
                          in_offset: int = 0, out_offset: int = 0) -> DeviceBuffer:
        """The same transform on resident buffers (MI355X extension); allocates out if absent."""
        if length == 0 or length > size or not self._pow2(size) or size > 1 << 33:
            raise InvalidInput("invalid resident X4 NTT geometry")
        self._region(inp, in_offset, length)
        if out is None:
            out = self.alloc_device(size, FP2)
            self._call_or_free(out, self.lib.volta_mi355x_x4_ntt_fp2_device, inp.id, in_offset, length, size, out.id,
                               out_offset)
            return out
        self._region(out, out_offset, size)
        self._check(self.lib.volta_mi355x_x4_ntt_fp2_device(self.raw, inp.id, in_offset, length, size, out.id,
                                                            out_offset))
        return out

    def x4c_direct_fold_arena_into_arena(self, arena: DeviceBuffer, input_offset_bytes: int, input_len: int,
                                         output_offset_bytes: int, challenge) -> None:
        """Fold the input_len codeword at input_offset_bytes into input_len/2 Fp2 at
        output_offset_bytes of the same arena (lib.rs:5028-5075)."""
        self._own(arena)
        c0, c1 = (int(challenge[0]), int(challenge[1]))
        if input_len < 2 or not self._pow2(input_len) or input_len > 1 << 33 or c0 >= P or c1 >= P:
            raise InvalidInput("invalid X4c direct-fold geometry")
        in_bytes, out_bytes = input_len * 16, input_len // 2 * 16
        for off, nb in ((input_offset_bytes, in_bytes), (output_offset_bytes, out_bytes)):
            if off % 16 or off + nb > arena.nbytes:
                raise InvalidInput("misaligned or out-of-bounds X4c direct-fold region")
        if input_offset_bytes < output_offset_bytes + out_bytes and output_offset_bytes < input_offset_bytes + in_bytes:
            raise InvalidInput("X4c direct-fold input and output overlap")
        self._check(self.lib.volta_cuda_x4c_direct_fold_arena(self.raw, arena.id, input_offset_bytes, input_len,
                                                              output_offset_bytes, c0, c1))

    # ---- pinned host pool and the X4c pinned transfers (lib.rs:4927-5027) -----------------
    def pinned_alloc(self, nbytes: int) -> int:
        out = ctypes.c_uint64()
        self._check(self.lib.volta_cuda_pinned_alloc(self.raw, nbytes, ctypes.byref(out)))
        return out.value

    def pinned_write(self, pinned_id: int, offset_bytes: int, host: np.ndarray) -> None:
        arr = np.ascontiguousarray(host)
        self._check(self.lib.volta_cuda_pinned_write(self.raw, pinned_id, offset_bytes, arr.ctypes.data, arr.nbytes))

    def pinned_wait_ready(self, pinned_id: int) -> None:
        self._check(self.lib.volta_cuda_pinned_wait_ready(self.raw, pinned_id))

    def pinned_free(self, pinned_id: int) -> None:
        self._check(self.lib.volta_cuda_pinned_free(self.raw, pinned_id))

    def x4c_upload_pinned(self, pinned_id: int, pinned_offset_bytes: int, arena: DeviceBuffer,
                          arena_offset_bytes: int, nbytes: int) -> None:
        self._own(arena)
        self._check(self.lib.volta_cuda_x4c_upload_pinned(self.raw, pinned_id, pinned_offset_bytes, arena.id,
                                                          arena_offset_bytes, nbytes))

    def x4c_direct_fold_pinned_tile(self, pinned_id: int, pinned_offset_bytes: int, arena: DeviceBuffer,
                                    output_offset_bytes: int, scratch_offset_bytes: int, input_len: int,
                                    output_start: int, output_count: int, challenge) -> None:
        """Outputs output_start.. of the fold of an input_len codeword from a pinned tile
        holding output_count positive then output_count negative values (lib.rs:4927-4998)."""
        self._own(arena)
        self._check(self.lib.volta_cuda_x4c_direct_fold_pinned_tile(
            self.raw, pinned_id, pinned_offset_bytes, arena.id, output_offset_bytes, scratch_offset_bytes, input_len,
            output_start, output_count, int(challenge[0]), int(challenge[1])))

    def fp2_mobius_inverse_inplace_device(self, values: DeviceBuffer, offset: int = 0, n: int | None = None) -> None:
        """For every index bit, upper += lower (lib.rs:6601-6620)."""
        n = values.len - offset if n is None else n
        if n == 0 or n & (n - 1):
            raise InvalidInput("invalid resident Fp2 Mobius inverse")
        self._region(values, offset, n)
        self._check(self.lib.volta_cuda_fp2_mobius_inverse_inplace_device(self.raw, values.id, offset, n))

    def _call_or_free(self, out: DeviceBuffer, fn, *args) -> None:
        rc = fn(self.raw, *args)
        if rc != 0:
            msg = self.last_error()
            try:
                self.free_device(out)
            except AccelError:
                pass
            raise GpuError(msg or f"status {rc}")
