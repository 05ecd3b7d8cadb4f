"""ctypes wrapper around liboracle.so, the CPU restatement of the reference's
Ligero commit arithmetic.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker.  The product path
(volta-zk_amd/volta_mi355x) never imports this module.

Function-level citations of the reference live in volta_oracle.h/.c.
"""
from __future__ import annotations

import ctypes
import os
import pathlib
import subprocess

import numpy as np

P = 0xFFFF_FFFF_0000_0001
EPS = 0xFFFF_FFFF
FNV_OFFSET = 0xCBF2_9CE4_8422_2325

_HERE = pathlib.Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liboracle.so"

FP2_DTYPE = np.dtype([("c0", "<u8"), ("c1", "<u8")])


class Fp2C(ctypes.Structure):
    _fields_ = [("c0", ctypes.c_uint64), ("c1", ctypes.c_uint64)]


def _stale() -> bool:
    if not _LIB_PATH.exists():
        return True
    built = _LIB_PATH.stat().st_mtime
    return any(p.stat().st_mtime > built for p in _HERE.glob("volta_oracle*.[ch]"))


def build(force: bool = False) -> None:
    """Compile liboracle.so with the committed Makefile (again when a source is newer)."""
    if force or _stale():
        subprocess.run(["make", "-B" if force else "-s", "-C", str(_HERE)], check=True,
                       stdout=subprocess.DEVNULL)


REFERENCE = pathlib.Path("/root/reference")


def build_reference() -> bool:
    """Compile oracle/_ref (the reference's X4 host sources, `make ref`) when
    the reference checkout exists; returns whether it was built."""
    if not (REFERENCE / "cuda" / "volta_x4b.cuh").exists():
        return False
    subprocess.run(["make", "-s", "-B", "-C", str(_HERE), "ref", "REF=" + str(REFERENCE)], check=True,
                   stdout=subprocess.DEVNULL)
    return True


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(_LIB_PATH))
        _declare(_lib)
    return _lib


def _declare(L: ctypes.CDLL) -> None:
    u64, sz, i32 = ctypes.c_uint64, ctypes.c_size_t, ctypes.c_int
    vp = ctypes.c_void_p
    sig = {
        "vo_fp_new": (u64, [u64]),
        "vo_fp_from_i64": (u64, [ctypes.c_int64]),
        "vo_fp_add": (u64, [u64, u64]),
        "vo_fp_sub": (u64, [u64, u64]),
        "vo_fp_neg": (u64, [u64]),
        "vo_fp_mul": (u64, [u64, u64]),
        "vo_fp_pow": (u64, [u64, u64]),
        "vo_fp_inv": (u64, [u64]),
        "vo_fp2_mul": (Fp2C, [Fp2C, Fp2C]),
        "vo_fp2_add": (Fp2C, [Fp2C, Fp2C]),
        "vo_fp2_mul_base": (Fp2C, [Fp2C, u64]),
        "vo_fp_mul_vec": (None, [vp, vp, vp, sz]),
        "vo_fp_add_vec": (None, [vp, vp, vp, sz]),
        "vo_fp_sub_vec": (None, [vp, vp, vp, sz]),
        "vo_root_of_unity": (u64, [ctypes.c_uint32]),
        "vo_ntt_twiddles": (None, [sz, vp]),
        "vo_ntt_forward": (None, [vp, sz, vp]),
        "vo_ntt_encode_batch": (None, [vp, sz, sz, sz, vp, i32]),
        "vo_ntt_forward_batch": (None, [vp, sz, sz, i32]),
        "vo_ntt_inverse_batch": (None, [vp, sz, sz, i32]),
        "vo_pcs_messages": (None, [vp, vp, sz, sz, sz, sz, vp, i32]),
        "vo_pcs_encode_i16": (None, [vp, vp, sz, sz, sz, sz, vp, i32]),
        "vo_pcs_combine_rows": (None, [vp, vp, vp, sz, sz, sz, sz, vp, i32]),
        "vo_combine_rows_fp": (None, [vp, vp, sz, sz, sz, vp, i32]),
        "vo_fp2_powers": (None, [Fp2C, sz, vp]),
        "vo_fp2_add_inplace": (None, [vp, vp, sz]),
        "vo_gather_columns": (None, [vp, sz, sz, vp, sz, vp]),
        "vo_gather_fp2_columns": (None, [vp, sz, sz, vp, sz, vp]),
        "vo_fp_rows": (None, [vp, u64, sz, sz, vp, i32]),
        "vo_fp2_rows_padded": (None, [vp, u64, sz, sz, sz, vp, i32]),
        "vo_raw_u64": (None, [vp, u64, sz, vp]),
        "vo_fnv_u64": (u64, [vp, sz, u64]),
        "vo_fp2_mul_stream": (None, [vp, vp, vp, sz, i32]),
        "vo_fp2_chain": (None, [vp, vp, vp, sz, i32, i32]),
        "vo_eq_rows": (None, [vp, sz, sz, vp]),
        "vo_fp2_row_dots": (None, [vp, sz, vp, sz, sz, sz, vp]),
        "vo_blake3": (None, [vp, sz, vp]),
        "vo_hash_fp_columns": (None, [vp, sz, sz, vp, i32]),
        "vo_hash_fp2_columns": (None, [vp, sz, sz, vp, i32]),
        "vo_merkle_tree": (None, [vp, sz, vp]),
        "vo_merkle_paths": (None, [vp, sz, vp, sz, vp]),
        "vo_merkle_bench_matrix": (None, [sz, sz, vp, i32]),
        "vo_commit_root": (i32, [vp, sz, sz, sz, sz, vp, vp, vp, vp, i32]),
        "vo_fp2_pow": (Fp2C, [Fp2C, u64]),
        "vo_fp2_inv": (Fp2C, [Fp2C]),
        "vo_x4_root_of_unity": (Fp2C, [ctypes.c_uint32]),
        "vo_x4_ntt": (None, [vp, sz, sz, vp]),
        "vo_x4_fold_codeword": (None, [vp, sz, Fp2C, vp]),
        "vo_x4_fold_coefficients": (None, [vp, sz, Fp2C, vp]),
        "vo_fp2_mobius": (None, [vp, sz, i32]),
        "vo_mle_eval_coefficients": (Fp2C, [vp, sz, vp, sz]),
        "vo_mle_eval_table": (Fp2C, [vp, sz, vp, sz]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def cgroup_cpu_quota(path: str = "/sys/fs/cgroup/cpu.max") -> int | None:
    """Whole CPUs granted by the cgroup v2 quota (floor(quota / period)), or
    None without a quota: the count scripts/p7_gpu_pcs_arithmetic.py:52-58 of
    the reference uses for its CPU denominator."""
    try:
        quota, period = open(path).read().split()[:2]
    except (OSError, ValueError):
        return None
    if quota == "max":
        return None
    return max(1, int(quota) // int(period))


def default_threads() -> int:
    """Cores this process may use: the cgroup's CPU quota when one is set,
    else (and never more than) the CPUs of its affinity mask."""
    try:
        affinity = max(1, len(os.sched_getaffinity(0)))
    except AttributeError:  # pragma: no cover
        affinity = os.cpu_count() or 1
    quota = cgroup_cpu_quota()
    return min(quota, affinity) if quota else affinity


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def _fp2_array(a) -> np.ndarray:
    a = np.ascontiguousarray(a)
    if a.dtype == FP2_DTYPE:
        return a
    a = np.ascontiguousarray(a, dtype=np.uint64)
    assert a.shape[-1] == 2
    return a.view(FP2_DTYPE).reshape(a.shape[:-1])


def fp2_to_u64(a: np.ndarray) -> np.ndarray:
    """View an Fp2 array as (..., 2) uint64."""
    return np.ascontiguousarray(a).view(np.uint64).reshape(a.shape + (2,))


# ---- scalar field -----------------------------------------------------------

def fp_new(x: int) -> int: return lib().vo_fp_new(x)
def fp_from_i64(x: int) -> int: return lib().vo_fp_from_i64(x)
def fp_add(a: int, b: int) -> int: return lib().vo_fp_add(a, b)
def fp_sub(a: int, b: int) -> int: return lib().vo_fp_sub(a, b)
def fp_neg(a: int) -> int: return lib().vo_fp_neg(a)
def fp_mul(a: int, b: int) -> int: return lib().vo_fp_mul(a, b)
def fp_pow(a: int, e: int) -> int: return lib().vo_fp_pow(a, e)
def fp_inv(a: int) -> int: return lib().vo_fp_inv(a)


def fp2_mul(a, b):
    r = lib().vo_fp2_mul(Fp2C(*a), Fp2C(*b))
    return (r.c0, r.c1)


def fp2_add(a, b):
    r = lib().vo_fp2_add(Fp2C(*a), Fp2C(*b))
    return (r.c0, r.c1)


def fp2_mul_base(a, x: int):
    r = lib().vo_fp2_mul_base(Fp2C(*a), x)
    return (r.c0, r.c1)


def _vec_op(name: str, a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint64)
    b = np.ascontiguousarray(b, dtype=np.uint64)
    out = np.empty_like(a)
    getattr(lib(), name)(_ptr(a), _ptr(b), _ptr(out), a.size)
    return out


def fp_mul_vec(a, b): return _vec_op("vo_fp_mul_vec", a, b)
def fp_add_vec(a, b): return _vec_op("vo_fp_add_vec", a, b)
def fp_sub_vec(a, b): return _vec_op("vo_fp_sub_vec", a, b)


# ---- NTT ----------------------------------------------------------------------

def root_of_unity(bits: int) -> int:
    return lib().vo_root_of_unity(bits)


def ntt_twiddles(n: int) -> np.ndarray:
    tw = np.empty(max(1, n // 2), dtype=np.uint64)
    lib().vo_ntt_twiddles(n, _ptr(tw))
    return tw[: n // 2]


def ntt_encode_batch(msgs: np.ndarray, n: int, threads: int | None = None) -> np.ndarray:
    msgs = np.ascontiguousarray(msgs, dtype=np.uint64)
    rows, msg_len = msgs.shape
    out = np.empty((rows, n), dtype=np.uint64)
    lib().vo_ntt_encode_batch(_ptr(msgs), rows, msg_len, n, _ptr(out),
                              threads or default_threads())
    return out


def ntt_forward_batch(data: np.ndarray, threads: int | None = None) -> np.ndarray:
    out = np.array(data, dtype=np.uint64, order="C", copy=True)
    rows, n = out.shape
    lib().vo_ntt_forward_batch(_ptr(out), rows, n, threads or default_threads())
    return out


def ntt_inverse_batch(data: np.ndarray, threads: int | None = None) -> np.ndarray:
    out = np.array(data, dtype=np.uint64, order="C", copy=True)
    rows, n = out.shape
    lib().vo_ntt_inverse_batch(_ptr(out), rows, n, threads or default_threads())
    return out


# ---- PCS rows ----------------------------------------------------------------

def _pads_or_dummy(pads, rows, pad):
    if pad == 0:
        return np.zeros(1, dtype=np.uint64)
    pads = np.ascontiguousarray(pads, dtype=np.uint64)
    assert pads.size == rows * pad
    return pads


def pcs_messages(w: np.ndarray, pads, rows: int, cols: int, pad: int, code_len: int,
                 threads: int | None = None) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.int16)
    assert w.size == rows * cols
    p = _pads_or_dummy(pads, rows, pad)
    out = np.empty((rows, code_len), dtype=np.uint64)
    lib().vo_pcs_messages(_ptr(w), _ptr(p), rows, cols, pad, code_len, _ptr(out),
                          threads or default_threads())
    return out


def pcs_encode_i16(w: np.ndarray, pads, rows: int, cols: int, pad: int, code_len: int,
                   threads: int | None = None) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.int16)
    assert w.size == rows * cols
    p = _pads_or_dummy(pads, rows, pad)
    out = np.empty((rows, code_len), dtype=np.uint64)
    lib().vo_pcs_encode_i16(_ptr(w), _ptr(p), rows, cols, pad, code_len, _ptr(out),
                            threads or default_threads())
    return out


def pcs_combine_rows(w: np.ndarray, pads, coeffs, rows: int, cols: int, pad: int,
                     combinations: int, threads: int | None = None) -> np.ndarray:
    """Returns (combinations, cols+pad) Fp2 as a (..., 2) uint64 array."""
    w = np.ascontiguousarray(w, dtype=np.int16)
    p = _pads_or_dummy(pads, rows, pad)
    c = _fp2_array(coeffs).reshape(-1)
    assert c.size == combinations * rows
    out = np.empty((combinations, cols + pad), dtype=FP2_DTYPE)
    lib().vo_pcs_combine_rows(_ptr(w), _ptr(p), _ptr(c), rows, cols, pad, combinations,
                              _ptr(out), threads or default_threads())
    return fp2_to_u64(out)


def combine_rows_fp(msgs: np.ndarray, coeffs, combinations: int,
                    threads: int | None = None) -> np.ndarray:
    msgs = np.ascontiguousarray(msgs, dtype=np.uint64)
    rows, cols = msgs.shape
    c = _fp2_array(coeffs).reshape(-1)
    assert c.size == combinations * rows
    out = np.empty((combinations, cols), dtype=FP2_DTYPE)
    lib().vo_combine_rows_fp(_ptr(msgs), _ptr(c), rows, cols, combinations, _ptr(out),
                             threads or default_threads())
    return fp2_to_u64(out)


def fp2_powers(base, count: int) -> np.ndarray:
    out = np.empty(count, dtype=FP2_DTYPE)
    lib().vo_fp2_powers(Fp2C(*base), count, _ptr(out))
    return fp2_to_u64(out)


def fp2_add_inplace(target: np.ndarray, add: np.ndarray) -> np.ndarray:
    t = _fp2_array(np.array(target, dtype=np.uint64, copy=True)).reshape(-1).copy()
    a = _fp2_array(add).reshape(-1)
    lib().vo_fp2_add_inplace(_ptr(t), _ptr(a), t.size)
    return fp2_to_u64(t)


def gather_columns(m: np.ndarray, idx: np.ndarray) -> np.ndarray:
    m = np.ascontiguousarray(m, dtype=np.uint64)
    idx = np.ascontiguousarray(idx, dtype=np.uint32)
    rows, cols = m.shape
    out = np.empty((idx.size, rows), dtype=np.uint64)
    lib().vo_gather_columns(_ptr(m), rows, cols, _ptr(idx), idx.size, _ptr(out))
    return out


def gather_fp2_columns(m: np.ndarray, idx: np.ndarray) -> np.ndarray:
    mm = _fp2_array(m)
    rows, cols = mm.shape
    idx = np.ascontiguousarray(idx, dtype=np.uint32)
    out = np.empty((idx.size, rows), dtype=FP2_DTYPE)
    lib().vo_gather_fp2_columns(_ptr(mm), rows, cols, _ptr(idx), idx.size, _ptr(out))
    return fp2_to_u64(out)


# ---- FpStream -----------------------------------------------------------------

def _seed(seed) -> np.ndarray:
    s = np.frombuffer(bytes(seed), dtype=np.uint8).copy()
    assert s.size == 32
    return s


def fp_rows(seed, base_domain: int, rows: int, count: int,
            threads: int | None = None) -> np.ndarray:
    s = _seed(seed)
    out = np.empty((rows, count), dtype=np.uint64)
    lib().vo_fp_rows(_ptr(s), base_domain, rows, count, _ptr(out), threads or default_threads())
    return out


def fp2_rows_padded(seed, base_domain: int, rows: int, count: int, padded: int,
                    threads: int | None = None) -> np.ndarray:
    s = _seed(seed)
    out = np.empty((rows, padded), dtype=FP2_DTYPE)
    lib().vo_fp2_rows_padded(_ptr(s), base_domain, rows, count, padded, _ptr(out),
                             threads or default_threads())
    return fp2_to_u64(out)


def raw_u64(seed, domain: int, count: int) -> np.ndarray:
    s = _seed(seed)
    out = np.empty(count, dtype=np.uint64)
    lib().vo_raw_u64(_ptr(s), domain, count, _ptr(out))
    return out


# ---- checksums / spike kernels ---------------------------------------------------

def fnv(values: np.ndarray, h: int = FNV_OFFSET) -> int:
    v = np.ascontiguousarray(values).view(np.uint64).reshape(-1)
    return lib().vo_fnv_u64(_ptr(v), v.size, h)


def fp2_mul_stream(a, b, threads: int | None = None) -> np.ndarray:
    a, b = _fp2_array(a).reshape(-1), _fp2_array(b).reshape(-1)
    out = np.empty_like(a)
    lib().vo_fp2_mul_stream(_ptr(a), _ptr(b), _ptr(out), a.size, threads or default_threads())
    return fp2_to_u64(out)


def fp2_chain(a, b, rounds: int, threads: int | None = None) -> np.ndarray:
    a, b = _fp2_array(a).reshape(-1), _fp2_array(b).reshape(-1)
    out = np.empty_like(a)
    lib().vo_fp2_chain(_ptr(a), _ptr(b), _ptr(out), a.size, rounds,
                       threads or default_threads())
    return fp2_to_u64(out)


# ---- opening-path helpers ------------------------------------------------------------------

def eq_rows(points, rows: int, dims: int) -> np.ndarray:
    """rows x 2^dims x 2: prod_k (bit k of x ? p_k : 1 - p_k) per row."""
    pts = _fp2_array(np.asarray(points, dtype=np.uint64).reshape(rows * dims, 2) if dims else np.zeros((1, 2), np.uint64))
    out = np.zeros(rows << dims, FP2_DTYPE)
    lib().vo_eq_rows(_ptr(pts), rows, dims, _ptr(out))
    return fp2_to_u64(out).reshape(rows, 1 << dims, 2)


def fp2_row_dots(a, a_stride: int, b, b_stride: int, rows: int, length: int) -> np.ndarray:
    """rows x 2: sum_j a[r a_stride + j] b[r b_stride + j]."""
    a, b = _fp2_array(a).reshape(-1), _fp2_array(b).reshape(-1)
    out = np.zeros(rows, FP2_DTYPE)
    lib().vo_fp2_row_dots(_ptr(a), a_stride, _ptr(b), b_stride, rows, length, _ptr(out))
    return fp2_to_u64(out)


# ---- BLAKE3 column leaves and Merkle tree (volta_oracle_blake3.c) ------------------------

def blake3(data: bytes) -> bytes:
    """blake3::hash (blake3 1.8.5, rust/volta-pcs/src/merkle.rs:9-11)."""
    buf = np.frombuffer(bytes(data), dtype=np.uint8).copy() if data else np.zeros(1, np.uint8)
    out = np.zeros(32, np.uint8)
    lib().vo_blake3(_ptr(buf), len(data), _ptr(out))
    return out.tobytes()


def hash_fp_columns(m: np.ndarray, rows: int, cols: int, threads: int | None = None) -> np.ndarray:
    """cols x 32 bytes: blake3 of each column's LE u64 words (ligero.rs:595-614)."""
    m = np.ascontiguousarray(m, dtype=np.uint64).reshape(-1)
    assert m.size == rows * cols
    out = np.zeros((cols, 32), np.uint8)
    lib().vo_hash_fp_columns(_ptr(m), rows, cols, _ptr(out), threads or default_threads())
    return out


def hash_fp2_columns(m, rows: int, cols: int, threads: int | None = None) -> np.ndarray:
    """cols x 32 bytes: blake3 of each column's (c0, c1) LE words."""
    m = _fp2_array(m).reshape(-1)
    assert m.size == rows * cols
    out = np.zeros((cols, 32), np.uint8)
    lib().vo_hash_fp2_columns(_ptr(m), rows, cols, _ptr(out), threads or default_threads())
    return out


def merkle_tree(leaves: np.ndarray) -> np.ndarray:
    """(2n - 1) x 32 bytes, levels from the leaves up, root last (merkle.rs:27-37)."""
    leaves = np.ascontiguousarray(leaves, dtype=np.uint8).reshape(-1, 32)
    n = leaves.shape[0]
    assert n >= 1 and n & (n - 1) == 0
    out = np.zeros((2 * n - 1, 32), np.uint8)
    lib().vo_merkle_tree(_ptr(leaves), n, _ptr(out))
    return out


def merkle_paths(tree: np.ndarray, leaves: int, indices) -> np.ndarray:
    """queries x log2(leaves) x 32 bytes of siblings (merkle.rs:43-51)."""
    tree = np.ascontiguousarray(tree, dtype=np.uint8).reshape(-1, 32)
    idx = np.ascontiguousarray(indices, dtype=np.uint32)
    bits = leaves.bit_length() - 1
    out = np.zeros((idx.size, bits, 32), np.uint8)
    lib().vo_merkle_paths(_ptr(tree), leaves, _ptr(idx), idx.size, _ptr(out))
    return out


def merkle_bench_matrix(rows: int, cols: int, threads: int | None = None) -> np.ndarray:
    """M[i] = (i * 0x9E3779B9 + 17) mod p, the reference's Merkle benchmark input."""
    out = np.zeros(rows * cols, np.uint64)
    lib().vo_merkle_bench_matrix(rows, cols, _ptr(out), threads or default_threads())
    return out


def commit_root(w: np.ndarray, rows: int, cols: int, pad: int, code_len: int, seed: bytes,
                threads: int | None = None, keep: bool = False):
    """The CPU commit (commit_impl, rust/volta-pcs/src/ligero.rs:543-624): pads,
    messages, per-row NTT, blake3 column leaves and the Merkle root.  Returns
    the 32-byte root, or (root, encoded rows x code_len, pads rows x pad) with
    ``keep``."""
    w = np.ascontiguousarray(w, dtype=np.int16).reshape(-1)
    assert w.size == rows * cols
    s = _seed(seed)
    root = np.zeros(32, np.uint8)
    enc = np.zeros((rows, code_len), np.uint64) if keep else None
    pads = np.zeros((rows, max(pad, 1)), np.uint64) if keep else None
    rc = lib().vo_commit_root(_ptr(w), rows, cols, pad, code_len, _ptr(s), _ptr(root),
                              _ptr(enc) if keep else None, _ptr(pads) if keep else None,
                              threads or default_threads())
    if rc != 0:
        raise ValueError("invalid commit geometry")
    if keep:
        return root.tobytes(), enc, pads[:, :pad]
    return root.tobytes()


# ---- X4 extension-field transforms (volta_oracle_x4.c) ----------------------------------

def _c(x) -> Fp2C:
    return Fp2C(int(x[0]), int(x[1]))


def _t(r: Fp2C) -> tuple:
    return (r.c0, r.c1)


def fp2_pow(a, e: int) -> tuple: return _t(lib().vo_fp2_pow(_c(a), e))
def fp2_inv(a) -> tuple: return _t(lib().vo_fp2_inv(_c(a)))


def x4_root_of_unity(bits: int) -> tuple:
    """The X4 domain root of order 2^bits, bits <= 33 (x4/ntt.rs:49-57)."""
    return _t(lib().vo_x4_root_of_unity(bits))


def x4_ntt(coeffs, n: int) -> np.ndarray:
    """n x 2: Fp2NttPlan(n).encode(coeffs) (x4/ntt.rs:66-122)."""
    c = _fp2_array(np.asarray(coeffs, dtype=np.uint64).reshape(-1, 2))
    assert 1 <= c.size <= n and n >= 2 and n & (n - 1) == 0
    out = np.zeros(n, FP2_DTYPE)
    lib().vo_x4_ntt(_ptr(c), c.size, n, _ptr(out))
    return fp2_to_u64(out)


def x4_fold_codeword(values, challenge) -> np.ndarray:
    """n/2 x 2: fold_codeword(values, challenge) (x4/ntt.rs:238-256)."""
    v = _fp2_array(np.asarray(values, dtype=np.uint64).reshape(-1, 2))
    out = np.zeros(v.size // 2, FP2_DTYPE)
    lib().vo_x4_fold_codeword(_ptr(v), v.size, _c(challenge), _ptr(out))
    return fp2_to_u64(out)


def x4_fold_coefficients(coeffs, challenge) -> np.ndarray:
    """n/2 x 2: c[2j] + challenge c[2j+1] (x4/ntt.rs:230-235)."""
    v = _fp2_array(np.asarray(coeffs, dtype=np.uint64).reshape(-1, 2))
    out = np.zeros(v.size // 2, FP2_DTYPE)
    lib().vo_x4_fold_coefficients(_ptr(v), v.size, _c(challenge), _ptr(out))
    return fp2_to_u64(out)


def fp2_mobius(values, inverse: bool) -> np.ndarray:
    """Moebius transform (inverse=False: evaluations -> coefficients) (x4/ntt.rs:147-188)."""
    v = _fp2_array(np.array(values, dtype=np.uint64).reshape(-1, 2))
    lib().vo_fp2_mobius(_ptr(v), v.size, 1 if inverse else 0)
    return fp2_to_u64(v)


def mle_eval_coefficients(coeffs, point) -> tuple:
    c = _fp2_array(np.asarray(coeffs, dtype=np.uint64).reshape(-1, 2))
    pt = _fp2_array(np.asarray(point, dtype=np.uint64).reshape(-1, 2))
    return _t(lib().vo_mle_eval_coefficients(_ptr(c), c.size, _ptr(pt), pt.size))


def mle_eval_table(table, point) -> tuple:
    t = _fp2_array(np.asarray(table, dtype=np.uint64).reshape(-1, 2))
    pt = _fp2_array(np.asarray(point, dtype=np.uint64).reshape(-1, 2))
    return _t(lib().vo_mle_eval_table(_ptr(t), t.size, _ptr(pt), pt.size))
