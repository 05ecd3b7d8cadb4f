#!/usr/bin/env python3
"""Benchmark of the Ligero RS-encode hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c3]

One step = one pass of the hot path over the resident synthetic batch of the
chosen configuration (default C3, the full GPT-2-small weight commit):
RS-encode of every row through the reference's own calls
(volta_cuda_pcs_messages_device then volta_cuda_ntt_fp_batch_device, as
finish_resident_commit makes them; the library encodes straight from the i16
weights) plus the two challenge-power row combinations (Fp2 powers + one
combination pass).  Inputs are resident in HBM before timing starts; outputs
stay resident.

Prints one JSON line: whole-step throughput in codeword Gelem/s, the
roofline of the dominant kernel (the encode) from HIP events recorded by the
library on its own stream, and a CPU baseline (the oracle restatement of the
reference CPU path, OpenMP over the host cores) on the same workload.  After
the timed steps it also times the commit's BLAKE3 column tree over the
resident codewords (`commit_tree`) and the X4 extension-field transforms
(`x4`: the rate-1/8 Fp2 encode NTT, codeword fold, Moebius inverse), each
reported beside `value`, not in it.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import pathlib
import statistics
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "volta-zk_amd"))

METRIC = "Ligero RS-encode Gelem/s (Goldilocks NTT) + % HBM roofline, 1 MI355X"
HBM_PEAK_GBS = 8000.0
WORKLOADS = {
    "c1": "c1: 256 x 2^12 uniform Fp (FpStream rows) -> 2^14 (rate 1/4) + 1 combination of 256 rows",
    "c2": "c2: GPT-2 c_attn 768x2304 i16 packed 1024 x 2^11 -> 2^13 (rate 1/4) + 2 challenge-power combinations",
    "c3": "c3: full GPT-2-small weights 124,439,808 i16 packed 2^16 x 2^11 -> 2^13 (rate 1/4) "
          "+ 2 challenge-power combinations",
    "c4": "c4: 2^15 x 2^12 packed-lane Fp -> 2^15 (rate 1/8)",
    "c5": "c5: 64 x 2^24 uniform Fp, forward + inverse NTT + 64-row combination + 256-column gather",
    "p15": "p15: production layer layout 24,576 x 2^13 i16 + 512 device ChaCha8 pads -> 2^15 (rate 1/4): "
           "pads + fused messages/encode (ligero.rs:468-511, layer_layout.rs:30)",
    "p17": "p17: production layer layout 2,080 x 2^15 i16 + 512 device ChaCha8 pads -> 2^17 (rate 1/4): "
           "pads + fused messages/encode (ligero.rs:468-511, layer_layout.rs:34)",
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Workload:
    """Resident inputs/outputs and one step as raw C-ABI calls (no allocation
    inside a step)."""

    def __init__(self, b, name: str):
        import numpy as np

        from volta_mi355x import FP2
        from volta_mi355x import workloads as W
        self.b, self.lib, self.raw, self.name = b, b.lib, b.raw, name
        cfg = self.cfg = W.CONFIGS[name]
        self.np = np
        rows, n = cfg.rows, cfg.n
        self.bufs = []

        def keep(x):
            self.bufs.append(x)
            return x

        if name in ("c2", "c3"):
            w = W.c3_weights() if name == "c3" else W.c2_weights()
            self.host_w = w
            self.w = keep(b.upload_device(w.reshape(-1)))
            self.pads = keep(b.alloc_device(1, np.uint64))
            self.enc = keep(b.alloc_device(rows * n, np.uint64))
            self.challenges = W.challenges_fp2(f"volta-mi355x/{name}/challenges", cfg.combinations)
            self.coeffs = keep(b.alloc_device(cfg.combinations * rows, FP2))
            self.u = keep(b.alloc_device(cfg.combinations * cfg.msg_len, FP2))
        elif name == "c1":
            self.msgs = keep(b.chacha8_prover_secret_fp_rows_device(W.SEED_C1_ROWS, 0, rows, cfg.msg_len))
            self.enc = keep(b.alloc_device(rows * n, np.uint64))
            ch = W.uniform_fp("volta-mi355x/c1/challenges", rows)
            co = np.zeros((rows, 2), np.uint64)
            co[:, 0] = ch
            self.coeffs = keep(b.alloc_device(rows, FP2))
            b.upload_into(self.coeffs, 0, co.reshape(-1))
            self.u = keep(b.alloc_device(cfg.msg_len, FP2))
        elif name == "c4":
            m = W.c4_messages()
            self.msgs = keep(b.upload_device(m.reshape(-1)))
            del m
            self.enc = keep(b.alloc_device(rows * n, np.uint64))
        elif name in ("p15", "p17"):
            w = W.gaussian_i16(f"volta-mi355x/{name}/weights", rows * cfg.msg_len)
            self.w = keep(b.upload_device(w))
            del w
            self.pads = keep(b.alloc_device(rows * cfg.pad, np.uint64))
            self.enc = keep(b.alloc_device(rows * n, np.uint64))
            self.seed = (__import__("ctypes").c_uint8 * 32).from_buffer_copy(W.seed_bytes(f"volta-mi355x/{name}/pads"))
        elif name == "c5":
            x = W.c5_rows()
            self.msgs = keep(b.upload_device(x.reshape(-1)))
            del x
            self.enc = keep(b.alloc_device(rows * n, np.uint64))
            self.back = keep(b.alloc_device(rows * n, np.uint64))
            self.challenges = W.challenges_fp2("volta-mi355x/c5/challenges", 1)
            self.coeffs = keep(b.alloc_device(rows, FP2))
            self.u = keep(b.alloc_device(n, FP2))
            q = W.c5_query_columns(n, 256)
            self.idx = keep(b.upload_device(q))
            self.cols_out = keep(b.alloc_device(rows * 256, np.uint64))
        else:
            raise SystemExit(f"unknown config {name}")

    def _ok(self, rc):
        if rc != 0:
            raise RuntimeError(self.b.last_error())

    def messages_buffer(self, nbytes: int) -> int:
        """A new resident buffer as Backend::pcs_messages_device allocates one
        per call (after the first step it reuses the freed storage)."""
        out = ctypes.c_uint64()
        self._ok(self.lib.volta_cuda_resident_alloc(self.raw, nbytes, ctypes.byref(out)))
        return out.value

    def step(self):
        L, r, cfg = self.lib, self.raw, self.cfg
        rows, n = cfg.rows, cfg.n
        if self.name in ("c2", "c3"):
            # the reference's commit calls (ligero.rs:477-496): message rows
            # into a new buffer, the batched NTT of those rows (encoded from
            # the weights), the rows freed
            m = self.messages_buffer(rows * n * 8)
            self._ok(L.volta_cuda_pcs_messages_device(r, self.w.id, 0, self.pads.id, 0, rows, cfg.msg_len, 0, n, m, 0))
            self._ok(L.volta_cuda_ntt_fp_batch_device(r, m, 0, rows, n, self.enc.id, 0))
            self._ok(L.volta_cuda_resident_free(r, m))
            for k, c in enumerate(self.challenges):
                self._ok(L.volta_cuda_fp2_powers_device(r, int(c[0]), int(c[1]), self.coeffs.id, k * rows, rows))
            self._ok(L.volta_cuda_pcs_combine_rows_device(r, self.w.id, 0, self.pads.id, 0, self.coeffs.id, 0, rows,
                                                          cfg.msg_len, 0, cfg.combinations, self.u.id, 0))
        elif self.name == "c1":
            self._ok(L.volta_mi355x_ntt_fp_encode_device(r, self.msgs.id, 0, rows, cfg.msg_len, n, self.enc.id, 0))
            self._ok(L.volta_mi355x_combine_rows_fp_device(r, self.msgs.id, 0, rows, cfg.msg_len, self.coeffs.id, 0,
                                                           1, self.u.id, 0))
        elif self.name == "c4":
            self._ok(L.volta_mi355x_ntt_fp_encode_device(r, self.msgs.id, 0, rows, cfg.msg_len, n, self.enc.id, 0))
        elif self.name in ("p15", "p17"):
            # the resident commit's calls (ligero.rs:474-496): pads, message rows
            # lift(w) || pads || 0, then their NTT (encoded from the sources)
            self._ok(L.volta_cuda_chacha8_prover_secret_fp_rows_device(r, self.pads.id, 0, self.seed, 0, rows,
                                                                       cfg.pad))
            m = self.messages_buffer(rows * n * 8)
            self._ok(L.volta_cuda_pcs_messages_device(r, self.w.id, 0, self.pads.id, 0, rows, cfg.msg_len, cfg.pad,
                                                      n, m, 0))
            self._ok(L.volta_cuda_ntt_fp_batch_device(r, m, 0, rows, n, self.enc.id, 0))
            self._ok(L.volta_cuda_resident_free(r, m))
        elif self.name == "c5":
            self._ok(L.volta_cuda_ntt_fp_batch_device(r, self.msgs.id, 0, rows, n, self.enc.id, 0))
            self._ok(L.volta_mi355x_ntt_fp_inverse_batch_device(r, self.enc.id, 0, rows, n, self.back.id, 0))
            c = self.challenges[0]
            self._ok(L.volta_cuda_fp2_powers_device(r, int(c[0]), int(c[1]), self.coeffs.id, 0, rows))
            self._ok(L.volta_mi355x_combine_rows_fp_device(r, self.enc.id, 0, rows, n, self.coeffs.id, 0, 1,
                                                           self.u.id, 0))
            self._ok(L.volta_cuda_pcs_gather_columns_device(r, self.enc.id, 0, rows, n, self.idx.id, 0, 256,
                                                            self.cols_out.id, 0, 0))

    def elements_per_step(self) -> int:
        # codeword elements produced (C5 counts forward and inverse outputs)
        return self.cfg.elements * (2 if self.name == "c5" else 1)

    def close(self):
        for x in reversed(self.bufs):
            self.b.free_device(x)


def copy_bandwidth(b, nbytes: int = 1 << 32, reps: int = 10) -> float:
    """Achievable HBM bandwidth from a 16-byte streaming copy (read+write)."""
    import numpy as np
    src = b.alloc_device(nbytes // 8, np.uint64)
    dst = b.alloc_device(nbytes // 8, np.uint64)
    b.zero_device(src, 0, nbytes // 8)
    L, r = b.lib, b.raw
    L.volta_mi355x_probe_copy_device(r, src.id, dst.id, nbytes)
    b.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        if L.volta_mi355x_probe_copy_device(r, src.id, dst.id, nbytes) != 0:
            raise RuntimeError(b.last_error())
    b.synchronize()
    dt = (time.perf_counter() - t0) / reps
    b.free_device(src)
    b.free_device(dst)
    return 2 * nbytes / dt / 1e9


def expand_bandwidth(b, src_bytes: int = 1 << 28, reps: int = 20) -> float:
    """Achievable HBM bandwidth for the encode's traffic shape: src_bytes read,
    16 x src_bytes written with the encode's 8-byte non-temporal stores
    (C3's 256 MiB of i16 in, 4 GiB of codewords out)."""
    import numpy as np
    src = b.alloc_device(src_bytes // 8, np.uint64)
    dst = b.alloc_device(src_bytes * 2, np.uint64)
    b.zero_device(src, 0, src_bytes // 8)
    L, r = b.lib, b.raw
    b._check(L.volta_mi355x_probe_expand_device(r, src.id, dst.id, src_bytes))
    b.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        b._check(L.volta_mi355x_probe_expand_device(r, src.id, dst.id, src_bytes))
    b.synchronize()
    dt = (time.perf_counter() - t0) / reps
    b.free_device(src)
    b.free_device(dst)
    return 17 * src_bytes / dt / 1e9


def seam_chain(b, wl: "Workload", reps: int = 10) -> dict | None:
    """The reference's unchanged commit calls (finish_resident_commit,
    ligero.rs:477-496): volta_cuda_pcs_messages_device then
    volta_cuda_ntt_fp_batch_device on the message rows, timed per chain with
    the library's HIP events after the timed steps (not part of `value`).
    `fused`: the calls as Rust makes them, the rows' buffer allocated before
    and freed after (the rows stay unwritten and the transform encodes from
    the weights); `written`: the same calls with the rows forced into HBM
    before the transform by a device-pointer query of their buffer (the
    caller may then write the rows itself, so the transform reads them whole:
    the chain without the deferral); `written_read_back`: the rows forced into
    HBM by reading 8 bytes of them back (the library wrote them and nothing
    else has, so the transform reads only their nonzero part)."""
    import numpy as np
    if wl.name not in ("c2", "c3"):
        return None
    cfg = wl.cfg
    rows, n = cfg.rows, cfg.n
    L, r = b.lib, b.raw

    probe = np.empty(1, np.uint64)

    def chain(force):
        m = wl.messages_buffer(rows * n * 8)
        wl._ok(L.volta_cuda_pcs_messages_device(r, wl.w.id, 0, wl.pads.id, 0, rows, cfg.msg_len, 0, n, m, 0))
        if force == "written":
            p = ctypes.c_void_p()
            wl._ok(L.volta_mi355x_resident_device_ptr(r, m, 0, 8, ctypes.byref(p)))
        elif force == "written_read_back":
            wl._ok(L.volta_cuda_resident_download(r, m, 0, probe.ctypes.data, 8))
        wl._ok(L.volta_cuda_ntt_fp_batch_device(r, m, 0, rows, n, wl.enc.id, 0))
        wl._ok(L.volta_cuda_resident_free(r, m))

    out = {"calls": "volta_cuda_pcs_messages_device + volta_cuda_ntt_fp_batch_device", "rows": rows,
           "code_len": n, "algorithmic_bytes": cfg.algorithmic_bytes, "reps": reps}
    for force in ("fused", "written", "written_read_back"):
        for _ in range(2):
            chain(force)
        b.synchronize()
        b.reset_stats()
        t0 = time.perf_counter()
        for _ in range(reps):
            chain(force)
        b.synchronize()
        wall = (time.perf_counter() - t0) / reps
        s = b.get_stats()
        ntt_ms = s["kernel_ns"]["pcs_ntt"] / reps / 1e6
        out[force] = {"ms_per_chain": round(wall * 1e3, 4), "ntt_call_ms": round(ntt_ms, 4),
                    "messages_call_ms": round(s["kernel_ns"]["pcs_rows"] / reps / 1e6, 4),
                    "achieved_gbs": round(cfg.algorithmic_bytes / wall / 1e9, 1),
                    "frac_of_peak": round(cfg.algorithmic_bytes / wall / 1e9 / HBM_PEAK_GBS, 4)}
    return out


FNV_OFFSET = 0xCBF29CE484222325


def published_shapes(b, reps: int = 10) -> dict:
    """The two shapes on this path for which the reference publishes GPU
    times (benchmarks/results/p7-gpu-pcs-arithmetic-2026-07-11-366ec4a.json,
    A100), with the reference's own inputs and output checksums, timed with
    the library's HIP events (not part of `value`):
    - P4_LAYER NTT (cuda/p7_pcs_arithmetic.cu:201-263): 1024 rows x 2^15,
      in[idx] = (idx 0x9E3779B9 + 17) mod p for column j < 16896, else 0,
      through volta_cuda_ntt_fp_batch_device on the pre-padded rows; checksum
      0xbe7b90425a4c7229 over all outputs;
    - the two-combination (:265-320): 1024 x 16384 u64 rows w[i] = (i
      0x85EBCA6B + 29) mod p, coefficient rows q[i] = (37i+11, 53i+5) and c[i]
      = (71i+7, 97i+13); checksum cs(uq) ^ cs(uc) 0x9E3779B97F4A7C15 =
      0x856f9a96d8e01901.
    Each checksum is recomputed from the device output of this run and must
    match, or the leg raises."""
    import numpy as np
    from volta_mi355x import FP2
    P = np.uint64(0xFFFF_FFFF_0000_0001)
    L, r = b.lib, b.raw
    mask = (1 << 64) - 1

    def fnv(a):
        a = np.ascontiguousarray(a).view(np.uint64).reshape(-1)
        return int(L.volta_mi355x_fnv64_host(a.ctypes.data, a.size, FNV_OFFSET))

    def timed(op, call):
        for _ in range(2):
            b._check(call())
        b.synchronize()
        b.reset_stats()
        t0 = time.perf_counter()
        for _ in range(reps):
            b._check(call())
        b.synchronize()
        wall = (time.perf_counter() - t0) / reps
        s = b.get_stats()
        return s["kernel_ns"][op] / max(s["calls"][op], 1) / 1e6, wall * 1e3

    out = {"source": "benchmarks/results/p7-gpu-pcs-arithmetic-2026-07-11-366ec4a.json (A100-SXM4-80GB)",
           "reps": reps}
    rows, n, msg_len = 1024, 1 << 15, 16896
    idx = np.arange(rows * n, dtype=np.uint64)
    x = ((idx * np.uint64(0x9E3779B9) + np.uint64(17)) % P).reshape(rows, n)
    x[:, msg_len:] = 0
    din = b.upload_device(x.reshape(-1))
    del x, idx
    dout = b.alloc_device(rows * n, np.uint64)
    ms, wall = timed("pcs_ntt", lambda: L.volta_cuda_ntt_fp_batch_device(r, din.id, 0, rows, n, dout.id, 0))
    cs = fnv(b.download_device(dout))
    for d in (din, dout):
        b.free_device(d)
    if cs != 0xBE7B90425A4C7229:
        raise RuntimeError(f"P4_LAYER NTT checksum {cs:#018x} != 0xbe7b90425a4c7229")
    io = 2 * rows * n * 8
    out["p4_layer_ntt"] = {
        "call": "volta_cuda_ntt_fp_batch_device", "rows": rows, "n": n, "msg_len": msg_len,
        "ms": round(ms, 4), "wall_ms_per_call": round(wall, 4), "gelem_per_s": round(rows * n / ms / 1e6, 2),
        "read_write_bytes": io, "achieved_gbs": round(io / ms / 1e6, 1),
        "checksum": f"{cs:#018x}", "checksum_expected": "0xbe7b90425a4c7229",
        "reference_a100_ms": 6.386, "reference_a100_gelem_per_s": 5.25, "speedup_vs_reference_a100": round(6.386 / ms, 1)}

    rows, cols = 1024, 16384
    i = np.arange(rows * cols, dtype=np.uint64)
    w = (i * np.uint64(0x85EBCA6B) + np.uint64(29)) % P
    del i
    k = np.arange(rows, dtype=np.uint64)
    q = np.stack([(k * np.uint64(37) + np.uint64(11)) % P, (k * np.uint64(53) + np.uint64(5)) % P], 1)
    c = np.stack([(k * np.uint64(71) + np.uint64(7)) % P, (k * np.uint64(97) + np.uint64(13)) % P], 1)
    dm = b.upload_device(w)
    dc = b.alloc_device(2 * rows, FP2)
    b.upload_into(dc, 0, np.concatenate([q, c]).reshape(-1))
    du = b.alloc_device(2 * cols, FP2)
    ms, wall = timed("pcs_rows", lambda: L.volta_mi355x_combine_rows_fp_device(r, dm.id, 0, rows, cols, dc.id, 0, 2,
                                                                              du.id, 0))
    u = b.download_device(du).view(np.uint64).reshape(2, cols, 2)
    for d in (dm, dc, du):
        b.free_device(d)
    cs = fnv(u[0]) ^ ((fnv(u[1]) * 0x9E3779B97F4A7C15) & mask)
    if cs != 0x856F9A96D8E01901:
        raise RuntimeError(f"combination checksum {cs:#018x} != 0x856f9a96d8e01901")
    rd = rows * cols * 8
    out["two_combination"] = {
        "call": "volta_mi355x_combine_rows_fp_device (u64 rows, 2 Fp2 coefficient rows)", "rows": rows,
        "cols": cols, "ms": round(ms, 4), "wall_ms_per_call": round(wall, 4),
        "g_weight_elem_per_s": round(rows * cols / ms / 1e6, 2), "read_bytes": rd,
        "achieved_gbs": round(rd / ms / 1e6, 1), "checksum": f"{cs:#018x}",
        "checksum_expected": "0x856f9a96d8e01901", "reference_a100_ms": 1.918,
        "speedup_vs_reference_a100": round(1.918 / ms, 1)}
    return out


def host_batch(b, wl: "Workload", reps: int = 3) -> dict | None:
    """The hybrid commit's transform (rust/volta-pcs/src/ligero.rs:564-581 ->
    Backend::ntt_fp_batch, rust/volta-accel/src/lib.rs:4722-4746): compact
    host rows lift(w) of msg_len u64 in, rows x n codewords back to host
    memory, through volta_cuda_ntt_fp_batch at the workload's shape.  Timed
    with the library's events (kernel, upload, download) and the wall clock
    around the call; the codewords must equal the resident encode's of the
    same weights (sampled rows), or the leg raises.  Not part of `value`."""
    import numpy as np
    if wl.name not in ("c2", "c3"):
        return None
    cfg = wl.cfg
    rows, n, m = cfg.rows, cfg.n, cfg.msg_len
    w = wl.host_w.reshape(rows, m)
    # Fp::from_i64 (rust/volta-field/src/lib.rs:32-40): x < 0 -> p - |x| = (2^64 + x) - (2^32 - 1)
    msgs = w.astype(np.int64).astype(np.uint64)
    neg = w < 0
    msgs[neg] -= np.uint64(0xFFFF_FFFF)
    del neg
    out = np.empty((rows, n), np.uint64)
    L, r = b.lib, b.raw
    call = lambda: b._check(L.volta_cuda_ntt_fp_batch(r, msgs.ctypes.data, rows, m, n, out.ctypes.data))
    call()
    b.reset_stats()
    walls = []
    for _ in range(reps):
        t0 = time.perf_counter()
        call()
        walls.append(time.perf_counter() - t0)
    s = b.get_stats()
    pick = [0, rows // 3, rows - 1]
    ref = np.stack([b.download_device(wl.enc, i * n, n) for i in pick])
    if not (out[pick] == ref).all():
        raise RuntimeError("host batch NTT differs from the resident encode of the same weights")
    kern = s["kernel_ns"]["pcs_ntt"] / reps / 1e6
    return {"call": "volta_cuda_ntt_fp_batch (compact host rows lift(w), msg_len per row)", "rows": rows,
            "msg_len": m, "n": n, "reps": reps, "kernel_ms": round(kern, 4),
            "h2d_ms": round(s["h2d_ns"] / reps / 1e6, 3), "d2h_ms": round(s["d2h_ns"] / reps / 1e6, 3),
            "wall_ms_per_call": round(statistics.median(walls) * 1e3, 2),
            "kernel_gelem_per_s": round(rows * n / kern / 1e6, 1),
            "note": "the wall time holds the PCIe copies of 8 B per message element in and 8 B per codeword "
                    "element out to pageable host memory"}


def fp2_chain_peak(b, log_n: int = 20, rounds: int = 256, reps: int = 10) -> dict:
    """Integer multiply peak from the reference's Fp2 chain kernel
    (cuda/p7_goldilocks_roofline.cu:79-89: x = x*b + (j+1, 2j+3), `rounds`
    times per element; its output checksum is pinned by the GPU tests), at the
    reference's own configuration 2^20 x 256.  One Fp2 multiply counts as 5
    base multiplies, the reference's convention (`fp_mul_per_fp2_mul`)."""
    import numpy as np
    from volta_mi355x import FP2
    n = 1 << log_n
    g = np.random.Generator(np.random.PCG64(5))
    a = b.upload_device(g.integers(0, 0xFFFF_FFFF_0000_0001, size=(n, 2), dtype=np.uint64), FP2)
    c = b.upload_device(g.integers(0, 0xFFFF_FFFF_0000_0001, size=(n, 2), dtype=np.uint64), FP2)
    out = b.alloc_device(n, FP2)
    L, r = b.lib, b.raw
    b._check(L.volta_mi355x_probe_fp2_device(r, a.id, c.id, out.id, n, rounds))
    b.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        b._check(L.volta_mi355x_probe_fp2_device(r, a.id, c.id, out.id, n, rounds))
    b.synchronize()
    dt = (time.perf_counter() - t0) / reps
    for x in (a, c, out):
        b.free_device(x)
    ops = n * rounds / dt
    return {"probe": "Fp2 multiply-add chain (p7_goldilocks_roofline.cu:79-89)", "elements": n, "rounds": rounds,
            "ms": round(dt * 1e3, 4), "fp2_mul_per_s": round(ops), "base_mul_equiv_per_s": round(5 * ops),
            "reference_a100_fp2_mul_per_s": 41180802646.5}


def commit_tree(b, wl: Workload, reps: int = 10) -> dict:
    """BLAKE3 column leaves + Merkle tree over the step's resident codeword
    matrix (the reference commit's last stage, ligero.rs:595-621), timed with
    the library's own HIP events after the timed steps; not part of `value`."""
    import numpy as np
    rows, n = wl.cfg.rows, wl.cfg.n
    tree = b.alloc_device((2 * n - 1) * 32, np.uint8)
    call = lambda: wl._ok(wl.lib.volta_cuda_hash_fp_tree_device(wl.raw, wl.enc.id, 0, rows, n, tree.id, 0))
    for _ in range(2):
        call()
    b.synchronize()
    b.reset_stats()
    for _ in range(reps):
        call()
    b.synchronize()
    s = b.get_stats()
    b.free_device(tree)
    ms = s["kernel_ns"]["pcs_merkle"] / max(s["calls"]["pcs_merkle"], 1) / 1e6
    matrix = rows * n * 8
    return {"kernel": "BLAKE3 column leaves + Merkle tree (volta_cuda_hash_fp_tree_device)",
            "rows": rows, "leaves": n, "ms_per_tree": round(ms, 4), "matrix_bytes": matrix,
            "achieved_gbs": round(matrix / ms / 1e6, 1), "reps": reps}


# The reference's two production commitments and its A100 times for them
# (benchmarks/results/c3-table-a100-2026-07-17-5a2edbe.json, pcs_commitments[0|1].commit_s).
# name, rows, col_bits, pad, code_bits, pad-seed byte, commit_s, open_s, claims per tensor
REFERENCE_COMMITS = (
    ("weights", 24576, 13, 512, 15, 0x51, 0.148233502, 0.266512943, (2,) * 48),
    ("embed", 2080, 15, 512, 17, 0x52, 0.05474647, 0.027055026, (4, 2)),
)


def reference_commits(reps: int = 5) -> dict:
    """C3_WEIGHTS and C3_EMBED committed as the reference's report commits
    them (rust/volta-bench/src/bin/p6_report.rs:2584-2635, 2929-2972): the
    layouts' tensors resident as separate buffers, then
    commit_resident_from_device with one strided placement per tensor (48 for
    the weights, wte and wpe for the embedding) -- zero the packed target,
    place, ChaCha8 pads, messages, NTT, BLAKE3 column tree, root read back.
    Then the device side of the resident opening (open_multi_zk_resident,
    ligero.rs:1216-1551) with as many block claims as the report makes (96 =
    two per weight tensor; 6 = four on wte, two on wpe, model_proof.rs:2185,
    2366-2367), random claim points and 120 queries: masks and their tree,
    the proximity pass, the block-claim pass, the mask dots, the query
    columns and paths, all read back.  Wall time around each call, median of
    `reps` after one warm-up, next to the reference's A100 times for the same
    commitment and opening (not part of `value`; the reference's opening time
    also holds its transcript and proof assembly on the host).  A context of
    its own with the report's timing policy, wall-only counters (the result
    file's resident_timing_policy): no timing events around each call."""
    import numpy as np

    from volta_mi355x import Backend, ligero
    from volta_mi355x import workloads as W
    b = Backend(timing_policy=1)
    P = W.P
    _pow2 = W._pow2
    out = {}
    for name, rows, col_bits, pad, code_bits, seed_byte, ref_s, ref_open_s, per_tensor in REFERENCE_COMMITS:
        slots, total = W.c3_weights_slots() if name == "weights" else W.c3_embed_slots()
        params = ligero.LigeroParams(rows=rows, col_bits=col_bits, pad=pad, code_bits=code_bits)
        assert total == params.rows * params.cols
        sources = [b.upload_device(W.slot_tensor(f"volta-mi355x/{name}", s_).reshape(-1)) for s_ in slots]
        placements = [ligero.ResidentWeightPlacement(src, 0, s_.k, s_.n, s_.offset, s_.stride, total)
                      for src, s_ in zip(sources, slots)]
        times, root, pm = [], b"", None
        for i in range(reps + 1):
            if pm is not None:
                ligero.free_resident_matrix(b, pm)
            b.synchronize()
            t0 = time.perf_counter()
            root, pm = ligero.commit_resident_from_device(b, placements, params, bytes([seed_byte]) * 32)
            dt = time.perf_counter() - t0
            if i:
                times.append(dt)
        for src in sources:
            b.free_device(src)
        t = statistics.median(times)
        g = np.random.Generator(np.random.PCG64(rows))
        claims = [(s_.offset, g.integers(0, P, size=((_pow2(s_.k) * _pow2(s_.n)).bit_length() - 1, 2),
                                         dtype=np.uint64))
                  for s_, count in zip(slots, per_tensor) for _ in range(count)]
        c = tuple(int(x) for x in g.integers(0, P, size=2, dtype=np.uint64))
        js = g.integers(0, params.code_len, size=120, dtype=np.uint32)
        open_times = []
        for i in range(reps + 1):
            b.synchronize()
            t0 = time.perf_counter()
            ligero.open_rows_resident(b, pm, claims, c, js, bytes([seed_byte ^ 0xFF]) * 32)
            dt = time.perf_counter() - t0
            if i:
                open_times.append(dt)
        ligero.free_resident_matrix(b, pm)
        to = statistics.median(open_times)
        out[name] = {"rows": rows, "cols": params.cols, "pad": pad, "code_len": params.code_len,
                     "tensors": len(slots), "ms_per_commit": round(t * 1e3, 3),
                     "gelem_per_s": round(rows * params.code_len / t / 1e9, 2), "root": root.hex(),
                     "reference_a100_ms": round(ref_s * 1e3, 2), "speedup_vs_reference_a100": round(ref_s / t, 1),
                     "claims": len(claims), "queries": 120, "ms_per_open": round(to * 1e3, 3),
                     "reference_a100_open_ms": round(ref_open_s * 1e3, 2),
                     "open_speedup_vs_reference_a100": round(ref_open_s / to, 1)}
    b.close()
    out["reference_source"] = ("benchmarks/results/c3-table-a100-2026-07-17-5a2edbe.json pcs_commitments[].commit_s, "
                               "open_s (resident_timing_policy wall-only-counters)")
    out["timing_policy"] = "wall-only counters"
    out["reps"] = reps
    return out


def x4_transforms(b, log_n: int = 24, reps: int = 10) -> dict:
    """The X4 extension-field transforms (not part of `value`): the rate-1/8
    encode NTT of 2^(log_n - 3) Fp2 coefficients into 2^log_n points
    (encode_rate_eighth, rust/volta-pcs/src/x4/ntt.rs:124-130), the fold of that
    codeword (ntt.rs:238-256) and the Moebius inverse of 2^(log_n - 3) values,
    each timed with the library's HIP events.  Algorithmic bytes: the NTT reads
    the coefficients and writes the codeword once (16 B per element), the fold
    reads n and writes n/2 elements, the Moebius reads and writes its table."""
    import numpy as np
    from volta_mi355x import FP2
    n, m = 1 << log_n, 1 << (log_n - 3)
    g = np.random.Generator(np.random.PCG64(33))
    coeffs = b.upload_device(g.integers(0, 0xFFFF_FFFF_0000_0001, size=(m, 2), dtype=np.uint64), FP2)
    arena = b.alloc_device(n + n // 2, FP2)
    table = b.upload_device(g.integers(0, 0xFFFF_FFFF_0000_0001, size=(m, 2), dtype=np.uint64), FP2)
    lib, raw = b.lib, b.raw

    def timed(op, call):
        for _ in range(2):
            b._check(call())
        b.synchronize()
        b.reset_stats()
        for _ in range(reps):
            b._check(call())
        b.synchronize()
        s = b.get_stats()
        return s["kernel_ns"][op] / max(s["calls"][op], 1) / 1e6

    ntt_ms = timed("pcs_ntt", lambda: lib.volta_mi355x_x4_ntt_fp2_device(raw, coeffs.id, 0, m, n, arena.id, 0))
    fold_ms = timed("pcs_rows", lambda: lib.volta_cuda_x4c_direct_fold_arena(raw, arena.id, 0, n, n * 16, 12345,
                                                                             678))
    mob_ms = timed("pcs_rows", lambda: lib.volta_cuda_fp2_mobius_inverse_inplace_device(raw, table.id, 0, m))
    for x in (coeffs, arena, table):
        b.free_device(x)
    ntt_bytes, fold_bytes, mob_bytes = 16 * (m + n), 16 * (n + n // 2), 32 * m
    passes = 1 if log_n <= 12 else 2 if log_n <= 20 else 3 if log_n <= 30 else 4
    return {
        "ntt": {"kernel": "volta_mi355x_x4_ntt_fp2_device (gather + column passes)", "coefficients": m,
                "points": n, "passes": passes, "ms": round(ntt_ms, 4), "algorithmic_bytes": ntt_bytes,
                "pass_bytes": 16 * m + 16 * n + (passes - 1) * 32 * n,
                "achieved_gbs": round(ntt_bytes / ntt_ms / 1e6, 1)},
        "fold": {"kernel": "volta_cuda_x4c_direct_fold_arena", "input_len": n, "ms": round(fold_ms, 4),
                 "algorithmic_bytes": fold_bytes, "achieved_gbs": round(fold_bytes / fold_ms / 1e6, 1)},
        "mobius_inverse": {"kernel": "volta_cuda_fp2_mobius_inverse_inplace_device", "n": m,
                           "ms": round(mob_ms, 4), "algorithmic_bytes": mob_bytes,
                           "achieved_gbs": round(mob_bytes / mob_ms / 1e6, 1)},
        "reps": reps,
    }


def cpu_baseline(name: str, wl: Workload) -> dict:
    """The oracle's restatement of the reference CPU path (per-row radix-2 DIT
    NttPlan::forward, combine_rows with its column chunks), OpenMP over this
    host's cores, on a bounded sample of the configuration's rows (about 6 s a
    run): the same step as the GPU's over those rows, median of 3 after one
    warm-up, scaled to codeword elements per second.  C5 times its forward and
    inverse transforms and the combination over a subset of its rows, one
    2^24-point transform per core, twice."""
    import numpy as np
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle
    oracle.build()
    from volta_mi355x import workloads as W
    cfg = W.CONFIGS[name]
    threads = oracle.default_threads()
    rows_all, n = cfg.rows, cfg.n

    if name in ("c2", "c3"):
        w = wl.host_w
        co = np.concatenate([oracle.fp2_powers(tuple(int(x) for x in c), cfg.rows) for c in wl.challenges])

        def run(rows):
            oracle.pcs_encode_i16(w[:rows].reshape(-1), None, rows, cfg.msg_len, 0, n, threads)
            cr = np.concatenate([co[k * cfg.rows:k * cfg.rows + rows] for k in range(cfg.combinations)])
            oracle.pcs_combine_rows(w[:rows].reshape(-1), None, cr, rows, cfg.msg_len, 0, cfg.combinations, threads)
        step = f"encode + {cfg.combinations} combinations"
    elif name == "c1":
        msgs = wl.b.download_device(wl.msgs).reshape(rows_all, cfg.msg_len)
        co = np.zeros((rows_all, 2), np.uint64)
        co[:, 0] = W.uniform_fp("volta-mi355x/c1/challenges", rows_all)

        def run(rows):
            oracle.ntt_encode_batch(msgs[:rows], n, threads)
            oracle.combine_rows_fp(msgs[:rows], co[:rows], 1, threads)
        step = "encode + 1 combination"
    elif name == "c4":
        cache = {}

        def run(rows):
            if rows not in cache:
                cache[rows] = W.c4_messages(rows, cfg.msg_len)
            oracle.ntt_encode_batch(cache[rows], n, threads)
        step = "encode"
    elif name in ("p15", "p17"):
        cache = {}
        seed = W.seed_bytes(f"volta-mi355x/{name}/pads")

        def run(rows):
            if rows not in cache:
                cache[rows] = W.gaussian_i16(f"volta-mi355x/{name}/weights", rows * cfg.msg_len)
            pads = oracle.fp_rows(seed, 0, rows, cfg.pad, threads)
            oracle.pcs_encode_i16(cache[rows], pads, rows, cfg.msg_len, cfg.pad, n, threads)
        step = "pads + encode"
    elif name == "c5":
        sample = min(rows_all, max(threads, 1))
        x = W.c5_rows(sample, n)
        c = tuple(int(v) for v in wl.challenges[0])
        t_all = []
        for _ in range(2):  # each run is tens of seconds: two runs, no warm-up
            t0 = time.perf_counter()
            fwd = oracle.ntt_forward_batch(x, threads)
            oracle.ntt_inverse_batch(fwd, threads)
            oracle.combine_rows_fp(fwd, oracle.fp2_powers(c, sample), 1, threads)
            t_all.append(time.perf_counter() - t0)
        t = statistics.median(t_all)
        return {"value": round(2 * sample * n / t / 1e9, 4), "unit": "Gelem/s", "cores": threads,
                "cores_counted": cpu_cores_note(threads), "cpu_model": cpu_model(), "kind": "port",
                "sample": f"{sample} of {rows_all} rows of c5 (forward + inverse + the combination over those rows; "
                          f"elements counted both ways as the GPU's), mean of 2 runs without warm-up, {t:.3f} s"}
    else:
        return None

    probe = min(rows_all, 256 if n >= 1 << 15 else 1024)
    t0 = time.perf_counter()
    run(probe)
    per_row = (time.perf_counter() - t0) / probe
    # bounded sample: about 6 s a run
    sample = int(min(rows_all, max(probe, 6.0 / max(per_row, 1e-9))))
    sample -= sample % probe
    sample = max(sample, probe)
    run(sample)  # warm-up at the sample's size
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        run(sample)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    return {
        "value": round(sample * n / t / 1e9, 4),
        "unit": "Gelem/s",
        "cores": threads,
        "cores_counted": cpu_cores_note(threads),
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": f"{sample} of {rows_all} rows of {name} ({step} over those rows), median of 3 after 1 warmup, "
                  f"{t:.3f} s",
    }


def cpu_model() -> str:
    """The host CPU as /proc/cpuinfo names it: model name, then vendor, family,
    model and stepping (a virtualised host may report only a generic model
    name), then the logical CPUs the kernel lists."""
    fields, logical = {}, 0
    try:
        for line in open("/proc/cpuinfo"):
            key, _, val = line.partition(":")
            key = key.strip()
            if key == "processor":
                logical += 1
            elif key in ("model name", "vendor_id", "cpu family", "model", "stepping") and key not in fields:
                fields[key] = val.strip()
    except OSError:
        return "unknown"
    name = fields.get("model name", "unknown")
    ids = ", ".join(f"{k} {fields[k]}" for k in ("vendor_id", "cpu family", "model", "stepping") if k in fields)
    return f"{name} ({ids}; {logical} logical CPUs listed)" if ids else name


def cpu_cores_note(threads: int) -> str:
    """How `cores` was counted (cgroup quota first, as the reference's
    scripts/p7_gpu_pcs_arithmetic.py:52-58, then the affinity mask)."""
    import oracle
    quota = oracle.cgroup_cpu_quota()
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        affinity = os.cpu_count() or 1
    q = f"cgroup cpu.max quota {quota}" if quota else "no cgroup cpu.max quota"
    return f"{threads} threads: {q}, affinity mask {affinity} CPUs, the smaller taken"


def traffic_for(name: str):
    f = ROOT / "profiles" / "traffic.json"
    if not f.exists():
        return None
    try:
        entry = json.loads(f.read_text()).get(name)
    except (ValueError, OSError):
        return None
    return entry.get("bytes") if isinstance(entry, dict) else None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="c3", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-copy-probe", action="store_true")
    ap.add_argument("--no-commit-tree", action="store_true")
    ap.add_argument("--no-x4", action="store_true")
    ap.add_argument("--no-seam-chain", action="store_true")
    ap.add_argument("--no-reference-commits", action="store_true")
    ap.add_argument("--no-published-shapes", action="store_true")
    ap.add_argument("--no-host-batch", action="store_true")
    ap.add_argument("--x4-log-n", type=int, default=24)
    a = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print("bench.py measures one GPU: every box in this setup has one MI355X and the encode path is "
              "row-parallel with no exchange; run with --gpus 1.", file=sys.stderr)
        return 2

    from volta_mi355x import Backend
    b = Backend(timing_policy=0)
    log(f"config {a.config}: generating and uploading inputs")
    wl = Workload(b, a.config)
    cfg = wl.cfg
    for _ in range(a.warmup):
        wl.step()
    b.synchronize()
    b.reset_stats()
    log(f"timing {a.steps} steps")
    t0 = time.perf_counter()
    for _ in range(a.steps):
        wl.step()
    b.synchronize()
    dt = time.perf_counter() - t0
    stats = b.get_stats()
    ms = dt / a.steps * 1e3
    value = wl.elements_per_step() * a.steps / dt / 1e9
    enc_calls = stats["calls"]["pcs_ntt"]
    enc_s = stats["kernel_ns"]["pcs_ntt"] / max(enc_calls, 1) / 1e9
    launches_per_step = max(enc_calls // a.steps, 1)
    alg = cfg.algorithmic_bytes  # per encode launch (C5: one direction)
    achieved = alg / enc_s / 1e9 if enc_s > 0 else None
    tree = None
    if not a.no_commit_tree and a.config != "c5":
        log("commit tree over the codewords")
        tree = commit_tree(b, wl)
    x4 = None
    if not a.no_x4:
        log(f"X4 transforms at 2^{a.x4_log_n} points")
        x4 = x4_transforms(b, a.x4_log_n)
    chain_leg = None
    if not a.no_seam_chain:
        log("seam chain (messages + NTT through the reference's calls)")
        chain_leg = seam_chain(b, wl)
    hbatch = None
    if not a.no_host_batch:
        log("host batch NTT (the hybrid commit's volta_cuda_ntt_fp_batch) at the workload's shape")
        hbatch = host_batch(b, wl)
    shapes = None
    if not a.no_published_shapes:
        log("the reference's published shapes (P4_LAYER NTT, 1024 x 16384 two-combination)")
        shapes = published_shapes(b)
    wl_close = wl.close
    commits = None
    if not a.no_reference_commits:
        log("the reference's production commitments (C3_WEIGHTS, C3_EMBED)")
        commits = reference_commits()
    copy_gbs = None if a.no_copy_probe else round(copy_bandwidth(b), 1)
    expand_gbs = None if a.no_copy_probe else round(expand_bandwidth(b), 1)
    chain = None if a.no_copy_probe else fp2_chain_peak(b)
    cpu = None
    if not a.no_cpu_baseline:
        log("cpu baseline")
        cpu = cpu_baseline(a.config, wl)
    wl_close()
    b.close()
    out = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "Gelem/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u64",
        "data": "synthetic",
        "config": {"workload": WORKLOADS[a.config], "rows": cfg.rows, "msg_len": cfg.msg_len, "code_len": cfg.n,
                   "combinations": cfg.combinations, "parallelism": "single-gpu"},
        "roofline": {
            "bound": "hbm",
            "kernel": "encode (PcsNtt launch)",
            "achieved": round(achieved, 1) if achieved else None,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4) if achieved else None,
            "traffic": traffic_for(a.config),
            "traffic_source": ("copied from profiles/traffic.json (rocprofv3 --pmc FETCH_SIZE x 2 + WRITE_SIZE of "
                               "the same kernel, taken in separate runs), not measured in this run"),
            "algorithmic_bytes": alg,
            "avg_launch_ms": round(enc_s * 1e3, 4),
            "launches_per_step": launches_per_step,
            "hbm_copy_gbs": copy_gbs,
            "hbm_expand_gbs": expand_gbs,
            "frac_of_expand": round(achieved / expand_gbs, 4) if achieved and expand_gbs else None,
        },
        "int_peak": chain,
        "cpu_baseline": cpu,
        "kernel_ms_per_step": {k: round(v / a.steps / 1e6, 4) for k, v in stats["kernel_ns"].items() if v},
        "seam_chain": chain_leg,
        "commit_tree": tree,
        "x4": x4,
        "reference_commits": commits,
        "reference_published_shapes": shapes,
        "host_batch": hbatch,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
