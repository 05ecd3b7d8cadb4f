"""Ligero commit arithmetic on the resident backend (host orchestration).

Mirrors the device chain of rust/volta-pcs/src/ligero.rs for the hot path:

* `commit_encode_resident` = finish_resident_commit (ligero.rs:468-511) up to
  the encoded matrix: ChaCha8 pads -> messages -> batched NTT.  Column hashing
  and the Merkle tree stay with the caller (the north star keeps them in Rust).
* `proximity_combinations` = the global row-combination pass of
  open_multi_zk_resident (ligero.rs:1258-1295): coefficients c^1..c^rows per
  challenge (fp2_powers_device), one pcs_combine_rows_device call for all
  challenges, reading the matrix once.

Transcript challenges and masks are inputs here, exactly as the Rust caller
supplies them.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .accel import FP2, Backend, DeviceBuffer, InvalidInput


@dataclass(frozen=True)
class LigeroParams:
    """rust/volta-pcs/src/ligero.rs:46-86."""
    rows: int
    col_bits: int
    pad: int
    code_bits: int
    n_queries: int = 0

    @property
    def cols(self) -> int:
        return 1 << self.col_bits

    @property
    def msg_len(self) -> int:
        return self.cols + self.pad

    @property
    def code_len(self) -> int:
        return 1 << self.code_bits

    def validate(self) -> None:
        if self.rows <= 0:
            raise InvalidInput("PCS needs at least one matrix row")
        if self.msg_len > self.code_len:
            raise InvalidInput("rate > 1")
        if self.n_queries > self.pad and self.pad:
            raise InvalidInput("column hiding needs n_queries <= pad")


def commit_encode_resident(backend: Backend, weights: DeviceBuffer, params: LigeroParams,
                           pad_seed: bytes | None = None, fused: bool = True):
    """Encode the packed i16 weight matrix (rows x cols, row-major, resident).

    Returns (encoded rows x code_len u64 buffer, pads buffer or None).
    With ``fused`` the message rows are built inside the transform load
    (volta_mi355x_pcs_encode_device); otherwise the reference's two-call
    chain pcs_messages_device + ntt_fp_batch_device runs.  Both give the same
    codewords.
    """
    params.validate()
    rows, cols, pad, n = params.rows, params.cols, params.pad, params.code_len
    if pad:
        if pad_seed is None:
            raise InvalidInput("a pad seed is required when pad > 0")
        pads = backend.chacha8_prover_secret_fp_rows_device(pad_seed, 0, rows, pad)
    else:
        # The seam cannot allocate zero bytes: a one-element placeholder.
        pads = backend.alloc_device(1, np.uint64)
    try:
        if fused:
            enc = backend.pcs_encode_device(weights, 0, pads, 0, rows, cols, pad, n)
        else:
            msgs = backend.pcs_messages_device(weights, 0, pads, 0, rows, cols, pad, n)
            try:
                enc = backend.ntt_fp_batch_device(msgs, rows, n)
            finally:
                backend.free_device(msgs)
    except Exception:
        backend.free_device(pads)
        raise
    if not pad:
        backend.free_device(pads)
        pads = None
    return enc, pads


def challenge_powers(backend: Backend, challenges, rows: int) -> DeviceBuffer:
    """Coefficient rows [c^1..c^rows] for each challenge, concatenated
    (combinations x rows Fp2, resident)."""
    chs = [tuple(int(x) for x in c) for c in challenges]
    coeffs = backend.alloc_device(len(chs) * rows, FP2)
    try:
        for k, c in enumerate(chs):
            pw = backend.fp2_powers_device(c, rows)
            try:
                backend.copy_device_rows(pw, 0, rows, coeffs, k * rows, rows, 1, rows)
            finally:
                backend.free_device(pw)
    except Exception:
        backend.free_device(coeffs)
        raise
    return coeffs


def proximity_combinations(backend: Backend, weights: DeviceBuffer, pads: DeviceBuffer | None,
                           params: LigeroParams, challenges) -> DeviceBuffer:
    """u_c[j] = sum_i c^(i+1) msg_i[j] for every challenge c, one matrix pass.
    Returns combinations x msg_len Fp2 (resident)."""
    coeffs = challenge_powers(backend, challenges, params.rows)
    placeholder = None
    if pads is None:
        placeholder = pads = backend.alloc_device(1, np.uint64)
    try:
        return backend.pcs_combine_rows_device(weights, 0, pads, 0, coeffs, 0, params.rows, params.cols,
                                               params.pad, len(challenges))
    finally:
        backend.free_device(coeffs)
        if placeholder is not None:
            backend.free_device(placeholder)
