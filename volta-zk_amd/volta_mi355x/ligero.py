"""Ligero commit arithmetic on the resident backend (host orchestration).

Mirrors the device chain of rust/volta-pcs/src/ligero.rs for the hot path,
making the same seam calls in the same order:

* `ResidentWeightPlacement` + `commit_resident_from_device` (ligero.rs:108-170,
  409-466): zero the packed i16 target, strided D2D placement of each tensor,
  then `finish_resident_commit` (ligero.rs:468-511): ChaCha8 pads -> messages
  -> batched NTT -> BLAKE3 column tree -> root.
* `commit_encode_resident`: the same chain up to the encoded matrix.
* `proximity_combinations` = the global row-combination pass of
  open_multi_zk_resident (ligero.rs:1258-1295): coefficients c^1..c^rows per
  challenge (fp2_powers_device), one pcs_combine_rows_device call for all
  challenges, reading the matrix once.
* `open_rows_resident`: every device step of open_multi_zk_resident
  (ligero.rs:1216-1551): mask rows, mask NTT and tree, u_c, the block-claim
  combinations u_g, the mask dots s_g, column gathers and Merkle paths.

Transcript challenges, claims and query indices are inputs here, exactly as
the Rust caller derives them; the protocol arithmetic above the seam
(ZeroBatch, corrections) stays with the caller.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .accel import FP2, Backend, DeviceBuffer, DeviceMerkleTree, InvalidInput


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


# ---- resident commitment (ligero.rs:108-170, 409-511) -------------------------------------

@dataclass(frozen=True)
class ResidentWeightPlacement:
    """One compact row-major i16 tensor (rows x cols elements of `source`
    starting at element `source_offset`) placed into the packed matrix at
    `destination_offset` with row stride `destination_stride`
    (ResidentWeightPlacement::new, ligero.rs:119-168, same checks and
    messages)."""
    source: DeviceBuffer
    source_offset: int
    rows: int
    cols: int
    destination_offset: int
    destination_stride: int
    packed_len: int

    def __post_init__(self):
        s = self.destination_stride
        if self.rows <= 0 or self.cols <= 0 or s < self.cols or s & (s - 1):
            raise InvalidInput("invalid resident weight placement geometry")
        if self.source_offset < 0 or self.source_offset + self.rows * self.cols > self.source.len:
            raise InvalidInput("resident weight placement source must be exact and compact")
        span = (1 << (self.rows - 1).bit_length()) * s
        if self.destination_offset % span:
            raise InvalidInput("resident weight placement block is not aligned")
        if self.destination_offset + span > self.packed_len:
            raise InvalidInput("resident weight placement exceeds packed target")

    @property
    def destination_end(self) -> int:
        return self.destination_offset + (1 << (self.rows - 1).bit_length()) * self.destination_stride


@dataclass
class ResidentProverMatrix:
    """Device-owned commitment state (ligero.rs:175-182)."""
    params: LigeroParams
    weights: DeviceBuffer
    pads: DeviceBuffer
    encoded: DeviceBuffer
    tree: DeviceMerkleTree


def commit_resident_from_device(backend: Backend, placements, params: LigeroParams, pad_seed: bytes,
                                fused: bool = False):
    """Returns (root, ResidentProverMatrix).  The packed target is allocated
    and zeroed by the commitment, then every placement is copied row by row
    (ligero.rs:409-466); overlapping placements are rejected before anything
    is allocated."""
    params.validate()
    packed_len = params.rows * params.cols
    if not placements:
        raise InvalidInput("resident PCS needs a weight placement")
    ranges = []
    for pl in placements:
        if pl.packed_len != packed_len:
            raise InvalidInput("resident weight placement targets the wrong PCS geometry")
        if pl.source.owner != id(backend):
            raise InvalidInput("resident weight placement belongs to a different CUDA context")
        ranges.append((pl.destination_offset, pl.destination_end))
    ranges.sort()
    if any(a[1] > b[0] for a, b in zip(ranges, ranges[1:])):
        raise InvalidInput("resident weight placements overlap")
    weights = backend.alloc_device(packed_len, np.int16)
    try:
        backend.zero_device(weights, 0, packed_len)
        for pl in placements:
            backend.copy_device_rows(pl.source, pl.source_offset, pl.cols, weights, pl.destination_offset,
                                     pl.destination_stride, pl.rows, pl.cols)
    except Exception:
        backend.free_device(weights)
        raise
    return finish_resident_commit(backend, weights, params, pad_seed, fused=fused)


def finish_resident_commit(backend: Backend, weights: DeviceBuffer, params: LigeroParams, pad_seed: bytes,
                           fused: bool = False):
    """ligero.rs:468-511: pads, messages, NTT (or the fused encode), messages
    freed, BLAKE3 column tree, root.  Takes ownership of `weights`: on error
    every buffer of the commitment, `weights` included, is freed."""
    rows, cols, pad, n = params.rows, params.cols, params.pad, params.code_len
    owned = [weights]
    try:
        pads = backend.chacha8_prover_secret_fp_rows_device(pad_seed, 0, rows, pad)
        owned.append(pads)
        if fused:
            encoded = backend.pcs_encode_device(weights, 0, pads, 0, rows, cols, pad, n)
        else:
            msgs = backend.pcs_messages_device(weights, 0, pads, 0, rows, cols, pad, n)
            try:
                encoded = backend.ntt_fp_batch_device(msgs, rows, n)
            finally:
                backend.free_device(msgs)
        owned.append(encoded)
        tree = backend.hash_fp_tree_device(encoded, rows, n)
        owned.append(tree.storage)
        root = backend.merkle_root_device(tree)
    except Exception:
        for b in owned:
            backend.free_device(b)
        raise
    return root, ResidentProverMatrix(params, weights, pads, encoded, tree)


def free_resident_matrix(backend: Backend, pm: ResidentProverMatrix) -> None:
    """Releases every allocation of a resident commitment (ligero.rs:513-541)."""
    for b in (pm.weights, pm.pads, pm.encoded, pm.tree.storage):
        if b.owner != id(backend):
            raise InvalidInput("resident prover matrix belongs to a different CUDA context")
    for b in (pm.weights, pm.pads, pm.encoded):
        backend.free_device(b)
    backend.free_device_merkle_tree(pm.tree)


# ---- resident opening, device steps (ligero.rs:1216-1551) -------------------------------

def claim_row0(params: LigeroParams, offset: int, point_len: int) -> int:
    """resident_claim_row0 (ligero.rs:953-972)."""
    if point_len < params.col_bits:
        raise InvalidInput("resident PCS block is smaller than a matrix row")
    if offset % (1 << point_len):
        raise InvalidInput("resident PCS block offset is not aligned")
    row0 = offset >> params.col_bits
    if row0 + (1 << (point_len - params.col_bits)) > params.rows:
        raise InvalidInput("resident PCS claim rows exceed matrix")
    return row0


def open_rows_resident(backend: Backend, pm: ResidentProverMatrix, claims, c, js, mask_seed: bytes) -> dict:
    """The device side of open_multi_zk_resident for claims [(offset, point)]
    (point: sequence of Fp2 pairs), the proximity challenge `c` and the query
    indices `js`, in the reference's call order.  Returns the proof material
    those calls produce: mask_root, u_c, u_gs, s_values (the mask dots, before
    the correlation is subtracted), data/mask columns and paths."""
    params = pm.params
    rows, cols, msg_len, n = params.rows, params.cols, params.msg_len, params.code_len
    col_bits, g_count = params.col_bits, len(claims)
    if g_count == 0:
        raise InvalidInput("resident PCS opening needs a claim")
    points = [np.ascontiguousarray(p, dtype=np.uint64).reshape(-1, 2) for _, p in claims]
    row0s = [claim_row0(params, off, len(p)) for (off, _), p in zip(claims, points)]
    mask_rows = g_count + 1
    owned = []

    def keep(b):
        owned.append(b)
        return b

    def drop(b):
        owned.remove(b)
        backend.free_device(b)

    try:
        # 1. masks (ligero.rs:1216-1256)
        mask_msgs = keep(backend.chacha8_prover_secret_fp2_rows_padded_device(mask_seed, 0, mask_rows, msg_len, n))
        mask_compact = keep(backend.alloc_device(mask_rows * msg_len, FP2))
        backend.copy_device_rows(mask_msgs, 0, n, mask_compact, 0, msg_len, mask_rows, msg_len)
        mask_encoded = keep(backend.ntt_fp2_batch_device(mask_msgs, mask_rows, n))
        drop(mask_msgs)
        mask_tree = backend.hash_fp2_tree_device(mask_encoded, mask_rows, n)
        keep(mask_tree.storage)
        mask_root = backend.merkle_root_device(mask_tree)
        # 2. proximity pass (ligero.rs:1258-1295)
        c_pows = keep(backend.fp2_powers_device(tuple(int(x) for x in c), rows))
        u_c_dev = keep(backend.pcs_combine_rows_device(pm.weights, 0, pm.pads, 0, c_pows, 0, rows, cols, params.pad,
                                                       1))
        backend.fp2_add_inplace_device(u_c_dev, 0, mask_compact, 0, msg_len)
        u_c = backend.download_device(u_c_dev, 0, msg_len).view(np.uint64).reshape(msg_len, 2)
        drop(u_c_dev)
        drop(c_pows)
        # 3. block-claim combinations (ligero.rs:1297-1366)
        coeffs = keep(backend.alloc_device(g_count * rows, FP2))
        backend.zero_device(coeffs, 0, g_count * rows)
        for g, (pt, row0) in enumerate(zip(points, row0s)):
            eq = keep(backend.equality_weights_device(pt[col_bits:]))
            backend.copy_device_rows(eq, 0, eq.len, coeffs, g * rows + row0, eq.len, 1, eq.len)
            drop(eq)
        u_g_dev = keep(backend.pcs_combine_rows_device(pm.weights, 0, pm.pads, 0, coeffs, 0, rows, cols, params.pad,
                                                       g_count))
        backend.fp2_add_inplace_device(u_g_dev, 0, mask_compact, msg_len, g_count * msg_len)
        u_gs = backend.download_device(u_g_dev, 0, g_count * msg_len).view(np.uint64).reshape(g_count, msg_len, 2)
        drop(u_g_dev)
        drop(coeffs)
        # 4. s_g = <mask row g, eq(point[..col_bits])> (ligero.rs:1368-1418)
        mpts = np.concatenate([p[:col_bits] for p in points]) if col_bits else None
        mask_points = keep(backend.upload_device(mpts, FP2)) if col_bits else None
        mask_eq = keep(backend.logup_eq_rows_device(mask_points, g_count, col_bits))
        dots = keep(backend.fp2_row_dots_device(mask_compact, msg_len, msg_len, mask_eq, 0, cols, g_count, cols))
        s_values = backend.download_device(dots, 0, g_count).view(np.uint64).reshape(g_count, 2)
        for b in (dots, mask_eq, mask_points, mask_compact):
            if b is not None:
                drop(b)
        # 5. query columns and paths (ligero.rs:1439-1551)
        idx = np.ascontiguousarray(js, dtype=np.uint32)
        indices = keep(backend.upload_device(idx))
        data_cols = keep(backend.pcs_gather_columns_device(pm.encoded, rows, n, idx))
        mask_cols = keep(backend.pcs_gather_columns_device(mask_encoded, mask_rows, n, idx, fp2=True))
        data_paths = keep(backend.merkle_paths_device(pm.tree, indices, idx.size))
        mask_paths = keep(backend.merkle_paths_device(mask_tree, indices, idx.size))
        bits = params.code_bits
        out = {
            "mask_root": mask_root,
            "u_c": u_c,
            "u_gs": u_gs,
            "s_values": s_values,
            "data_columns": backend.download_device(data_cols).reshape(idx.size, rows),
            "mask_columns": backend.download_device(mask_cols).view(np.uint64).reshape(idx.size, mask_rows, 2),
            "data_paths": backend.download_device(data_paths).reshape(idx.size, bits, 32),
            "mask_paths": backend.download_device(mask_paths).reshape(idx.size, bits, 32),
        }
    finally:
        for b in reversed(owned):
            backend.free_device(b)
    return out
