"""Synthetic inputs for the five benchmark configurations.

The generators are this build's choice (the configurations name only the
distributions); each is deterministic, and tests/golden/config_inputs.json
holds a SHA-256 fingerprint plus the first and last elements of every
configuration's packed input (checked by tests/test_config_fixtures.py), so
a change of generator or of numpy's streams is caught.

C1  256 rows x 2^12 uniform Fp -> 2^14 (rate 1/4); rows from
    FpStream::domain_separated(SEED_C1, row) (device ChaCha8, the reference's
    generator); one combination with 256 uniform Fp challenges embedded (c, 0).
C2  768x2304 i16 uniform in [-2^15, 2^15) flattened row-major into
    1024 x 2048 (zero tail) -> 2^13; two combinations with coefficients
    c^1..c^rows for two seeded Fp2 challenges.
C3  124,439,808 i16 ~ N(0, 2000^2) rounded and clipped, flattened into
    2^16 x 2^11 (zero tail) -> 2^13; two challenge-power combinations.
C4  2^15 x 2^12 Fp, each four uniform i16 lanes as a little-endian base-2^16
    integer canonicalised with Fp::new -> 2^15 (rate 1/8).
C5  64 x 2^24 uniform Fp, forward then inverse NTT, a 64-row combination,
    and a gather of 256 seeded columns.

Two further configurations follow the reference's production layer layouts
(rust/volta-pcs/src/layer_layout.rs:30, 34) and its resident commit chain
(ligero.rs:468-511): i16 weights ~ N(0, 2000^2) plus 512 ChaCha8 masking pads
per row, generated on the device each commit, encoded as lift(w) || pads || 0.
P15 24,576 x 2^13 i16 + 512 pads -> 2^15.
P17 2,080 x 2^15 i16 + 512 pads -> 2^17.
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass

import numpy as np

P = 0xFFFF_FFFF_0000_0001

# GPT-2 small parameter count used by C3: the listed weight matrices sum to
# 124,318,464; the configuration's 124,439,808 also counts 121,344 bias and
# LayerNorm parameters, so exactly that many values are generated.
GPT2_SMALL_WEIGHTS = 124_439_808


def seed_bytes(label: str) -> bytes:
    """32-byte seed for a label (SHA-256 of the label)."""
    return hashlib.sha256(label.encode()).digest()


def rng(label: str) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(int.from_bytes(seed_bytes(label)[:8], "little")))


@dataclass(frozen=True)
class Config:
    name: str
    rows: int
    msg_len: int     # message length per row (cols of the packed matrix)
    n: int           # codeword length
    kind: str        # "fp" (u64 messages) or "i16"
    combinations: int
    pad: int = 0     # ChaCha8 pads per row after the i16 weights

    @property
    def elements(self) -> int:
        return self.rows * self.n

    @property
    def algorithmic_bytes(self) -> int:
        """Input read once + codewords written once (+ the pads written and read once)."""
        return (self.rows * self.msg_len * (8 if self.kind == "fp" else 2) + self.rows * self.n * 8
                + 2 * self.rows * self.pad * 8)


CONFIGS = {
    "c1": Config("c1", 256, 1 << 12, 1 << 14, "fp", 1),
    "c2": Config("c2", 1024, 1 << 11, 1 << 13, "i16", 2),
    "c3": Config("c3", 1 << 16, 1 << 11, 1 << 13, "i16", 2),
    "c4": Config("c4", 1 << 15, 1 << 12, 1 << 15, "fp", 0),
    "c5": Config("c5", 64, 1 << 24, 1 << 24, "fp", 1),
    "p15": Config("p15", 24576, 1 << 13, 1 << 15, "i16", 0, 512),
    "p17": Config("p17", 2080, 1 << 15, 1 << 17, "i16", 0, 512),
}

SEED_C1_ROWS = seed_bytes("volta-mi355x/c1/rows")
SEED_C1_CHALLENGES = seed_bytes("volta-mi355x/c1/challenges")


def c2_weights(rows: int = 1024, cols: int = 2048) -> np.ndarray:
    """768x2304 uniform i16 flattened into rows x cols (zero tail)."""
    w = rng("volta-mi355x/c2/weights").integers(-(1 << 15), 1 << 15, size=768 * 2304, dtype=np.int16)
    out = np.zeros(rows * cols, dtype=np.int16)
    k = min(w.size, out.size)
    out[:k] = w[:k]
    return out.reshape(rows, cols)


def gaussian_i16(label: str, count: int, sigma: float = 2000.0) -> np.ndarray:
    g = rng(label)
    out = np.empty(count, dtype=np.int16)
    step = 1 << 24
    for s in range(0, count, step):
        e = min(count, s + step)
        v = g.standard_normal(size=e - s, dtype=np.float32)
        v *= np.float32(sigma)
        np.rint(v, out=v)
        np.clip(v, -32768, 32767, out=v)
        out[s:e] = v.astype(np.int16)
    return out


def c3_weights(rows: int = 1 << 16, cols: int = 1 << 11, count: int = GPT2_SMALL_WEIGHTS) -> np.ndarray:
    """Gaussian GPT-2-small-sized weight vector packed into rows x cols.

    A smaller ``rows`` takes the leading rows of the same packed matrix (used
    by parity tests), so every row matches the full configuration's row."""
    total = rows * cols
    out = np.zeros(total, dtype=np.int16)
    k = min(count, total)
    out[:k] = gaussian_i16("volta-mi355x/c3/weights", k)
    return out.reshape(rows, cols)


def c4_messages(rows: int = 1 << 15, cols: int = 1 << 12) -> np.ndarray:
    """Four uniform i16 lanes per element, lane 0 lowest, base 2^16, Fp::new."""
    g = rng("volta-mi355x/c4/lanes")
    lanes = g.integers(0, 1 << 16, size=(rows * cols, 4), dtype=np.uint64)
    x = lanes[:, 0] | (lanes[:, 1] << np.uint64(16)) | (lanes[:, 2] << np.uint64(32)) | (lanes[:, 3] << np.uint64(48))
    x = np.where(x >= np.uint64(P), x - np.uint64(P), x)
    return x.reshape(rows, cols)


def uniform_fp(label: str, shape) -> np.ndarray:
    """Exactly uniform values in [0, p)."""
    return rng(label).integers(0, P, size=shape, dtype=np.uint64)


def c5_rows(rows: int = 64, n: int = 1 << 24) -> np.ndarray:
    return uniform_fp("volta-mi355x/c5/rows", (rows, n))


def challenges_fp2(label: str, count: int) -> np.ndarray:
    """`count` uniform Fp2 challenges as (count, 2) u64."""
    return uniform_fp(label, (count, 2))


def c5_query_columns(n: int = 1 << 24, queries: int = 256) -> np.ndarray:
    return rng("volta-mi355x/c5/queries").integers(0, n, size=queries, dtype=np.uint32)


# ---- the reference's production commitment layouts ---------------------------------------------

@dataclass(frozen=True)
class TensorSlot:
    """One tensor's block in a commitment (rust/volta-pcs/src/layer_layout.rs
    TensorSlot): k rows of n i16 placed from ``offset`` with row stride
    ``stride`` (n rounded up to a power of two), inside a k_pad x n_pad block."""
    name: str
    k: int
    n: int
    offset: int
    stride: int


def block_layout(shapes, pad_outer: bool = True):
    """LayerWeightLayout2::for_shapes(_exact) (layer_layout.rs:221-253): each
    (k, n) tensor gets a k_pad x n_pad block (next powers of two); blocks are
    placed largest first (ties in input order) so every offset is a multiple
    of its block; the total is the end of the last block, rounded up to a
    power of two unless ``pad_outer`` is false.  Returns (slots in input
    order, total)."""
    blocks = [(name, k, n, _pow2(k) * _pow2(n)) for name, k, n in shapes]
    order = sorted(range(len(blocks)), key=lambda i: -blocks[i][3])  # sorted() is stable
    offsets, cursor = {}, 0
    for i in order:
        offsets[i] = cursor
        cursor += blocks[i][3]
    total = _pow2(cursor) if pad_outer else cursor
    slots = [TensorSlot(name, k, n, offsets[i], _pow2(n)) for i, (name, k, n, _) in enumerate(blocks)]
    assert all(s.offset % (_pow2(s.k) * _pow2(s.n)) == 0 for s in slots)
    return slots, total


def _pow2(x: int) -> int:
    return 1 << (x - 1).bit_length()


# One GPT-2-small layer (layout_gpt2_layer, layer_layout.rs:122-143): c_attn on
# its permuted 768 x 4096 column layout, attn_proj, ffn_up, ffn_down.
GPT2_LAYER_SHAPES = (("c_attn", 768, 4096), ("attn_proj", 768, 768), ("ffn_up", 768, 3072),
                     ("ffn_down", 3072, 768))


def c3_weights_slots():
    """The consolidated weights commitment (layout_gpt2_weights_c3,
    layer_layout.rs:170-178; C3_WEIGHTS = 24,576 x 2^13, layer_layout.rs:30):
    twelve 2^24-coefficient layer blocks, the layer layout inside each.  The
    reference's report commits these 48 tensors by strided device placements
    (rust/volta-bench/src/bin/p6_report.rs:2584-2615)."""
    layer, total = block_layout(GPT2_LAYER_SHAPES)
    assert total == 1 << 24
    slots = [TensorSlot(f"h{l}.{s.name}", s.k, s.n, l * total + s.offset, s.stride)
             for l in range(12) for s in layer]
    return slots, 12 * total


def c3_embed_slots():
    """The exact-block embedding commitment (layout_gpt2_embed_c3,
    layer_layout.rs:209-214; C3_EMBED = 2,080 x 2^15, layer_layout.rs:34): wte
    50,257 x 768 and wpe 1,024 x 768 without the outer 2^27 pad
    (p6_report.rs:2929-2952)."""
    return block_layout((("wte", 50257, 768), ("wpe", 1024, 768)), pad_outer=False)


def slot_tensor(label: str, slot: TensorSlot) -> np.ndarray:
    """Gaussian i16 weights for one tensor (k x n), seeded by label and name."""
    return gaussian_i16(f"{label}/{slot.name}", slot.k * slot.n).reshape(slot.k, slot.n)
