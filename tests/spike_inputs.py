"""Input formulas of the reference's standalone arithmetic benchmarks, whose
recorded output checksums pin both the oracle and the device path."""
import numpy as np

P = 0xFFFF_FFFF_0000_0001
MASK64 = (1 << 64) - 1


def ntt_input(rows, bits, msg_len):
    """cuda/p7_pcs_arithmetic.cu:207-211: in[idx] = (idx*0x9E3779B9 + 17) mod p
    for column j < msg_len (idx the global row-major index), else 0."""
    n = 1 << bits
    idx = np.arange(rows * n, dtype=np.uint64)
    v = ((idx * np.uint64(0x9E3779B9) + np.uint64(17)) % np.uint64(P)).reshape(rows, n)
    v[:, msg_len:] = 0
    return v


def combine_inputs(rows, cols):
    """cuda/p7_pcs_arithmetic.cu:270-275: u64 weights and the q/c coefficient rows."""
    i = np.arange(rows * cols, dtype=np.uint64)
    w = ((i * np.uint64(0x85EBCA6B) + np.uint64(29)) % np.uint64(P)).reshape(rows, cols)
    r = np.arange(rows, dtype=np.uint64)
    Pu = np.uint64(P)
    q = np.stack([(r * np.uint64(37) + np.uint64(11)) % Pu, (r * np.uint64(53) + np.uint64(5)) % Pu], 1)
    c = np.stack([(r * np.uint64(71) + np.uint64(7)) % Pu, (r * np.uint64(97) + np.uint64(13)) % Pu], 1)
    return w, q, c


def combine_checksum(fnv, uq, uc):
    """cuda/p7_pcs_arithmetic.cu:318: cs(uq) XOR cs(uc) * 0x9E3779B97F4A7C15."""
    return fnv(uq) ^ ((fnv(uc) * 0x9E3779B97F4A7C15) & MASK64)


def fp2_inputs(n):
    """cuda/p7_goldilocks_roofline.cu:112-119."""
    x = np.arange(n, dtype=np.uint64)
    Pu = np.uint64(P)
    a = np.stack([(x * np.uint64(0x9E3779B9) + np.uint64(17)) % Pu, (x * np.uint64(0x85EBCA6B) + np.uint64(29)) % Pu], 1)
    b = np.stack([(x * np.uint64(0xC2B2AE35) + np.uint64(31)) % Pu, (x * np.uint64(0x27D4EB2F) + np.uint64(43)) % Pu], 1)
    return a, b


NTT_GOLDEN = [(32, 12, 2304, 0xA87A560725F2D016), (1024, 15, 16896, 0xBE7B90425A4C7229)]
COMBINE_GOLDEN = [(32, 2048, 0x0852323A5805ED2C), (1024, 16384, 0x856F9A96D8E01901)]
FP2_STREAM_GOLDEN = [(20, 0xAB1B94B1D98FD160), (24, 0x33EB029C2CCB481F)]
FP2_CHAIN_GOLDEN = [(16, 64, 0x994B7AB598EDF5D0), (20, 256, 0x2D1768754CF29569)]

# BLAKE3 Merkle pins.
# rust/volta-pcs/src/merkle.rs:89-96: root over the 16 leaves blake3([i]), i < 16.
MERKLE16_ROOT = bytes([0x45, 0x14, 0xd7, 0xcb, 0xd7, 0xa1, 0x95, 0x56, 0x08, 0x77, 0x4f, 0xf4, 0xce, 0x36, 0x98, 0x40,
                       0xa4, 0xe4, 0x0e, 0x72, 0x2c, 0xaa, 0x2a, 0x8c, 0xce, 0xe2, 0xf6, 0xd0, 0x53, 0x9d, 0x9f, 0x17])
# benchmarks/results/p7-gpu-blake3-merkle[-quick]-2026-07-11-3b0a916.json: column tree root over
# M[i] = (i * 0x9E3779B9 + 17) mod p (cuda/p7_blake3_merkle.cu:243), rows x cols.
MERKLE_BENCH_GOLDEN = [(32, 1024, "f427c1a8e4024b372e694b20215a860cfbf94c2463e2a5f76021243f1f8722e1"),
                       (1024, 32768, "c90027afa35e9f24dd436d51d734b63e52c9788f50a1658c7a6a2a2685ca4d5f")]
# Published BLAKE3 digests (the specification's reference implementation) of "" and "abc".
BLAKE3_PUBLISHED = [(b"", "af1349b9f5f9a1a6a0404dea36dcc9499bcb25c9adc112b7cc9a93cae41f3262"),
                    (b"abc", "6437b3ac38465133ffb63b75273a8db548c558465d79db03fd359c6cd5bd9d85")]


def merkle_bench_matrix(rows, cols):
    """cuda/p7_blake3_merkle.cu:243 (i * 0x9E3779B9 + 17 evaluated in wrapping u64)."""
    i = np.arange(rows * cols, dtype=np.uint64)
    return ((i * np.uint64(0x9E3779B9) + np.uint64(17)) % np.uint64(P)).reshape(rows, cols)
