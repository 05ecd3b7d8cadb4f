"""GPU parity of the BLAKE3 column leaves, Merkle tree and paths against the
oracle (volta_oracle_blake3.c) and the reference's recorded roots.

Shapes cover one partial block per column, whole and partial chunks, chunk
counts that are and are not powers of two (the joins of column_groups and
merge_groups), Fp2 elements, and at full C3 size the aligned 16-chunk groups
(sampled columns, full upper tree).
"""
import numpy as np
import pytest

import spike_inputs as spike

pytestmark = pytest.mark.gpu

P = 0xFFFF_FFFF_0000_0001


def rand_fp(seed, shape):
    return np.random.default_rng(seed).integers(0, P, size=shape, dtype=np.uint64)


def device_tree(backend, m, rows, cols, fp2=False):
    from volta_mi355x import FP2
    dm = backend.upload_device(m.reshape(-1, 2) if fp2 else m.reshape(-1), FP2 if fp2 else None)
    tree = (backend.hash_fp2_tree_device if fp2 else backend.hash_fp_tree_device)(dm, rows, cols)
    got = backend.download_device(tree.storage).reshape(-1, 32)
    root = backend.merkle_root_device(tree)
    backend.free_device_merkle_tree(tree)
    backend.free_device(dm)
    assert root == got[-1].tobytes()
    return got


@pytest.mark.parametrize("rows,cols", [(1, 1), (1, 4), (3, 2), (8, 64), (16, 8), (100, 32), (127, 16), (128, 16),
                                       (129, 64), (256, 4), (384, 8), (1000, 64), (1024, 128), (1100, 2),
                                       (2112, 16), (5000, 8)])
def test_fp_tree_matches_oracle(backend, oracle, rows, cols):
    m = rand_fp(rows * 7919 + cols, (rows, cols))
    got = device_tree(backend, m, rows, cols)
    want = oracle.merkle_tree(oracle.hash_fp_columns(m, rows, cols))
    assert got.shape == want.shape
    assert (got == want).all()


@pytest.mark.parametrize("rows,cols", [(1, 1), (5, 8), (64, 4), (65, 16), (200, 2), (777, 8)])
def test_fp2_tree_matches_oracle(backend, oracle, rows, cols):
    m = rand_fp(rows * 31 + cols, (rows, cols, 2))
    got = device_tree(backend, m, rows, cols, fp2=True)
    want = oracle.merkle_tree(oracle.hash_fp2_columns(m, rows, cols))
    assert (got == want).all()


@pytest.mark.parametrize("rows,cols,want", spike.MERKLE_BENCH_GOLDEN)
def test_reference_bench_roots_on_device(backend, rows, cols, want):
    """The reference's recorded roots (1 chunk per column; 8 chunks per column)."""
    m = spike.merkle_bench_matrix(rows, cols)
    dm = backend.upload_device(m.reshape(-1))
    tree = backend.hash_fp_tree_device(dm, rows, cols)
    assert backend.merkle_root_device(tree).hex() == want
    backend.free_device_merkle_tree(tree)
    backend.free_device(dm)


def test_paths_match_oracle(backend, oracle):
    rows, cols = 40, 256
    m = rand_fp(77, (rows, cols))
    dm = backend.upload_device(m.reshape(-1))
    tree = backend.hash_fp_tree_device(dm, rows, cols)
    idx = np.array([0, 1, 255, 128, 77, 3, 3, 254], dtype=np.uint32)
    di = backend.upload_device(idx)
    dp = backend.merkle_paths_device(tree, di, idx.size)
    got = backend.download_device(dp).reshape(idx.size, 8, 32)
    host_tree = backend.download_device(tree.storage).reshape(-1, 32)
    for b in (dp, di, dm):
        backend.free_device(b)
    backend.free_device_merkle_tree(tree)
    want = oracle.merkle_paths(host_tree, cols, idx)
    assert (got == want).all()
    # an index the seam would reject reads as zero hashes instead of faulting
    dm = backend.upload_device(m.reshape(-1))
    tree = backend.hash_fp_tree_device(dm, rows, cols)
    di = backend.upload_device(np.array([cols, 5], dtype=np.uint32))
    dp = backend.merkle_paths_device(tree, di, 2)
    got = backend.download_device(dp).reshape(2, 8, 32)
    for b in (dp, di, dm):
        backend.free_device(b)
    backend.free_device_merkle_tree(tree)
    assert not got[0].any() and got[1].any()


def test_host_column_hashes_and_geometry(backend, oracle):
    rows, cols = 24, 32
    m = rand_fp(3, (rows, cols))
    assert (backend.hash_fp_columns(m, rows, cols) == oracle.hash_fp_columns(m, rows, cols)).all()
    from volta_mi355x import InvalidInput
    for r, c in [(4, 32), (12, 32), (24, 3)]:
        with pytest.raises(InvalidInput):
            backend.hash_fp_columns(np.zeros(r * c, np.uint64), r, c)
    # the C side applies the same rule
    out = np.zeros(32 * 32, np.uint8)
    rc = backend.lib.volta_cuda_hash_fp_columns(backend.raw, m.ctypes.data, 12, 32, out.ctypes.data)
    assert rc != 0 and "geometry" in backend.last_error()
    rc = backend.lib.volta_cuda_hash_fp_tree_device(backend.raw, 0, 0, 8, 3, 0, 0)
    assert rc != 0 and "geometry" in backend.last_error()


def test_merkle_stats_op(backend):
    rows, cols = 16, 8
    dm = backend.upload_device(rand_fp(1, (rows, cols)).reshape(-1))
    backend.reset_stats()
    tree = backend.hash_fp_tree_device(dm, rows, cols)
    s = backend.get_stats()
    assert s["calls"]["pcs_merkle"] == 1 and s["calls"]["pcs_ntt"] == 0
    backend.free_device_merkle_tree(tree)
    backend.free_device(dm)


def _sampled_tree_check(backend, oracle, dm, rows, cols, cols_to_check):
    tree = backend.hash_fp_tree_device(dm, rows, cols)
    leaves = backend.download_device(tree.storage, 0, cols * 32).reshape(cols, 32)
    full = backend.download_device(tree.storage).reshape(-1, 32)
    backend.free_device_merkle_tree(tree)
    # upper tree from the device leaves
    assert (oracle.merkle_tree(leaves) == full).all()
    # sampled leaves from the device's own column gather
    idx = np.array(cols_to_check, dtype=np.uint32)
    cols_dev = backend.pcs_gather_columns_device(dm, rows, cols, idx)
    colv = backend.download_device(cols_dev).reshape(idx.size, rows)
    backend.free_device(cols_dev)
    for q, j in enumerate(idx):
        assert leaves[j].tobytes() == oracle.hash_fp_columns(np.ascontiguousarray(colv[q]), rows, 1)[0].tobytes(), j


def test_partial_last_group_sampled(backend, oracle):
    """4096 columns x 135 chunks (the last one half full): groups of 2 chunks
    with a one-chunk tail group (565 MB)."""
    rows, cols = 135 * 128 - 64, 4096
    dm = backend.chacha8_prover_secret_fp_rows_device(bytes(range(32)), 11, rows, cols)
    _sampled_tree_check(backend, oracle, dm, rows, cols, [0, 1, 63, 64, 2047, 4094, 4095])
    backend.free_device(dm)


def test_c3_encoded_matrix_tree_sampled(backend, oracle):
    """The commit of C3's shape: 2^16 x 2^13 Fp (4 GiB), 512 chunks per column
    in 32 aligned groups of 16; sampled leaves, the full upper tree."""
    rows, cols = 1 << 16, 1 << 13
    dm = backend.chacha8_prover_secret_fp_rows_device(bytes([7] * 32), 0, rows, cols)
    _sampled_tree_check(backend, oracle, dm, rows, cols, [0, 1, 4095, 8191])
    backend.free_device(dm)


def test_host_column_hashes_staged_upload(backend, oracle):
    """volta_cuda_hash_fp_columns on a 64 MiB host matrix (8192 rows of 1024
    columns): its upload goes through the pinned staging buffers."""
    rows, cols = 8192, 1024
    m = np.random.Generator(np.random.PCG64(9300)).integers(0, P, size=rows * cols, dtype=np.uint64)
    assert (backend.hash_fp_columns(m, rows, cols) == oracle.hash_fp_columns(m, rows, cols)).all()
