"""Every leg of the benchmark configurations at its full shape, on the GPU,
through the C ABI, against the oracle (bit-exact).

Where the oracle cannot redo a full-size transform in seconds (C5's 2^24-point
rows), the whole output is pinned by size-independent properties instead: the
column-sum identity sum_r encode(m_r) = encode(sum_r m_r) (linearity, the
verifier's own check, rust/volta-pcs/src/ligero.rs:1841-1856) and forward ->
inverse round trips, next to oracle parity on sampled rows."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

P = 0xFFFF_FFFF_0000_0001


def column_sums_mod_p(oracle, m: np.ndarray) -> np.ndarray:
    """Sum over the rows (< 2^31 of them) of a rows x cols u64 matrix, mod p:
    hi 2^32 + lo with hi = a 2^32 + b is b 2^32 + a (2^32 - 1) + lo mod p
    (2^64 = 2^32 - 1), two canonical terms added by the oracle."""
    lo = (m & np.uint64(0xFFFF_FFFF)).sum(axis=0, dtype=np.uint64)
    hi = (m >> np.uint64(32)).sum(axis=0, dtype=np.uint64)
    a, b = hi >> np.uint64(32), hi & np.uint64(0xFFFF_FFFF)
    return oracle.fp_add_vec(b << np.uint64(32), a * np.uint64(0xFFFF_FFFF) + lo)


def device_column_sums(backend, buf, rows, cols):
    """The same sums on the device: the combination with all-one coefficients."""
    ones = backend.upload_device(np.tile(np.array([1, 0], np.uint64), rows))
    out = backend.combine_rows_fp_device(buf, rows, cols, ones, 1)
    s = backend.download_device(out).view(np.uint64).reshape(cols, 2)
    backend.free_device(ones)
    backend.free_device(out)
    assert (s[:, 1] == 0).all()
    return s[:, 0]


def test_c1_encode_and_combination_at_shape(backend, oracle):
    """C1: 256 FpStream rows of 2^12 -> 2^14, and the combination of all 256
    rows with 256 uniform challenges embedded as (c, 0), as bench.py runs it."""
    from volta_mi355x import FP2, workloads as W
    cfg = W.CONFIGS["c1"]
    dm = backend.chacha8_prover_secret_fp_rows_device(W.SEED_C1_ROWS, 0, cfg.rows, cfg.msg_len)
    msgs = backend.download_device(dm).reshape(cfg.rows, cfg.msg_len)
    ch = W.uniform_fp("volta-mi355x/c1/challenges", cfg.rows)
    co = np.zeros((cfg.rows, 2), np.uint64)
    co[:, 0] = ch
    dc = backend.alloc_device(cfg.rows, FP2)
    backend.upload_into(dc, 0, co.reshape(-1))
    u = backend.combine_rows_fp_device(dm, cfg.rows, cfg.msg_len, dc, 1)
    enc = backend.ntt_fp_encode_device(dm, cfg.rows, cfg.msg_len, cfg.n)
    got_u = backend.download_device(u).view(np.uint64).reshape(1, cfg.msg_len, 2)
    got_e = backend.download_device(enc).reshape(cfg.rows, cfg.n)
    for b in (dm, dc, u, enc):
        backend.free_device(b)
    assert (got_u == oracle.combine_rows_fp(msgs, co, 1)).all()
    assert (got_e == oracle.ntt_encode_batch(msgs, cfg.n)).all()


def test_c4_every_row(backend, oracle):
    """C4 at full size: 2^15 packed-lane rows of 2^12 -> 2^15.  Every codeword
    element against the oracle, in blocks of 4096 rows, and all rows once more
    through the column-sum identity."""
    from volta_mi355x import workloads as W
    cfg = W.CONFIGS["c4"]
    m = W.c4_messages()
    d = backend.upload_device(m.reshape(-1))
    out = backend.ntt_fp_encode_device(d, cfg.rows, cfg.msg_len, cfg.n)
    block = 4096
    for r0 in range(0, cfg.rows, block):
        got = backend.download_device(out, r0 * cfg.n, block * cfg.n).reshape(block, cfg.n)
        want = oracle.ntt_encode_batch(m[r0:r0 + block], cfg.n)
        bad = np.nonzero((got != want).any(axis=1))[0]
        assert bad.size == 0, f"rows {(bad[:8] + r0).tolist()} differ"
    sums = device_column_sums(backend, out, cfg.rows, cfg.n)
    backend.free_device(d)
    backend.free_device(out)
    want = oracle.ntt_encode_batch(column_sums_mod_p(oracle, m).reshape(1, -1), cfg.n)[0]
    assert (sums == want).all()


def test_c5_round_trip_combination_and_gather(backend, oracle):
    """C5 at full size, every leg bench.py times: 64 x 2^24 forward (4 rows
    against the oracle, all rows by the column-sum identity), the inverse
    restoring every input, the 64-row challenge-power combination of the
    codewords and the 256-column gather, both against the oracle."""
    from volta_mi355x import workloads as W
    cfg = W.CONFIGS["c5"]
    rows, n = cfg.rows, cfg.n
    x = W.c5_rows()
    sample = [0, 17, 42, 63]
    x_sample = x[sample].copy()
    inp = backend.upload_device(x.reshape(-1))
    fwd = backend.ntt_fp_batch_device(inp, rows, n)
    back = backend.ntt_fp_inverse_batch_device(fwd, rows, n)
    assert (backend.download_device(back).reshape(rows, n) == x).all()
    backend.free_device(back)
    sums = device_column_sums(backend, fwd, rows, n)
    assert (sums == oracle.ntt_forward_batch(column_sums_mod_p(oracle, x).reshape(1, -1))[0]).all()
    c = tuple(int(v) for v in W.challenges_fp2("volta-mi355x/c5/challenges", 1)[0])
    co = backend.fp2_powers_device(c, rows)
    u = backend.combine_rows_fp_device(fwd, rows, n, co, 1)
    q = W.c5_query_columns(n, 256)
    cols = backend.pcs_gather_columns_device(fwd, rows, n, q)
    got_u = backend.download_device(u).view(np.uint64).reshape(1, n, 2)
    got_cols = backend.download_device(cols).reshape(256, rows)
    enc = backend.download_device(fwd).reshape(rows, n)
    for b in (inp, fwd, co, u, cols):
        backend.free_device(b)
    del x
    assert (enc[sample] == oracle.ntt_forward_batch(x_sample)).all()
    assert (got_cols == enc[:, q].T).all()
    assert (got_u == oracle.combine_rows_fp(enc, oracle.fp2_powers(c, rows), 1)).all()
