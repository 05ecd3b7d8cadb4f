"""Seeded sweeps of random geometries through the C ABI against the oracle,
bit-exact: transform sizes and batch shapes that the targeted tests do not
pick, element offsets on both sides, message lengths anywhere in the row,
combinations with and without pads, and the reference's two-call commit chain.
Each case's parameters are printed before it runs."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

P = 0xFFFF_FFFF_0000_0001


def gen(seed):
    return np.random.Generator(np.random.PCG64(seed))


@pytest.mark.parametrize("seed", range(12))
def test_forward_and_inverse_transforms_at_random_shapes(backend, oracle, seed):
    g = gen(1000 + seed)
    bits = int(g.integers(1, 21))
    n = 1 << bits
    rows = int(g.integers(1, max(2, min(6, (1 << 21) // n) + 1)))
    off_in, off_out = int(g.integers(0, 40)), int(g.integers(0, 40))
    print(f"seed {seed}: n 2^{bits}, rows {rows}, offsets {off_in}/{off_out}", flush=True)
    host = g.integers(0, P, size=(rows, n), dtype=np.uint64)
    inp = backend.alloc_device(off_in + rows * n, np.uint64)
    backend.upload_into(inp, off_in, host.reshape(-1))
    out = backend.alloc_device(off_out + rows * n, np.uint64)
    lib, raw = backend.lib, backend.raw
    assert lib.volta_cuda_ntt_fp_batch_device(raw, inp.id, off_in, rows, n, out.id, off_out) == 0, backend.last_error()
    fwd = backend.download_device(out, off_out, rows * n).reshape(rows, n)
    assert lib.volta_mi355x_ntt_fp_inverse_batch_device(raw, out.id, off_out, rows, n, inp.id, off_in) == 0, \
        backend.last_error()
    back = backend.download_device(inp, off_in, rows * n).reshape(rows, n)
    backend.free_device(inp)
    backend.free_device(out)
    assert (fwd == oracle.ntt_forward_batch(host)).all()
    assert (back == host).all()


@pytest.mark.parametrize("seed", range(12))
def test_commit_chain_at_random_shapes(backend, oracle, seed):
    """pcs_messages_device then ntt_fp_batch_device (the reference's two
    calls, encoded from the weights), random cols, pad and code length."""
    g = gen(2000 + seed)
    bits = int(g.integers(4, 18))
    n = 1 << bits
    pad = int(g.integers(0, 3)) * int(g.integers(1, max(2, n // 8)))
    cols = int(g.integers(1, n - pad + 1))
    rows = int(g.integers(1, max(2, min(9, (1 << 20) // n) + 1)))
    w_off, p_off = int(g.integers(0, 9)), int(g.integers(0, 9))
    print(f"seed {seed}: n 2^{bits}, rows {rows}, cols {cols}, pad {pad}, offsets {w_off}/{p_off}", flush=True)
    w = g.integers(-(1 << 15), 1 << 15, size=rows * cols, dtype=np.int16)
    w[: min(2, w.size)] = [-32768, 32767][: min(2, w.size)]
    pads = g.integers(0, P, size=rows * pad, dtype=np.uint64) if pad else np.zeros(1, np.uint64)
    dw = backend.alloc_device(w_off + w.size, np.int16)
    backend.upload_into(dw, w_off, w)
    dp = backend.alloc_device(p_off + pads.size, np.uint64)
    backend.upload_into(dp, p_off, pads)
    msgs = backend.pcs_messages_device(dw, w_off, dp, p_off, rows, cols, pad, n)
    enc = backend.ntt_fp_batch_device(msgs, rows, n)
    got = backend.download_device(enc).reshape(rows, n)
    got_m = backend.download_device(msgs).reshape(rows, n)
    for b in (dw, dp, msgs, enc):
        backend.free_device(b)
    want_m = oracle.pcs_messages(w, pads if pad else None, rows, cols, pad, n)
    assert (got_m == want_m).all()
    assert (got == oracle.ntt_forward_batch(want_m)).all()


@pytest.mark.parametrize("seed", range(10))
def test_combinations_at_random_shapes(backend, oracle, seed):
    from volta_mi355x import FP2
    g = gen(3000 + seed)
    rows = int(g.integers(1, 3000))
    cols = int(g.integers(1, 2100))
    pad = int(g.integers(0, 2)) * int(g.integers(1, 600))
    comb = int(g.integers(1, 10))
    w_off, c_off = int(g.integers(0, 9)), int(g.integers(0, 9))
    print(f"seed {seed}: rows {rows}, cols {cols}, pad {pad}, combinations {comb}, offsets {w_off}/{c_off}",
          flush=True)
    w = g.integers(-(1 << 15), 1 << 15, size=rows * cols, dtype=np.int16)
    pads = g.integers(0, P, size=rows * pad, dtype=np.uint64) if pad else np.zeros(1, np.uint64)
    co = g.integers(0, P, size=(comb * rows, 2), dtype=np.uint64)
    co[g.integers(0, comb * rows, size=comb * rows // 2)] = 0  # some zero coefficients and zero chunks
    dw = backend.alloc_device(w_off + w.size, np.int16)
    backend.upload_into(dw, w_off, w)
    dp = backend.upload_device(pads)
    dc = backend.alloc_device(c_off + comb * rows, FP2)
    backend.upload_into(dc, c_off, co.reshape(-1))
    out = backend.pcs_combine_rows_device(dw, w_off, dp, 0, dc, c_off, rows, cols, pad, comb)
    got = backend.download_device(out).view(np.uint64).reshape(comb, cols + pad, 2)
    for b in (dw, dp, dc, out):
        backend.free_device(b)
    assert (got == oracle.pcs_combine_rows(w, pads if pad else None, co, rows, cols, pad, comb)).all()


@pytest.mark.parametrize("seed", range(6))
def test_fp2_transforms_and_gathers_at_random_shapes(backend, oracle, seed):
    from volta_mi355x import FP2
    g = gen(4000 + seed)
    bits = int(g.integers(2, 19))
    n = 1 << bits
    rows = int(g.integers(1, max(2, min(5, (1 << 20) // n) + 1)))
    q = int(g.integers(1, 300))
    print(f"seed {seed}: Fp2 n 2^{bits}, rows {rows}, queries {q}", flush=True)
    host = g.integers(0, P, size=(rows, n, 2), dtype=np.uint64)
    inp = backend.alloc_device(rows * n, FP2)
    backend.upload_into(inp, 0, host.reshape(-1))
    out = backend.ntt_fp2_batch_device(inp, rows, n)
    got = backend.download_device(out).view(np.uint64).reshape(rows, n, 2)
    idx = g.integers(0, n, size=q, dtype=np.uint32)
    cols = backend.pcs_gather_columns_device(out, rows, n, idx, fp2=True)
    got_cols = backend.download_device(cols).view(np.uint64).reshape(q, rows, 2)
    for b in (inp, out, cols):
        backend.free_device(b)
    for comp in (0, 1):
        assert (got[:, :, comp] == oracle.ntt_forward_batch(host[:, :, comp].copy())).all()
    assert (got_cols == np.transpose(got[:, idx], (1, 0, 2))).all()
