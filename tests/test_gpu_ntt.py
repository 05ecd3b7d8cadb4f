"""GPU parity of the transforms, through the C ABI, against the oracle and the
reference-recorded checksums.  Bit-exact everywhere (integer field work)."""
import random

import numpy as np
import pytest

import spike_inputs as spike

pytestmark = pytest.mark.gpu

P = spike.P


def rand_fp(seed, shape):
    return np.random.Generator(np.random.PCG64(seed)).integers(0, P, size=shape, dtype=np.uint64)


def run_ntt(backend, host, n):
    rows = host.size // n
    inp = backend.upload_device(host.reshape(-1))
    try:
        out = backend.ntt_fp_batch_device(inp, rows, n)
        try:
            return backend.download_device(out).reshape(rows, n)
        finally:
            backend.free_device(out)
    finally:
        backend.free_device(inp)


# ---- field arithmetic on the device, pinned by reference-recorded outputs ------

def test_fp2_stream_probe_matches_reference_checksum(backend, oracle):
    log2, expected = spike.FP2_STREAM_GOLDEN[0]
    a, b = spike.fp2_inputs(1 << log2)
    da, db = backend.upload_device(a.reshape(-1)), backend.upload_device(b.reshape(-1))
    out = backend.alloc_device(2 << log2, np.uint64)
    backend._check(backend.lib.volta_mi355x_probe_fp2_device(backend.raw, da.id, db.id, out.id, 1 << log2, 0))
    got = backend.download_device(out)
    for buf in (da, db, out):
        backend.free_device(buf)
    assert oracle.fnv(got) == expected


def test_fp2_chain_probe_matches_reference_checksum(backend, oracle):
    log2, rounds, expected = spike.FP2_CHAIN_GOLDEN[0]
    a, b = spike.fp2_inputs(1 << log2)
    da, db = backend.upload_device(a.reshape(-1)), backend.upload_device(b.reshape(-1))
    out = backend.alloc_device(2 << log2, np.uint64)
    backend._check(backend.lib.volta_mi355x_probe_fp2_device(backend.raw, da.id, db.id, out.id, 1 << log2, rounds))
    got = backend.download_device(out)
    for buf in (da, db, out):
        backend.free_device(buf)
    assert oracle.fnv(got) == expected


# ---- forward NTT -------------------------------------------------------------------------

@pytest.mark.parametrize("bits", list(range(1, 15)))
def test_ntt_lds_sizes_match_oracle(backend, oracle, bits):
    n = 1 << bits
    host = rand_fp(bits, (3, n))
    host[0, :min(4, n)] = [0, 1, P - 1, P - 2][:min(4, n)]  # boundary values
    assert (run_ntt(backend, host, n) == oracle.ntt_forward_batch(host)).all()


@pytest.mark.parametrize("bits,rows", [(15, 3), (16, 2), (17, 2), (19, 1)])
def test_ntt_four_step_sizes_match_oracle(backend, oracle, bits, rows):
    n = 1 << bits
    host = rand_fp(100 + bits, (rows, n))
    assert (run_ntt(backend, host, n) == oracle.ntt_forward_batch(host)).all()


@pytest.mark.parametrize("rows,bits,msg_len,expected", spike.NTT_GOLDEN)
def test_ntt_reference_checksums_on_device(backend, oracle, rows, bits, msg_len, expected):
    out = run_ntt(backend, spike.ntt_input(rows, bits, msg_len), 1 << bits)
    assert oracle.fnv(out) == expected


def test_ntt_offsets_and_input_preserved(backend, oracle):
    n, rows = 256, 4
    host = rand_fp(7, (rows, n))
    big = backend.alloc_device(rows * n + 3 * n, np.uint64)
    backend.upload_into(big, n, host.reshape(-1))
    out = backend.alloc_device(rows * n + 5, np.uint64)
    backend._check(backend.lib.volta_cuda_ntt_fp_batch_device(backend.raw, big.id, n, rows, n, out.id, 5))
    got = backend.download_device(out, 5, rows * n).reshape(rows, n)
    still = backend.download_device(big, n, rows * n).reshape(rows, n)
    backend.free_device(big)
    backend.free_device(out)
    assert (got == oracle.ntt_forward_batch(host)).all()
    assert (still == host).all()


def test_inverse_round_trip_and_oracle(backend, oracle):
    for bits, rows in [(6, 3), (13, 4), (16, 2), (20, 1), (21, 1)]:
        n = 1 << bits
        host = rand_fp(200 + bits, (rows, n))
        inp = backend.upload_device(host.reshape(-1))
        fwd = backend.ntt_fp_batch_device(inp, rows, n)
        inv = backend.ntt_fp_inverse_batch_device(fwd, rows, n)
        back = backend.download_device(inv).reshape(rows, n)
        inv_of_host = backend.ntt_fp_inverse_batch_device(inp, rows, n)
        direct = backend.download_device(inv_of_host).reshape(rows, n)
        for b in (inp, fwd, inv, inv_of_host):
            backend.free_device(b)
        assert (back == host).all()
        assert (direct == oracle.ntt_inverse_batch(host)).all()


def test_forward_and_inverse_2_25(backend, oracle):
    """One 2^25 row: three passes of radix 2^9 (the largest plan of that radix)."""
    n = 1 << 25
    host = rand_fp(25, (1, n))
    inp = backend.upload_device(host.reshape(-1))
    fwd = backend.ntt_fp_batch_device(inp, 1, n)
    inv = backend.ntt_fp_inverse_batch_device(fwd, 1, n)
    got = backend.download_device(fwd).reshape(1, n)
    back = backend.download_device(inv).reshape(1, n)
    for b in (inp, fwd, inv):
        backend.free_device(b)
    assert (back == host).all()
    assert (got == oracle.ntt_forward_batch(host)).all()


def test_inverse_round_trip_four_passes(backend):
    """One 2^26 row: four passes of radix 2^7, 2^7, 2^6, 2^6, so the
    inverse's gather maps rows through two middle digits."""
    n = 1 << 26
    host = rand_fp(26, (1, n))
    inp = backend.upload_device(host.reshape(-1))
    fwd = backend.ntt_fp_batch_device(inp, 1, n)
    inv = backend.ntt_fp_inverse_batch_device(fwd, 1, n)
    back = backend.download_device(inv).reshape(1, n)
    for b in (inp, fwd, inv):
        backend.free_device(b)
    assert (back == host).all()


def test_batch_beyond_one_launch_slice(backend, oracle):
    """65,537 rows of 2^13: the pass engine launches at most 65,535 rows per
    grid; rows on both sides of each slice boundary match the oracle."""
    rows, n = 65537, 1 << 13
    g = np.random.Generator(np.random.PCG64(65537))
    host = g.integers(0, P, size=(rows, n), dtype=np.uint64)
    inp = backend.upload_device(host.reshape(-1))
    out = backend.ntt_fp_batch_device(inp, rows, n)
    picks = [0, 1, 65533, 65534, 65535, 65536]
    got = np.stack([backend.download_device(out, r * n, n) for r in picks])
    backend.free_device(inp)
    backend.free_device(out)
    assert (got == oracle.ntt_forward_batch(host[picks].copy())).all()


def test_host_entry_points(backend, oracle):
    n = 1 << 10
    msgs = rand_fp(11, (5, 300))
    got = backend.ntt_fp_batch(msgs, 5, 300, n)
    assert (got == oracle.ntt_encode_batch(msgs, n)).all()
    one = backend.ntt_fp(msgs[0], n)
    assert (one == got[0]).all()
    f2 = rand_fp(12, (40, 2))
    got2 = backend.ntt_fp2(f2, 64)
    for comp in (0, 1):
        want = oracle.ntt_encode_batch(f2[:, comp].reshape(1, -1).copy(), 64)[0]
        assert (got2[:, comp] == want).all()


def test_fp2_batch_device_componentwise(backend, oracle):
    rows, n = 3, 1 << 12
    host = rand_fp(13, (rows, n, 2))
    from volta_mi355x import FP2
    inp2 = backend.alloc_device(rows * n, FP2)
    backend.upload_into(inp2, 0, host.reshape(-1))
    out = backend.ntt_fp2_batch_device(inp2, rows, n)
    got = backend.download_device(out).view(np.uint64).reshape(rows, n, 2)
    for b in (inp2, out):
        backend.free_device(b)
    for comp in (0, 1):
        assert (got[:, :, comp] == oracle.ntt_forward_batch(host[:, :, comp].copy())).all()


@pytest.mark.parametrize("bits,rows", [(13, 3), (14, 2), (15, 4), (16, 2), (17, 3), (18, 2)])
def test_fp2_batch_device_random_rows_pass_engine(backend, oracle, bits, rows):
    """The opening's mask transform (ntt_fp2_batch_device at the code length,
    mask rows = claims + 1 > 1): random Fp2 rows on the pass engine, rows
    after the first reached through the batch offset, with an element offset
    on both sides."""
    from volta_mi355x import FP2
    n = 1 << bits
    host = rand_fp(bits * 31 + rows, (rows, n, 2))
    host[0, :2] = [[P - 1, P - 1], [0, 1]]
    inp = backend.alloc_device(rows * n + 3, FP2)
    backend.upload_into(inp, 3, host.reshape(-1))
    out = backend.alloc_device(rows * n + 5, FP2)
    backend._check(backend.lib.volta_cuda_ntt_fp2_batch_device(backend.raw, inp.id, 3, rows, n, out.id, 5))
    got = backend.download_device(out, 5, rows * n).view(np.uint64).reshape(rows, n, 2)
    kept = backend.download_device(inp, 3, rows * n).view(np.uint64).reshape(rows, n, 2)
    for b in (inp, out):
        backend.free_device(b)
    assert (kept == host).all()  # out of place: the input is preserved
    for comp in (0, 1):
        assert (got[:, :, comp] == oracle.ntt_forward_batch(host[:, :, comp].copy())).all(), comp


@pytest.mark.parametrize("bits", [6, 12, 13, 16])
def test_overlapping_ntt_regions_are_rejected(backend, bits):
    """The resident transforms are out of place (the input is preserved,
    .cu:6545-6579): any overlap of input and output, exact aliasing
    included, is an error and leaves the buffer untouched."""
    from volta_mi355x import FP2
    lib, raw = backend.lib, backend.raw
    n = 1 << bits
    host = rand_fp(bits, 2 * n + 8)
    buf = backend.upload_device(host)
    for call in (lib.volta_cuda_ntt_fp_batch_device, lib.volta_mi355x_ntt_fp_inverse_batch_device):
        for in_off, out_off in ((0, 0), (0, n // 2 + 1), (8, 0), (n, n)):
            assert call(raw, buf.id, in_off, 1, n, buf.id, out_off) != 0, (in_off, out_off)
            assert "overlap" in backend.last_error()
    assert lib.volta_cuda_ntt_fp_batch_device(raw, buf.id, 0, 1, n, buf.id, n) == 0  # adjacent: fine
    f2 = backend.alloc_device(2 * n, FP2)
    assert lib.volta_cuda_ntt_fp2_batch_device(raw, f2.id, 0, 1, n, f2.id, 0) != 0
    assert "overlap" in backend.last_error()
    assert (backend.download_device(buf)[:n] == host[:n]).all()
    backend.free_device(buf)
    backend.free_device(f2)


def test_base_field_sizes_above_the_two_adicity_are_rejected(backend):
    """p - 1 = 2^32 (2^32 - 1): base-field roots exist up to 2^32 points; the
    reference's twiddle table for 2^32 would be 16 GiB.  Sizes above 2^31 are
    refused before any table is built or uploaded."""
    lib, raw = backend.lib, backend.raw
    buf = backend.alloc_device(8, np.uint64)
    before = backend.get_stats()["h2d_bytes"]
    live = backend.get_stats()["live_device_bytes"]
    for n in (1 << 32, 1 << 33):
        assert lib.volta_cuda_ntt_fp_batch_device(raw, buf.id, 0, 1, n, buf.id, 0) != 0
        assert "geometry" in backend.last_error() or "size" in backend.last_error()
    assert backend.get_stats()["h2d_bytes"] == before
    assert backend.get_stats()["live_device_bytes"] == live
    backend.free_device(buf)


def test_compact_encode_device(backend, oracle):
    for rows, msg_len, bits in [(7, 100, 9), (4, 4096, 14), (3, 1000, 16)]:
        n = 1 << bits
        msgs = rand_fp(300 + bits, (rows, msg_len))
        d = backend.upload_device(msgs.reshape(-1))
        out = backend.ntt_fp_encode_device(d, rows, msg_len, n)
        got = backend.download_device(out).reshape(rows, n)
        backend.free_device(d)
        backend.free_device(out)
        assert (got == oracle.ntt_encode_batch(msgs, n)).all()


@pytest.mark.parametrize("n", [1 << 12, 1 << 14, 1 << 16])
def test_encode_of_empty_messages_is_zero(backend, n):
    """msg_len = 0, which the seam accepts: every codeword is zero on the
    one-tile path (2^12) and on the pass engine, whose loads still read an
    in-bounds word and mask it."""
    d = backend.upload_device(np.array([12345], dtype=np.uint64))
    out = backend.ntt_fp_encode_device(d, 3, 0, n)
    got = backend.download_device(out)
    backend.free_device(d)
    backend.free_device(out)
    assert got.shape == (3 * n,) and not got.any()
    host = backend.ntt_fp_batch(np.zeros(0, np.uint64), 2, 0, n)
    assert not np.asarray(host).any()


# The pass engine's gather reads only step-1 inputs that can be nonzero: with
# A-point first DFTs (A = 8 at 2^13, 16 at 2^14 .. 2^17, 32 at 2^18), a message
# of len elements needs ceil(len A / n) of them, rounded up to a compiled count
# (1, 2, 3|4, A/4+1, 8, 16, A).  Lengths at and one past each boundary k n / A.
ZERO_TAIL_CASES = [(13, 8, (1, 2, 3, 4, 8)), (14, 16, (1, 2, 4, 5, 8, 16)), (15, 16, (1, 2, 4, 5, 8, 16)),
                   (17, 16, (1, 2, 4, 5, 8)), (18, 32, (1, 2, 4, 8, 9, 16))]


@pytest.mark.parametrize("bits,a,ks", ZERO_TAIL_CASES)
def test_encode_zero_tail_boundaries(backend, oracle, bits, a, ks):
    n = 1 << bits
    lens = sorted({1, n - 1, n} | {k * n // a + d for k in ks for d in (0, 1) if k * n // a + d <= n})
    for msg_len in lens:
        msgs = rand_fp(bits * 100003 + msg_len, (2, msg_len))
        d = backend.upload_device(msgs.reshape(-1))
        out = backend.ntt_fp_encode_device(d, 2, msg_len, n)
        got = backend.download_device(out).reshape(2, n)
        backend.free_device(d)
        backend.free_device(out)
        assert (got == oracle.ntt_encode_batch(msgs, n)).all(), (bits, msg_len)


@pytest.mark.parametrize("bits,a", [(15, 16), (18, 32)])
def test_pcs_encode_zero_tail_boundaries(backend, oracle, bits, a):
    """The i16 weights || pads source with cols + pad at and one past k n / A,
    the boundary falling inside the weights or inside the pads."""
    n = 1 << bits
    q = n // a
    for cols, pad in [(2 * q - 3, 3), (2 * q - 3, 4), (4 * q, 1), (5 * q - 512, 512), (5 * q - 511, 512),
                      (q // 2, q // 2), (1, 0)]:
        g = np.random.Generator(np.random.PCG64(bits * 7919 + cols * 31 + pad))
        w = g.integers(-(1 << 15), 1 << 15, size=2 * cols, dtype=np.int16)
        pads = rand_fp(cols + pad, 2 * pad) if pad else np.zeros(1, np.uint64)
        dw, dp = backend.upload_device(w), backend.upload_device(pads)
        out = backend.pcs_encode_device(dw, 0, dp, 0, 2, cols, pad, n)
        got = backend.download_device(out).reshape(2, n)
        for b in (dw, dp, out):
            backend.free_device(b)
        assert (got == oracle.pcs_encode_i16(w, pads, 2, cols, pad, n)).all(), (bits, cols, pad)


def test_column_tables_and_their_fallback_agree(oracle):
    """A column pass spanning at most 2^18 points reads its pre-twiddles from a
    table built on first use.  Inside a coarse timing scope, where tables may
    not grow, a pass whose table is missing builds them from the two-level
    table instead.  Both give the oracle's transform; only the second call
    grows device memory, by the 2^17-word table of the radix-2^9 pass."""
    from volta_mi355x import FP2, Backend
    rows, n = 2, 1 << 17
    host = rand_fp(171, (rows, n))
    with Backend(timing_policy=1) as b:
        # an Fp2 transform of 2^17 uploads the twiddles; its passes (2^6, 2^6,
        # 2^5) build other column tables than the Fp passes (2^9, 2^8)
        d2 = b.upload_device(np.zeros((rows * n, 2), np.uint64), FP2)
        o2 = b.ntt_fp2_batch_device(d2, rows, n)
        inp = b.upload_device(host.reshape(-1))
        outs = [b.alloc_device(rows * n, np.uint64) for _ in range(2)]
        live = b.get_stats()["live_device_bytes"]
        assert b.lib.volta_cuda_begin_coarse_timing(b.raw, 3) == 0
        assert b.lib.volta_cuda_ntt_fp_batch_device(b.raw, inp.id, 0, rows, n, outs[0].id, 0) == 0
        assert b.lib.volta_cuda_end_coarse_timing(b.raw) == 0
        assert b.get_stats()["live_device_bytes"] == live
        assert b.lib.volta_cuda_ntt_fp_batch_device(b.raw, inp.id, 0, rows, n, outs[1].id, 0) == 0
        assert b.get_stats()["live_device_bytes"] == live + n * 8
        want = oracle.ntt_forward_batch(host)
        for o in outs:
            assert (b.download_device(o).reshape(rows, n) == want).all()
        assert not b.download_device(o2).view(np.uint64).any()
        ws, res, cached = b.memory_breakdown()
        assert ws + res + cached == b.get_stats()["live_device_bytes"]
        for x in (d2, o2, inp, *outs):
            b.free_device(x)


# ---- PCS encode of i16 message rows ---------------------------------------------------

@pytest.mark.parametrize("rows,cols,pad,bits", [(5, 16, 0, 6), (9, 100, 7, 8), (17, 2048, 0, 13), (4, 2048, 512, 13),
                                                (3, 4096, 0, 14), (2, 1024, 3, 15),
                                                # the n = 2^13 fast path: full, partial and 1-column rows
                                                (3, 1, 0, 13), (5, 1000, 0, 13), (64, 2047, 0, 13),
                                                (1000, 2048, 0, 13),
                                                # the reference's production layouts (layer_layout.rs:26-45):
                                                # 2^13 or 2^15 columns + 512 pads -> 2^15 .. 2^18, fewer rows
                                                (70, 2048, 512, 13), (3, 8192, 512, 15), (2, 8192, 512, 16),
                                                (2, 32768, 512, 17), (1, 32768, 512, 18), (3, 5000, 37, 16)])
def test_pcs_encode_fused_and_chain_match_oracle(backend, oracle, rows, cols, pad, bits):
    n = 1 << bits
    g = np.random.Generator(np.random.PCG64(rows * 1000 + cols))
    w = g.integers(-(1 << 15), 1 << 15, size=rows * cols, dtype=np.int16)
    w[:3] = [-32768, 32767, -1]
    pads = rand_fp(cols, rows * pad) if pad else np.zeros(1, np.uint64)
    dw, dp = backend.upload_device(w), backend.upload_device(pads)
    fused = backend.pcs_encode_device(dw, 0, dp, 0, rows, cols, pad, n)
    msgs = backend.pcs_messages_device(dw, 0, dp, 0, rows, cols, pad, n)
    chain = backend.ntt_fp_batch_device(msgs, rows, n)
    got_f = backend.download_device(fused).reshape(rows, n)
    got_m = backend.download_device(msgs).reshape(rows, n)
    got_c = backend.download_device(chain).reshape(rows, n)
    for b in (dw, dp, fused, msgs, chain):
        backend.free_device(b)
    want = oracle.pcs_encode_i16(w, pads, rows, cols, pad, n)
    assert (got_m == oracle.pcs_messages(w, pads, rows, cols, pad, n)).all()
    assert (got_c == want).all()
    assert (got_f == want).all()


@pytest.mark.parametrize("cols", [1, 63, 64, 65, 1024, 2047, 2048])
@pytest.mark.parametrize("kind", ["top band", "byte edges"])
def test_fast_encode_byte_split_edges(backend, oracle, cols, kind):
    """The n = 2^13 fast path splits each i16 into two signed bytes for the
    matrix-core product (x = 256 (x >> 8) + ((x & 255) - 128) + 128): rows of
    values whose high byte is 127 with a low byte >= 128 (32640 .. 32767), and
    of every low-byte and high-byte extreme, at zero-tail lengths around the
    64-column rows of the four-step split; every element against the oracle,
    through the reference's two calls."""
    rows, n = 33, 8192
    g = np.random.Generator(np.random.PCG64(cols * 7 + len(kind)))
    if kind == "top band":
        w = g.integers(32640, 32768, size=rows * cols).astype(np.int16)
    else:
        edges = np.array([-32768, -32767, -32641, -32640, -129, -128, -127, -1, 0, 1, 127, 128, 255, 256, 32639,
                          32640, 32767], np.int16)
        w = g.choice(edges, size=rows * cols)
    dw, dp = backend.upload_device(w), backend.alloc_device(1, np.uint64)
    msgs = backend.pcs_messages_device(dw, 0, dp, 0, rows, cols, 0, n)
    enc = backend.ntt_fp_batch_device(msgs, rows, n)  # the recorded rows: the fast path from the weights
    got = backend.download_device(enc).reshape(rows, n)
    for b in (dw, dp, msgs, enc):
        backend.free_device(b)
    assert (got == oracle.pcs_encode_i16(w, None, rows, cols, 0, n)).all()


@pytest.mark.parametrize("rows", [4096, 4097, 8200])
def test_fast_encode_both_phase_b_orders(backend, oracle, rows):
    """The n = 2^13 fast path puts parity 1's shifts after phase B's barrier
    when each workgroup walks at most 8 rows (4,096 rows on 256 CUs) and
    before it otherwise: rows on both sides of that bound, every element
    against the oracle, through the reference's two calls."""
    cols, n = 2048, 8192
    w = np.random.Generator(np.random.PCG64(rows)).integers(-32768, 32768, size=rows * cols, dtype=np.int16)
    dw, dp = backend.upload_device(w), backend.alloc_device(1, np.uint64)
    msgs = backend.pcs_messages_device(dw, 0, dp, 0, rows, cols, 0, n)
    enc = backend.ntt_fp_batch_device(msgs, rows, n)
    got = backend.download_device(enc).reshape(rows, n)
    for b in (dw, dp, msgs, enc):
        backend.free_device(b)
    want = oracle.pcs_encode_i16(w, None, rows, cols, 0, n)
    bad = np.nonzero((got != want).any(axis=1))[0]
    assert bad.size == 0, f"rows {bad[:8].tolist()} differ"


# ---- benchmark configurations ---------------------------------------------------------

def test_c1_full_config(backend, oracle):
    """C1: 256 rows of FpStream-generated messages -> 2^14 codewords."""
    from volta_mi355x import workloads as W
    cfg = W.CONFIGS["c1"]
    dm = backend.chacha8_prover_secret_fp_rows_device(W.SEED_C1_ROWS, 0, cfg.rows, cfg.msg_len)
    msgs = backend.download_device(dm).reshape(cfg.rows, cfg.msg_len)
    assert (msgs == oracle.fp_rows(W.SEED_C1_ROWS, 0, cfg.rows, cfg.msg_len)).all()
    out = backend.ntt_fp_encode_device(dm, cfg.rows, cfg.msg_len, cfg.n)
    got = backend.download_device(out).reshape(cfg.rows, cfg.n)
    backend.free_device(dm)
    backend.free_device(out)
    assert (got == oracle.ntt_encode_batch(msgs, cfg.n)).all()


def test_c2_full_config(backend, oracle):
    from volta_mi355x import workloads as W
    cfg = W.CONFIGS["c2"]
    w = W.c2_weights()
    dw, dp = backend.upload_device(w.reshape(-1)), backend.alloc_device(1, np.uint64)
    out = backend.pcs_encode_device(dw, 0, dp, 0, cfg.rows, cfg.msg_len, 0, cfg.n)
    got = backend.download_device(out).reshape(cfg.rows, cfg.n)
    for b in (dw, dp, out):
        backend.free_device(b)
    assert (got == oracle.pcs_encode_i16(w, None, cfg.rows, cfg.msg_len, 0, cfg.n)).all()


@pytest.mark.parametrize("path", ["reference_chain", "fused_entry"])
def test_c3_full_config_every_row(backend, oracle, path):
    """C3 at full size (2^16 rows of 2^11 i16 -> 2^13): every codeword element
    against the oracle, in blocks of 8192 rows (the oracle, threaded, redoes
    the whole encode in seconds), and the whole output once more by a linear
    invariant: the sum of all codewords equals the encode of the sum of all
    messages.  Through the reference's two calls as the bench times them
    (pcs_messages_device into a fresh buffer, ntt_fp_batch_device of those
    rows, the rows freed unread: finish_resident_commit, ligero.rs:477-496) and
    through the fused extension entry point."""
    from volta_mi355x import workloads as W
    cfg = W.CONFIGS["c3"]
    w = W.c3_weights()
    dw, dp = backend.upload_device(w.reshape(-1)), backend.alloc_device(1, np.uint64)
    if path == "reference_chain":
        msgs = backend.pcs_messages_device(dw, 0, dp, 0, cfg.rows, cfg.msg_len, 0, cfg.n)
        out = backend.ntt_fp_batch_device(msgs, cfg.rows, cfg.n)
        backend.free_device(msgs)
    else:
        out = backend.pcs_encode_device(dw, 0, dp, 0, cfg.rows, cfg.msg_len, 0, cfg.n)
    block = 8192
    for r0 in range(0, cfg.rows, block):
        got = backend.download_device(out, r0 * cfg.n, block * cfg.n).reshape(block, cfg.n)
        want = oracle.pcs_encode_i16(w[r0:r0 + block].reshape(-1), None, block, cfg.msg_len, 0, cfg.n)
        bad = np.nonzero((got != want).any(axis=1))[0]
        assert bad.size == 0, f"rows {(bad[:8] + r0).tolist()} differ"
    # column sums via the combination with all-one coefficients (u64 rows)
    ones = backend.upload_device(np.tile(np.array([1, 0], np.uint64), cfg.rows))
    colsum = backend.combine_rows_fp_device(out, cfg.rows, cfg.n, ones, 1)
    s = backend.download_device(colsum).view(np.uint64).reshape(cfg.n, 2)
    for b in (dw, dp, out, ones, colsum):
        backend.free_device(b)
    msum = w.astype(np.int64).sum(axis=0)
    msum = np.where(msum < 0, msum.astype(np.uint64) + np.uint64(P), msum.astype(np.uint64))
    want_sum = oracle.ntt_encode_batch(msum.astype(np.uint64).reshape(1, -1), cfg.n)[0]
    assert (s[:, 1] == 0).all()
    assert (s[:, 0] == want_sum).all()


def test_c4_rows(backend, oracle):
    from volta_mi355x import workloads as W
    cfg = W.CONFIGS["c4"]
    rows = 24
    m = W.c4_messages(rows, cfg.msg_len)
    d = backend.upload_device(m.reshape(-1))
    out = backend.ntt_fp_encode_device(d, rows, cfg.msg_len, cfg.n)
    got = backend.download_device(out).reshape(rows, cfg.n)
    backend.free_device(d)
    backend.free_device(out)
    assert (got == oracle.ntt_encode_batch(m, cfg.n)).all()


def test_c5_rows_forward_inverse(backend, oracle):
    """Two 2^24 rows: forward vs oracle, then the inverse restores the input."""
    rows, n = 2, 1 << 24
    host = rand_fp(55, (rows, n))
    inp = backend.upload_device(host.reshape(-1))
    fwd = backend.ntt_fp_batch_device(inp, rows, n)
    got = backend.download_device(fwd).reshape(rows, n)
    inv = backend.ntt_fp_inverse_batch_device(fwd, rows, n)
    back = backend.download_device(inv).reshape(rows, n)
    for b in (inp, fwd, inv):
        backend.free_device(b)
    assert (back == host).all()
    assert (got == oracle.ntt_forward_batch(host)).all()


# ---- n = 2^13 in one pass: written u64 rows and the host batch -------------------------

@pytest.mark.parametrize("rows", [1, 3, 64, 513, 1031])
def test_ntt13_one_pass_device_rows(backend, oracle, rows):
    """volta_cuda_ntt_fp_batch_device at n = 2^13 on arbitrary canonical rows
    (the rows a caller wrote: every column input can be nonzero), as many
    rows as workgroups and more (the persistent grid walks them), boundary
    values included, with element offsets on both sides."""
    n = 1 << 13
    host = rand_fp(1300 + rows, (rows, n))
    host[0, :6] = [0, 1, P - 1, P - 2, 1 << 32, (1 << 63) + 5]
    if rows > 2:
        host[1] = P - 1
        host[2] = 0
    off_in, off_out = 24, 40
    din = backend.alloc_device(off_in + rows * n, np.uint64)
    backend.upload_into(din, off_in, host.reshape(-1))
    dout = backend.alloc_device(off_out + rows * n, np.uint64)
    assert backend.lib.volta_cuda_ntt_fp_batch_device(backend.raw, din.id, off_in, rows, n, dout.id, off_out) == 0, \
        backend.last_error()
    got = backend.download_device(dout, off_out, rows * n).reshape(rows, n)
    kept = backend.download_device(din, off_in, rows * n).reshape(rows, n)
    for b in (din, dout):
        backend.free_device(b)
    assert (kept == host).all()  # input preserved
    want = oracle.ntt_forward_batch(host)
    bad = np.nonzero((got != want).any(axis=1))[0]
    assert bad.size == 0, f"rows {bad[:8].tolist()} differ"


@pytest.mark.parametrize("bits", [13, 14])
def test_one_pass_device_rows_with_zero_tails(backend, oracle, bits):
    """Rows passed at full length (read whole: the caller may have written
    them) that are zero from 8 M on (M = n / 32), as message rows are: each
    wave of the one-pass kernel checks its inputs there and runs stage A's
    first two stages as copies when they are all zero.  Most rows have that
    tail, some carry one nonzero value at a position that falls to a different
    wave each time, a few are dense."""
    n = 1 << bits
    m8 = 8 * (n // 32)
    rows = 300
    host = rand_fp(4400 + bits, (rows, n))
    host[:, m8:] = 0
    host[0, :4] = [0, 1, P - 1, P - 2]
    for r in range(1, 40):
        host[r, m8 + (r * 97) % (n - m8)] = P - 1 - r
    host[40:44] = rand_fp(4500 + bits, (4, n))
    host[44, n - 1] = 1
    d = backend.upload_device(host.reshape(-1))
    dout = backend.alloc_device(rows * n, np.uint64)
    assert backend.lib.volta_cuda_ntt_fp_batch_device(backend.raw, d.id, 0, rows, n, dout.id, 0) == 0, \
        backend.last_error()
    got = backend.download_device(dout).reshape(rows, n)
    for b in (d, dout):
        backend.free_device(b)
    want = oracle.ntt_forward_batch(host)
    bad = np.nonzero((got != want).any(axis=1))[0]
    assert bad.size == 0, f"rows {bad[:8].tolist()} differ"


@pytest.mark.parametrize("msg_len", [1, 5, 2047, 2048, 2049, 4096, 8191, 8192])
def test_ntt13_one_pass_host_batch_lengths(backend, oracle, msg_len):
    """The host batch (volta_cuda_ntt_fp_batch, compact rows of msg_len, the
    hybrid commit's call, rust/volta-pcs/src/ligero.rs:564-581) at n = 2^13 on
    both sides of the zero-tail switch (msg_len <= 2048 reads one input of
    each four per column)."""
    n, rows = 1 << 13, 37
    host = rand_fp(1400 + msg_len, (rows, msg_len))
    host[0, 0] = P - 1
    got = backend.ntt_fp_batch(host, rows, msg_len, n)
    padded = np.zeros((rows, n), np.uint64)
    padded[:, :msg_len] = host
    assert (got == oracle.ntt_forward_batch(padded)).all()


@pytest.mark.parametrize("rows,msg_len", [(2063, 2048), (2061, 2049), (300, 8192)])
def test_host_batch_staged_copies(backend, oracle, rows, msg_len):
    """Host batches whose copies go through the pinned staging buffers
    (32 MiB and up: 2,063 x 2,048 and 2,061 x 2,049 inputs of 33.8 MB, their
    135 MB outputs in 9 chunks of 16 MiB over 8 buffers, the last chunk
    short; 300 x 8,192 stages only the download).  The caller's arrays are
    pageable, the input starting 8 bytes into its allocation; every element
    against the oracle, and the input left as it was."""
    n = 1 << 13
    vals = rand_fp(5200 + rows, (rows, msg_len))
    vals[0, :3] = [0, 1, P - 1]
    vals[-1, -1] = P - 2
    buf = np.empty(rows * msg_len + 1, np.uint64)
    buf[1:] = vals.reshape(-1)
    host = buf[1:].reshape(rows, msg_len)
    before = host.copy()
    got = backend.ntt_fp_batch(host, rows, msg_len, n)
    assert (host == before).all()
    assert got.shape == (rows, n)
    assert (got == oracle.ntt_encode_batch(vals, n)).all()


# ---- n = 2^15 in one pass (ntt15.hip) ------------------------------------------------


@pytest.mark.parametrize("msg_len", [1, 7, 2048, 2049, 4095, 4096, 4097, 8191, 8192, 8193, 16384, 16896, 32768])
def test_ntt15_one_pass_host_batch_lengths(backend, oracle, msg_len):
    """The host batch at n = 2^15 on both sides of each of the kernel's input
    widths (2^11 .. 2^15 nonzero inputs; up to 2^13 the next row's inputs load
    a row ahead, past it at the top of their own row)."""
    n, rows = 1 << 15, 37
    host = rand_fp(1500 + msg_len, (rows, msg_len))
    host[0, 0] = P - 1
    host[1, -1] = P - 2
    got = backend.ntt_fp_batch(host, rows, msg_len, n)
    padded = np.zeros((rows, n), np.uint64)
    padded[:, :msg_len] = host
    assert (got == oracle.ntt_forward_batch(padded)).all()


@pytest.mark.parametrize("rows", [1, 255, 256, 257, 600])
def test_ntt15_one_pass_device_rows(backend, oracle, rows):
    """C4's device encode (compact rows of 2^12 -> 2^15) with fewer rows than
    workgroups, exactly as many, and more (each workgroup walks several rows,
    loading the next one's inputs during the current one)."""
    n, msg_len = 1 << 15, 4096
    host = rand_fp(1600 + rows, (rows, msg_len))
    host[0, :4] = [0, 1, P - 1, (1 << 63) + 3]
    d = backend.upload_device(host.reshape(-1))
    out = backend.ntt_fp_encode_device(d, rows, msg_len, n)
    got = backend.download_device(out).reshape(rows, n)
    backend.free_device(d)
    backend.free_device(out)
    want = oracle.ntt_encode_batch(host, n)
    bad = np.nonzero((got != want).any(axis=1))[0]
    assert bad.size == 0, f"rows {bad[:8].tolist()} differ"


@pytest.mark.parametrize("rows,cols,pad", [(300, 8192, 512), (300, 8192, 0), (3, 8192, 1024), (5, 4096, 512),
                                           (5, 4096, 0), (3, 8192, 1025), (3, 6000, 512)])
def test_ntt15_one_pass_message_rows(backend, oracle, rows, cols, pad):
    """lift(w) || pads || 0 -> 2^15 through the fused encode and through the
    reference's two calls (deferred rows): the one-pass kernel for 2^12 and
    2^13 weight columns with up to 1024 pads, the pass engine for the rest."""
    n = 1 << 15
    g = np.random.Generator(np.random.PCG64(rows * 7 + cols + pad))
    w = g.integers(-(1 << 15), 1 << 15, size=rows * cols, dtype=np.int16)
    w[:3] = [-32768, 32767, -1]
    pads = rand_fp(cols + pad, rows * pad) if pad else np.zeros(1, np.uint64)
    dw, dp = backend.upload_device(w), backend.upload_device(pads)
    fused = backend.pcs_encode_device(dw, 0, dp, 0, rows, cols, pad, n)
    msgs = backend.pcs_messages_device(dw, 0, dp, 0, rows, cols, pad, n)
    chain = backend.ntt_fp_batch_device(msgs, rows, n)
    got_f = backend.download_device(fused).reshape(rows, n)
    got_c = backend.download_device(chain).reshape(rows, n)
    for b in (dw, dp, fused, msgs, chain):
        backend.free_device(b)
    want = oracle.pcs_encode_i16(w, pads, rows, cols, pad, n)
    assert (got_f == want).all()
    assert (got_c == want).all()


# ---- n = 2^14 in one pass (ntt_rr.hip) -----------------------------------------------


@pytest.mark.parametrize("msg_len", [1, 4096, 4097, 8192, 8193, 16384])
def test_ntt14_one_pass_host_batch_lengths(backend, oracle, msg_len):
    """The host batch at n = 2^14 on both sides of each stage-A input width
    (2^12, 2^13, 2^14 nonzero inputs)."""
    n, rows = 1 << 14, 37
    host = rand_fp(1700 + msg_len, (rows, msg_len))
    host[0, 0] = P - 1
    host[1, -1] = P - 2
    got = backend.ntt_fp_batch(host, rows, msg_len, n)
    padded = np.zeros((rows, n), np.uint64)
    padded[:, :msg_len] = host
    assert (got == oracle.ntt_forward_batch(padded)).all()


@pytest.mark.parametrize("rows", [1, 255, 256, 257, 700])
def test_ntt14_one_pass_device_rows(backend, oracle, rows):
    """C1's device encode (compact rows of 2^12 -> 2^14) with fewer rows than
    workgroups, as many, and more (each workgroup walks several rows)."""
    n, msg_len = 1 << 14, 4096
    host = rand_fp(1800 + rows, (rows, msg_len))
    host[0, :4] = [0, 1, P - 1, (1 << 63) + 3]
    d = backend.upload_device(host.reshape(-1))
    out = backend.ntt_fp_encode_device(d, rows, msg_len, n)
    got = backend.download_device(out).reshape(rows, n)
    backend.free_device(d)
    backend.free_device(out)
    want = oracle.ntt_encode_batch(host, n)
    bad = np.nonzero((got != want).any(axis=1))[0]
    assert bad.size == 0, f"rows {bad[:8].tolist()} differ"


@pytest.mark.parametrize("bits", [19, 20])
def test_batched_last_pass_reads_the_n_word_table(oracle, bits):
    """A batch of at least 16 transforms of 2^19 .. 2^24 points runs its last
    column pass from an n-word pre-twiddle table (times n^-1 for the inverse),
    with every row's copy of a tile dispatched back to back.  Forward and
    inverse against the oracle, the same rows as a 15-row batch (the two-level
    table path), an Fp2 batch of 16 rows, and a second call that allocates
    nothing."""
    from volta_mi355x import FP2, Backend
    n = 1 << bits
    host = rand_fp(1900 + bits, (16, n))
    want = oracle.ntt_forward_batch(host)
    want_inv = oracle.ntt_inverse_batch(host)
    with Backend() as b:
        inp = b.upload_device(host.reshape(-1))
        out = b.ntt_fp_batch_device(inp, 16, n)
        assert (b.download_device(out).reshape(16, n) == want).all()
        inv = b.ntt_fp_inverse_batch_device(inp, 16, n)
        assert (b.download_device(inv).reshape(16, n) == want_inv).all()
        # the same transforms again: the tables are cached
        before = b.get_stats()
        for x in (out, inv):
            b.free_device(x)
        out = b.ntt_fp_batch_device(inp, 16, n)
        inv = b.ntt_fp_inverse_batch_device(inp, 16, n)
        after = b.get_stats()
        assert after["allocation_calls"] == before["allocation_calls"]
        assert (b.download_device(out).reshape(16, n) == want).all()
        assert (b.download_device(inv).reshape(16, n) == want_inv).all()
        # fifteen rows take the two-level table
        part = b.ntt_fp_batch_device(inp, 15, n)
        assert (b.download_device(part).reshape(15, n) == want[:15]).all()
        part_inv = b.ntt_fp_inverse_batch_device(inp, 15, n)
        assert (b.download_device(part_inv).reshape(15, n) == want_inv[:15]).all()
        # Fp2 rows: both coordinates through the base-field table
        h2 = rand_fp(2900 + bits, (16, n, 2))
        d2 = b.alloc_device(16 * n, FP2)
        b.upload_into(d2, 0, h2.reshape(-1))
        o2 = b.ntt_fp2_batch_device(d2, 16, n)
        got2 = b.download_device(o2).view(np.uint64).reshape(16, n, 2)
        for comp in (0, 1):
            assert (got2[:, :, comp] == oracle.ntt_forward_batch(h2[:, :, comp].copy())).all()
        ws, res, cached = b.memory_breakdown()
        assert ws + res + cached == b.get_stats()["live_device_bytes"]
        for x in (inp, out, inv, part, part_inv, d2, o2):
            b.free_device(x)
