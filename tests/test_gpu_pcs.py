"""GPU parity of the PCS row primitives through the C ABI: combinations,
messages, powers, adds, gathers, ChaCha8 rows; plus the seam's error and
stats contract (rust/volta-pcs/tests/cuda.rs:186-547 and
rust/volta-accel/src/lib.rs:7587-8435 are the reference's own checks)."""
import numpy as np
import pytest

import spike_inputs as spike

pytestmark = pytest.mark.gpu

P = spike.P


def rand_fp(seed, shape):
    return np.random.Generator(np.random.PCG64(seed)).integers(0, P, size=shape, dtype=np.uint64)


def rand_i16(seed, size):
    return np.random.Generator(np.random.PCG64(seed)).integers(-(1 << 15), 1 << 15, size=size, dtype=np.int16)


# ---- combinations ------------------------------------------------------------------

@pytest.mark.parametrize("rows,cols,pad,comb,w_off", [
    (1, 1, 0, 1, 0), (7, 11, 3, 4, 0), (300, 2048, 0, 2, 0), (129, 13, 5, 3, 1), (1000, 64, 512, 1, 3),
    (4097, 8, 0, 2, 0),
])
def test_combine_rows_device_matches_oracle(backend, oracle, rows, cols, pad, comb, w_off):
    w = rand_i16(rows + cols, rows * cols)
    w[:2] = [-32768, 32767][:w.size]
    pads = rand_fp(rows * 7 + pad, rows * pad) if pad else np.zeros(1, np.uint64)
    co = rand_fp(comb + 99, (comb * rows, 2))
    # a leading offset exercises unaligned weight rows
    dw = backend.alloc_device(w_off + w.size, np.int16)
    backend.upload_into(dw, w_off, w)
    dp, dc = backend.upload_device(pads), backend.upload_device(co.reshape(-1))
    from volta_mi355x import FP2
    dc2 = backend.alloc_device(comb * rows, FP2)
    backend.upload_into(dc2, 0, co.reshape(-1))
    out = backend.pcs_combine_rows_device(dw, w_off, dp, 0, dc2, 0, rows, cols, pad, comb)
    got = backend.download_device(out).view(np.uint64).reshape(comb, cols + pad, 2)
    for b in (dw, dp, dc, dc2, out):
        backend.free_device(b)
    assert (got == oracle.pcs_combine_rows(w, pads, co, rows, cols, pad, comb)).all()


def block_sparse_coefficients(seed, rows, comb):
    """Coefficients as an opening's block claims make them: zero outside a
    block of rows, plus the cases the zero-chunk skip must get right."""
    g = np.random.Generator(np.random.PCG64(seed))
    co = np.zeros((comb, rows, 2), np.uint64)
    # 0: all zero; 1: one aligned block; 2: a block across chunk boundaries;
    # 3: a pair of rows whose coefficients sum to 0 mod p, and a far row;
    # the rest dense
    co[1, 64:96] = g.integers(0, P, size=(32, 2), dtype=np.uint64)
    co[2, 100:300] = g.integers(0, P, size=(200, 2), dtype=np.uint64)
    c = g.integers(1, P, size=2, dtype=np.uint64)
    co[3, 5], co[3, 6] = c, np.uint64(P) - c
    co[3, rows - 1] = g.integers(0, P, size=2, dtype=np.uint64)
    co[4:] = g.integers(0, P, size=(comb - 4, rows, 2), dtype=np.uint64)
    return co.reshape(comb * rows, 2)


@pytest.mark.parametrize("rows,cols,pad,comb", [(4096, 2048, 512, 7), (4096, 2048, 0, 6), (512, 256, 8, 7),
                                               (320, 64, 3, 5)])
def test_combine_rows_with_zero_coefficient_chunks(backend, oracle, rows, cols, pad, comb):
    """Block-claim coefficients (zero outside a block): chunks whose
    coefficients are all zero are skipped, a chunk whose nonzero coefficients
    sum to 0 mod p is not, odd and even combination counts; through the
    allocating and the allocation-free entry points."""
    from volta_mi355x import FP2
    w = rand_i16(rows * comb, rows * cols)
    pads = rand_fp(rows + pad, rows * pad) if pad else np.zeros(1, np.uint64)
    co = block_sparse_coefficients(rows + comb, rows, comb)
    dw, dp, dc = backend.upload_device(w), backend.upload_device(pads), backend.upload_device(co, FP2)
    want = oracle.pcs_combine_rows(w, pads if pad else None, co, rows, cols, pad, comb)
    assert not want[0].any() and want[3].any()
    out = backend.pcs_combine_rows_device(dw, 0, dp, 0, dc, 0, rows, cols, pad, comb)
    got = backend.download_device(out).view(np.uint64).reshape(comb, cols + pad, 2)
    assert (got == want).all()
    # the allocation-free entry, twice: its scratch holds the previous call's
    # partials (the two 4096-row shapes need more partials than it holds at
    # the default row chunks, so they run with larger ones, zero chunks still
    # skipped)
    out2 = backend.alloc_device(comb * (cols + pad), FP2)
    for _ in range(2):
        rc = backend.lib.volta_mi355x_pcs_combine_rows_device_noalloc(
            backend.raw, dw.id, 0, dp.id, 0, dc.id, 0, rows, cols, pad, comb, out2.id, 0)
        assert rc == 0, backend.last_error()
        assert (backend.download_device(out2).view(np.uint64).reshape(comb, cols + pad, 2) == want).all()
    for b in (dw, dp, dc, out, out2):
        backend.free_device(b)


def test_combine_rows_host_entry_point(backend, oracle):
    rows, cols, pad, comb = 33, 40, 6, 2
    w = rand_i16(1, rows * cols)
    pads = rand_fp(2, rows * pad)
    co = rand_fp(3, (comb * rows, 2))
    got = backend.pcs_combine_rows(w, pads, co, rows, cols, pad, comb)
    assert (got == oracle.pcs_combine_rows(w, pads, co, rows, cols, pad, comb)).all()


@pytest.mark.parametrize("rows,cols,expected", spike.COMBINE_GOLDEN)
def test_combine_fp_rows_reference_checksums_on_device(backend, oracle, rows, cols, expected):
    w, q, c = spike.combine_inputs(rows, cols)
    dm = backend.upload_device(w.reshape(-1))
    from volta_mi355x import FP2
    dc = backend.alloc_device(2 * rows, FP2)
    backend.upload_into(dc, 0, np.concatenate([q, c]).reshape(-1))
    out = backend.combine_rows_fp_device(dm, rows, cols, dc, 2)
    u = backend.download_device(out).view(np.uint64).reshape(2, cols, 2)
    for b in (dm, dc, out):
        backend.free_device(b)
    assert spike.combine_checksum(oracle.fnv, u[0], u[1]) == expected


def test_combine_fp_rows_matches_oracle_odd_shape(backend, oracle):
    rows, cols, comb = 257, 37, 3
    m = rand_fp(5, (rows, cols))
    m[0, :3] = [P - 1, P - 1, 0]
    co = rand_fp(6, (comb * rows, 2))
    co[:2] = P - 1
    dm = backend.upload_device(m.reshape(-1))
    from volta_mi355x import FP2
    dc = backend.alloc_device(comb * rows, FP2)
    backend.upload_into(dc, 0, co.reshape(-1))
    out = backend.combine_rows_fp_device(dm, rows, cols, dc, comb)
    got = backend.download_device(out).view(np.uint64).reshape(comb, cols, 2)
    for b in (dm, dc, out):
        backend.free_device(b)
    assert (got == oracle.combine_rows_fp(m, co, comb)).all()


def test_proximity_combinations_c2(backend, oracle):
    """C2's two challenge-power combinations (coefficients c^1..c^rows)."""
    from volta_mi355x import ligero, workloads as W
    cfg = W.CONFIGS["c2"]
    w = W.c2_weights()
    chs = W.challenges_fp2("volta-mi355x/c2/challenges", 2)
    params = ligero.LigeroParams(cfg.rows, 11, 0, 13)
    dw = backend.upload_device(w.reshape(-1))
    out = ligero.proximity_combinations(backend, dw, None, params, chs)
    got = backend.download_device(out).view(np.uint64).reshape(2, cfg.msg_len, 2)
    backend.free_device(dw)
    backend.free_device(out)
    co = np.concatenate([oracle.fp2_powers(tuple(int(x) for x in c), cfg.rows) for c in chs])
    assert (got == oracle.pcs_combine_rows(w, None, co, cfg.rows, cfg.msg_len, 0, 2)).all()


def test_proximity_combinations_c3_full(backend, oracle):
    from volta_mi355x import ligero, workloads as W
    cfg = W.CONFIGS["c3"]
    w = W.c3_weights()
    chs = W.challenges_fp2("volta-mi355x/c3/challenges", 2)
    params = ligero.LigeroParams(cfg.rows, 11, 0, 13)
    dw = backend.upload_device(w.reshape(-1))
    out = ligero.proximity_combinations(backend, dw, None, params, chs)
    got = backend.download_device(out).view(np.uint64).reshape(2, cfg.msg_len, 2)
    backend.free_device(dw)
    backend.free_device(out)
    co = np.concatenate([oracle.fp2_powers(tuple(int(x) for x in c), cfg.rows) for c in chs])
    assert (got == oracle.pcs_combine_rows(w, None, co, cfg.rows, cfg.msg_len, 0, 2)).all()


def test_linearity_ties_combination_to_encode(backend, oracle):
    """The verifier's identity (rust/volta-pcs/src/ligero.rs:1841-1856):
    encode(sum_i r_i m_i) = sum_i r_i encode(m_i)."""
    rows, cols, n = 64, 512, 2048
    w = rand_i16(21, rows * cols)
    co = rand_fp(22, (rows, 2))
    dw, dp = backend.upload_device(w), backend.alloc_device(1, np.uint64)
    from volta_mi355x import FP2
    dc = backend.alloc_device(rows, FP2)
    backend.upload_into(dc, 0, co.reshape(-1))
    enc = backend.pcs_encode_device(dw, 0, dp, 0, rows, cols, 0, n)
    lhs_msg = backend.pcs_combine_rows_device(dw, 0, dp, 0, dc, 0, rows, cols, 0, 1)
    rhs = backend.combine_rows_fp_device(enc, rows, n, dc, 1)
    u = backend.download_device(lhs_msg).view(np.uint64).reshape(cols, 2)
    r = backend.download_device(rhs).view(np.uint64).reshape(n, 2)
    for b in (dw, dp, dc, enc, lhs_msg, rhs):
        backend.free_device(b)
    for comp in (0, 1):
        want = oracle.ntt_encode_batch(u[:, comp].reshape(1, -1).copy(), n)[0]
        assert (r[:, comp] == want).all()


# ---- small primitives ----------------------------------------------------------------

@pytest.mark.parametrize("count", [1, 7, 64, 255, 4097, 70001, (1 << 18) - 1, 1 << 18, 300001])
def test_fp2_powers_counts(backend, oracle, count):
    """c^(i+1) from the three-level table (below 2^18 powers, its last entry
    included) or from the squarings over the set bits of i+1 (2^18 and up):
    a single element, partial blocks and several grid strides match the
    serial powers."""
    c = (123456789123, int(P - 5))
    d = backend.fp2_powers_device(c, count)
    got = backend.download_device(d).view(np.uint64).reshape(-1, 2)
    backend.free_device(d)
    assert (got == oracle.fp2_powers(c, count)).all()


def test_fp2_powers_and_add(backend, oracle):
    c = (int(P - 2), 123456789)
    d = backend.fp2_powers_device(c, 1000)
    got = backend.download_device(d).view(np.uint64).reshape(-1, 2)
    assert (got == oracle.fp2_powers(c, 1000)).all()
    other = rand_fp(8, (1000, 2))
    from volta_mi355x import FP2
    da = backend.alloc_device(1000, FP2)
    backend.upload_into(da, 0, other.reshape(-1))
    backend.fp2_add_inplace_device(d, 10, da, 20, 500)
    after = backend.download_device(d).view(np.uint64).reshape(-1, 2)
    backend.free_device(d)
    backend.free_device(da)
    want = got.copy()
    want[10:510] = oracle.fp2_add_inplace(got[10:510], other[20:520])
    assert (after == want).all()


def test_gather_columns_device_and_host(backend, oracle):
    rows, cols = 64, 1 << 12
    m = rand_fp(9, (rows, cols))
    idx = np.random.Generator(np.random.PCG64(3)).integers(0, cols, size=256, dtype=np.uint32)
    dm = backend.upload_device(m.reshape(-1))
    out = backend.pcs_gather_columns_device(dm, rows, cols, idx)
    got = backend.download_device(out).reshape(256, rows)
    backend.free_device(dm)
    backend.free_device(out)
    assert (got == oracle.gather_columns(m, idx)).all()
    assert (backend.pcs_gather_columns(m, idx) == got).all()
    m2 = rand_fp(10, (rows, 128, 2))
    from volta_mi355x import FP2
    dm2 = backend.alloc_device(rows * 128, FP2)
    backend.upload_into(dm2, 0, m2.reshape(-1))
    idx2 = np.array([127, 0, 5], dtype=np.uint32)
    out2 = backend.pcs_gather_columns_device(dm2, rows, 128, idx2, fp2=True)
    got2 = backend.download_device(out2).view(np.uint64).reshape(3, rows, 2)
    backend.free_device(dm2)
    backend.free_device(out2)
    assert (got2 == oracle.gather_fp2_columns(m2, idx2)).all()


KAT_SEED = bytes((17 * i + 3) % 256 for i in range(32))


def test_chacha8_rows_match_fpstream_and_kat(backend, oracle):
    # rust/volta-accel/src/lib.rs:7517-7528: the 6th raw draw of row 0 is >= p
    d = backend.chacha8_prover_secret_fp_rows_device(KAT_SEED, 0x19664BCA, 3, 10)
    got = backend.download_device(d).reshape(3, 10)
    backend.free_device(d)
    assert (got == oracle.fp_rows(KAT_SEED, 0x19664BCA, 3, 10)).all()
    raw = oracle.raw_u64(KAT_SEED, 0x19664BCA, 8)
    assert int(raw[5]) == 0xFFFF_FFFF_B146_1B28 and int(got[0, 5]) == int(raw[6])
    d2 = backend.chacha8_prover_secret_fp2_rows_padded_device(KAT_SEED, 5, 4, 7, 9)
    got2 = backend.download_device(d2).view(np.uint64).reshape(4, 9, 2)
    backend.free_device(d2)
    assert (got2 == oracle.fp2_rows_padded(KAT_SEED, 5, 4, 7, 9)).all()


# Bernstein ChaCha8, all-zero key and nonce: the published keystream blocks 0
# and 1.  None of these 16 words is >= p, so FpStream row 0 of the zero seed in
# domain 0 is exactly that keystream read as little-endian u64.
ZERO_KEY_BLOCKS_0_1 = bytes.fromhex(
    "3e00ef2f895f40d67f5bb8e81f09a5a12c840ec3ce9a7f3b181be188ef711a1e"
    "984ce172b9216f419f445367456d5619314a42a3da86b001387bfdb80e0cfe42"
    "d2aefa0deaa5c151bf0adb6c01f2a5adc0fd581259f9a2aadcf20f8fd566a26b"
    "5032ec38bbc5da98ee0c6f568b872a65a08abf251deb21bb4b56e5d8821e68aa")


def test_chacha8_device_rows_published_keystream_two_blocks(backend):
    d = backend.chacha8_prover_secret_fp_rows_device(bytes(32), 0, 1, 16)
    got = backend.download_device(d)
    backend.free_device(d)
    assert got.astype("<u8").tobytes() == ZERO_KEY_BLOCKS_0_1


@pytest.mark.parametrize("count", [6, 8, 511, 512, 1000])
def test_chacha8_rows_rejection_shifts_later_draws(backend, oracle, count):
    """Rows are filled by one wave, 64 blocks (512 raw draws) per round.  On
    the reference KAT stream the 6th raw draw of row 0 is rejected, so every
    later value moves up by one: count 8 takes its last value from block 1,
    count 512 from a second round; row 1 has no rejection."""
    d = backend.chacha8_prover_secret_fp_rows_device(KAT_SEED, 0x19664BCA, 2, count)
    got = backend.download_device(d).reshape(2, count)
    backend.free_device(d)
    assert (got == oracle.fp_rows(KAT_SEED, 0x19664BCA, 2, count)).all()
    d2 = backend.chacha8_prover_secret_fp2_rows_padded_device(KAT_SEED, 0x19664BCA, 2, count // 2 + 1, count // 2 + 5)
    got2 = backend.download_device(d2).view(np.uint64).reshape(2, count // 2 + 5, 2)
    backend.free_device(d2)
    assert (got2 == oracle.fp2_rows_padded(KAT_SEED, 0x19664BCA, 2, count // 2 + 1, count // 2 + 5)).all()


@pytest.mark.parametrize("rows,count", [(2, 8192), (3, 33280), (97, 8704), (1, 40000)])
def test_chacha8_long_rows_one_workgroup_each(backend, oracle, rows, count):
    """Few long rows are filled by 16 waves each, 1024 blocks per round; on
    the reference KAT stream row 0 rejects its 6th raw draw, which shifts
    every later place across all waves and rounds."""
    d = backend.chacha8_prover_secret_fp_rows_device(KAT_SEED, 0x19664BCA, rows, count)
    got = backend.download_device(d).reshape(rows, count)
    backend.free_device(d)
    assert (got == oracle.fp_rows(KAT_SEED, 0x19664BCA, rows, count)).all()
    d2 = backend.chacha8_prover_secret_fp2_rows_padded_device(KAT_SEED, 0x19664BCA, rows, count // 2 + 1,
                                                              count // 2 + 3)
    got2 = backend.download_device(d2).view(np.uint64).reshape(rows, count // 2 + 3, 2)
    backend.free_device(d2)
    assert (got2 == oracle.fp2_rows_padded(KAT_SEED, 0x19664BCA, rows, count // 2 + 1, count // 2 + 3)).all()


def test_chacha8_rows_large(backend, oracle):
    seed = bytes(range(32))
    d = backend.chacha8_prover_secret_fp_rows_device(seed, 1000, 513, 512)
    got = backend.download_device(d).reshape(513, 512)
    backend.free_device(d)
    assert (got == oracle.fp_rows(seed, 1000, 513, 512)).all()


# ---- seam contract: errors and stats -------------------------------------------------

def test_host_geometry_whose_byte_counts_overflow(backend):
    """Host-pointer calls whose element counts multiply past 2^64 are refused
    before any staging copy or launch (each factor of a byte count is checked,
    not only the last multiplication)."""
    lib, raw = backend.lib, backend.raw
    w = np.zeros(8, np.int16)
    m = np.zeros(8, np.uint64)
    co = np.zeros(4, np.uint64)
    idx = np.zeros(1, np.uint32)
    out = np.zeros(64, np.uint64)
    big = 1 << 62
    assert lib.volta_cuda_pcs_combine_rows(raw, w.ctypes.data, None, co.ctypes.data, big, 8, 0, 1,
                                           out.ctypes.data) != 0
    assert "overflows size_t" in backend.last_error()
    assert lib.volta_cuda_pcs_combine_rows(raw, w.ctypes.data, m.ctypes.data, co.ctypes.data, 4, 2, big, 1,
                                           out.ctypes.data) != 0
    assert "overflows size_t" in backend.last_error()
    assert lib.volta_cuda_pcs_gather_columns(raw, m.ctypes.data, big, 8, idx.ctypes.data, 1, out.ctypes.data) != 0
    assert "overflows size_t" in backend.last_error()
    assert lib.volta_cuda_hash_fp_columns(raw, m.ctypes.data, big, 16, out.ctypes.data) != 0
    assert "overflows size_t" in backend.last_error()


def test_geometry_and_id_errors(backend):
    from volta_mi355x import GpuError, InvalidInput
    buf = backend.alloc_device(16, np.uint64)
    out = backend.alloc_device(16, np.uint64)
    lib, raw = backend.lib, backend.raw
    assert lib.volta_cuda_ntt_fp_batch_device(raw, buf.id, 0, 1, 12, out.id, 0) != 0  # n not a power of two
    assert "invalid resident Fp NTT geometry" in backend.last_error()
    assert lib.volta_cuda_ntt_fp_batch_device(raw, buf.id, 0, 2, 16, out.id, 0) != 0  # region too small
    assert "out of bounds" in backend.last_error()
    stale = buf.id
    backend.free_device(buf)
    assert lib.volta_cuda_ntt_fp_batch_device(raw, stale, 0, 1, 16, out.id, 0) != 0
    assert "unknown resident buffer id" in backend.last_error()
    assert lib.volta_cuda_resident_free(raw, stale) != 0
    # storage is reused under a new generation; the stale id stays invalid
    again = backend.alloc_device(16, np.uint64)
    assert again.id != stale
    assert lib.volta_cuda_resident_zero(raw, stale, 0, 8) != 0
    with pytest.raises(InvalidInput):
        backend.pcs_messages_device(again, 0, again, 0, 1, 8, 0, 4)  # cols > code_len
    assert lib.volta_cuda_pcs_combine_rows_device(raw, again.id, 0, again.id, 0, again.id, 0, 0, 1, 0, 1, out.id,
                                                  0) != 0
    # mock-correlation domains must not set the reserved bits
    seed = (np.ctypeslib.as_ctypes(np.zeros(32, np.uint8)))
    assert lib.volta_cuda_mock_correlation_sub_masks_device(raw, out.id, 0, seed, 1 << 61, 1, 1) != 0
    assert "reserved correlation bits" in backend.last_error()
    assert lib.volta_cuda_chacha8_prover_secret_fp_rows_device(raw, out.id, 0, seed, 0, 0, 1) != 0
    # out-of-scope symbols fail explicitly
    import ctypes
    assert lib.volta_cuda_x4c_arena_reset(raw, ctypes.c_uint64(out.id), ctypes.c_size_t(0), ctypes.c_size_t(16),
                                          ctypes.c_int(0)) != 0
    assert "not implemented" in backend.last_error()
    backend.free_device(again)
    backend.free_device(out)
    with pytest.raises(GpuError):
        backend._check(lib.volta_cuda_resident_free(raw, 12345))


def test_stats_contract_of_a_cold_encode():
    """Mirrors rust/volta-pcs/tests/cuda.rs:235-244: a cold context uploads
    exactly the n/2 twiddle table (the only H2D besides explicit uploads) and
    generated pads count rows*pad*8 bytes."""
    from volta_mi355x import Backend, ligero
    with Backend() as b:
        rows, cols, pad, n = 16, 64, 8, 256
        w = rand_i16(40, rows * cols)
        dw = b.upload_device(w)
        b.reset_stats()
        params = ligero.LigeroParams(rows, 6, pad, 8)
        enc, pads = ligero.commit_encode_resident(b, dw, params, pad_seed=bytes(32), fused=False)
        s = b.get_stats()
        assert s["h2d_bytes"] == n // 2 * 8
        assert s["d2h_bytes"] == 0
        assert s["device_generated_bytes"] == rows * pad * 8
        assert s["calls"]["pcs_ntt"] == 1 and s["calls"]["pcs_rows"] == 2
        assert s["kernel_ns"]["pcs_ntt"] > 0
        # a second encode of the same size uploads nothing
        b.reset_stats()
        enc2, pads2 = ligero.commit_encode_resident(b, dw, params, pad_seed=bytes(32), fused=True)
        s2 = b.get_stats()
        assert s2["h2d_bytes"] == 0 and s2["calls"]["pcs_ntt"] == 1
        assert (b.download_device(enc) == b.download_device(enc2)).all()
        for x in (dw, enc, pads, enc2, pads2):
            b.free_device(x)
        live = b.get_stats()["live_device_bytes"]
        ws, res, cached = b.memory_breakdown()
        assert ws + res + cached == live and res == 0


def test_deferred_timing_records_the_events_it_reads():
    """Deferred events (policy 0): a device-only primitive records its two
    kernel markers and nothing else, and at the flush one elapsed-time query.
    When the previous record's closing marker is the last thing on the stream
    and the device has not reached it, that marker opens the next record (one
    event-state query instead of a second record); otherwise the call records
    both markers after that query.  A host-pointer primitive also times its
    upload and download (h2d_ns, d2h_ns)."""
    from volta_mi355x import FP2, Backend
    with Backend(timing_policy=0) as b:
        a, t = b.alloc_device(64, FP2), b.alloc_device(64, FP2)
        b.zero_device(a, 0, 64)
        b.zero_device(t, 0, 64)
        L, r = b.lib, b.raw
        for _ in range(600):  # every ring slot has its events created
            assert L.volta_cuda_fp2_add_inplace_device(r, t.id, 0, a.id, 0, 64) == 0
        s0 = b.get_stats()
        for _ in range(100):
            assert L.volta_cuda_fp2_add_inplace_device(r, t.id, 0, a.id, 0, 64) == 0
        s1 = b.get_stats()
        calls = s1["timing_event_api_calls"] - s0["timing_event_api_calls"]
        assert 100 * 3 <= calls <= 100 * 4 - 1  # the first call after the stats read has nothing to borrow
        assert s1["timing_records"] - s0["timing_records"] == 100
        assert s1["h2d_ns"] == s0["h2d_ns"] and s1["d2h_ns"] == s0["d2h_ns"]
        msgs = rand_fp(5, (4, 300))
        got = b.ntt_fp_batch(msgs, 4, 300, 1 << 10)
        s2 = b.get_stats()
        assert s2["h2d_ns"] > s1["h2d_ns"] and s2["d2h_ns"] > s1["d2h_ns"]
        assert s2["kernel_ns"]["pcs_ntt"] > s1["kernel_ns"]["pcs_ntt"]
        for x in (a, t):
            b.free_device(x)
    assert got.shape == (4, 1 << 10)


def test_deferred_timing_borrows_markers_only_while_the_device_is_behind():
    """Calls enqueued faster than the device runs them open with the previous
    call's closing marker: one record, one state query and one elapsed query
    per call.  Calls separated by host idle time record their own opening
    marker, so the idle time is no kernel's (kernel_ns stays far below it)."""
    import time
    from volta_mi355x import FP2, Backend
    n = 1 << 22  # 64 MiB per operand: each add runs tens of microseconds on the device
    with Backend(timing_policy=0) as b:
        a, t = b.alloc_device(n, FP2), b.alloc_device(n, FP2)
        b.zero_device(a, 0, n)
        b.zero_device(t, 0, n)
        L, r = b.lib, b.raw
        for _ in range(600):  # every ring slot has its events created
            assert L.volta_cuda_fp2_add_inplace_device(r, t.id, 0, a.id, 0, 64) == 0
        s0 = b.get_stats()
        for _ in range(100):
            assert L.volta_cuda_fp2_add_inplace_device(r, t.id, 0, a.id, 0, n) == 0
        s1 = b.get_stats()
        calls = s1["timing_event_api_calls"] - s0["timing_event_api_calls"]
        assert s1["timing_records"] - s0["timing_records"] == 100
        assert calls <= 100 * 3 + 10, calls  # nearly every call borrowed its opening marker
        busy = s1["kernel_ns"]["pcs_rows"] - s0["kernel_ns"]["pcs_rows"]
        assert busy > 0
        for _ in range(20):
            assert L.volta_cuda_fp2_add_inplace_device(r, t.id, 0, a.id, 0, 64) == 0
            b.synchronize()
            time.sleep(0.005)
        s2 = b.get_stats()
        idle = s2["kernel_ns"]["pcs_rows"] - s1["kernel_ns"]["pcs_rows"]
        assert s2["timing_records"] - s1["timing_records"] == 20
        assert idle < 20 * 1_000_000, idle  # 20 tiny kernels, not 100 ms of host sleep
        for x in (a, t):
            b.free_device(x)


def test_deferred_messages_call_has_no_record():
    """A messages call that only records its rows (the deferred commit path)
    runs nothing on the device: it is counted as a call but takes no timing
    record and no event, and the transform after it is timed as usual."""
    from volta_mi355x import Backend
    rows, cols, n = 64, 2048, 8192
    w = rand_i16(41, rows * cols)
    with Backend(timing_policy=0) as b:
        dw, dp = b.upload_device(w), b.alloc_device(1, np.uint64)
        out = b.alloc_device(rows * n, np.uint64)
        b.synchronize()
        b.reset_stats()
        m = b.pcs_messages_device(dw, 0, dp, 0, rows, cols, 0, n)
        s = b.get_stats()
        assert s["calls"]["pcs_rows"] == 1 and s["timing_records"] == 0 and s["kernel_ns"]["pcs_rows"] == 0
        assert s["timing_event_api_calls"] == 0
        assert b.lib.volta_cuda_ntt_fp_batch_device(b.raw, m.id, 0, rows, n, out.id, 0) == 0
        s = b.get_stats()
        assert s["calls"]["pcs_ntt"] == 1 and s["timing_records"] == 1 and s["kernel_ns"]["pcs_ntt"] > 0
        for x in (m, dw, dp, out):
            b.free_device(x)


def test_coarse_timing_scope_and_wall_only_policy():
    import ctypes
    from volta_mi355x import Backend
    with Backend(timing_policy=1) as b:
        d = b.alloc_device(1 << 12, np.uint64)
        b.reset_stats()
        lib, raw = b.lib, b.raw
        assert lib.volta_cuda_begin_coarse_timing(raw, 3) == 0
        assert lib.volta_cuda_begin_coarse_timing(raw, 3) != 0  # no nesting
        out_id = ctypes.c_uint64()
        assert lib.volta_cuda_resident_alloc(raw, 8, ctypes.byref(out_id)) != 0
        assert "coarse timing scope" in b.last_error()
        assert lib.volta_cuda_end_coarse_timing(raw) == 0
        o2 = b.ntt_fp_batch_device(d, 1, 1 << 12)
        s = b.get_stats()
        assert s["timing_mode"] == 4 and s["timing_event_api_calls"] == 0
        assert s["calls"]["pcs_ntt"] == 1 and s["kernel_ns"]["pcs_ntt"] == 0
        assert s["coarse_timing_scopes"] == 1
        b.free_device(d)
        b.free_device(o2)


# ---- opening-path helpers ----------------------------------------------------------------

@pytest.mark.parametrize("rows,dims", [(1, 0), (3, 1), (2, 3), (4, 4), (5, 7), (2, 12), (1, 18), (1, 5), (1, 9),
                                       (1, 11), (7, 6), (96, 13)])
def test_eq_rows_match_oracle(backend, oracle, rows, dims):
    from volta_mi355x import FP2
    pts = rand_fp(rows * 100 + dims, (rows * dims, 2)) if dims else None
    dp = backend.upload_device(pts, FP2) if dims else None
    out = backend.logup_eq_rows_device(dp, rows, dims)
    got = backend.download_device(out).view(np.uint64).reshape(rows, 1 << dims, 2)
    backend.free_device(out)
    if dp is not None:
        backend.free_device(dp)
    want = oracle.eq_rows(pts if dims else np.zeros((0, 2), np.uint64), rows, dims)
    assert (got == want).all()


def test_equality_weights_and_row_dots_evaluate_an_mle(backend, oracle):
    """The opening's use (ligero.rs:1300-1400): eq weights of a point dotted
    with a row give the row's multilinear extension at that point."""
    from volta_mi355x import FP2
    dims, rows = 6, 3
    point = rand_fp(41, (dims, 2))
    weights = backend.equality_weights_device(point)
    vals = rand_fp(42, (rows * 80, 2))  # rows of 64 values at stride 80
    dv = backend.alloc_device(rows * 80, FP2)
    backend.upload_into(dv, 0, vals.reshape(-1))
    # b stride 0 is not allowed (stride >= len): replicate the weights per row
    w = backend.download_device(weights).view(np.uint64).reshape(-1, 2)
    dw = backend.upload_device(np.tile(w, (rows, 1)), FP2)
    out = backend.fp2_row_dots_device(dv, 0, 80, dw, 0, 64, rows, 64)
    got = backend.download_device(out).view(np.uint64).reshape(rows, 2)
    for x in (weights, dv, dw, out):
        backend.free_device(x)
    assert (w.reshape(1, 64, 2) == oracle.eq_rows(point, 1, dims)).all()
    assert (got == oracle.fp2_row_dots(vals, 80, np.tile(w, (rows, 1)), 64, rows, 64)).all()

    # independent of the table: fold row 0 by the coordinates, LSB first,
    # f'(y) = f(2y) (1 - p_k) + f(2y + 1) p_k, in big integers
    def mul(a, b):
        return ((a[0] * b[0] + 7 * a[1] * b[1]) % P, (a[0] * b[1] + a[1] * b[0]) % P)

    f = [(int(v[0]), int(v[1])) for v in vals[:64]]
    for k in range(dims):
        pk = (int(point[k][0]), int(point[k][1]))
        one_minus = ((1 - pk[0]) % P, (-pk[1]) % P)
        f = [tuple((x + y) % P for x, y in zip(mul(f[2 * i], one_minus), mul(f[2 * i + 1], pk)))
             for i in range(len(f) // 2)]
    assert tuple(int(v) for v in got[0]) == f[0]


@pytest.mark.parametrize("rows,length,sa,sb,a_off", [(1, 1, 1, 1, 0), (7, 300, 301, 310, 5), (40, 2048, 2048, 4096, 0),
                                                      (3, 70000, 70000, 70000, 1)])
def test_fp2_row_dots_match_oracle(backend, oracle, rows, length, sa, sb, a_off):
    from volta_mi355x import FP2
    a = rand_fp(rows + length, (a_off + (rows - 1) * sa + length, 2))
    b = rand_fp(rows * 3 + length, ((rows - 1) * sb + length, 2))
    da, db = backend.upload_device(a, FP2), backend.upload_device(b, FP2)
    out = backend.fp2_row_dots_device(da, a_off, sa, db, 0, sb, rows, length)
    got = backend.download_device(out).view(np.uint64).reshape(rows, 2)
    for x in (da, db, out):
        backend.free_device(x)
    assert (got == oracle.fp2_row_dots(a[a_off:], sa, b, sb, rows, length)).all()


def test_opening_helper_errors(backend):
    from volta_mi355x import FP2
    lib, raw = backend.lib, backend.raw
    a = backend.alloc_device(64, FP2)
    # output overlapping an input
    assert lib.volta_cuda_fp2_row_dots_device(raw, a.id, 0, 8, a.id, 0, 8, a.id, 2, 2, 8) != 0
    assert "overlaps" in backend.last_error()
    assert lib.volta_cuda_fp2_row_dots_device(raw, a.id, 0, 4, a.id, 0, 8, a.id, 40, 2, 8) != 0  # stride < len
    assert "geometry" in backend.last_error()
    assert lib.volta_cuda_logup_eq_rows_device(raw, 0, 0, 1, 3, a.id, 0) != 0  # dims without points
    assert "geometry" in backend.last_error()
    assert lib.volta_cuda_logup_eq_rows_device(raw, a.id, 0, 1, 8, a.id, 0) != 0  # 256 outputs > 64 slots
    backend.free_device(a)


# ---- host-pointer calls whose copies take the pinned staging (32 MiB and up) ----------

def test_resident_round_trip_staged(backend):
    """A 40 MiB + 8 B upload and download through the resident buffer API at
    an element offset: both copies go through the pinned staging buffers
    (three chunks, the last short); the download equals what was uploaded,
    and the words around the region are untouched."""
    n, off = (40 << 20) // 8 + 1, 3
    data = rand_fp(9100, n)
    d = backend.alloc_device(n + off + 2, np.uint64)
    backend.zero_device(d, 0, n + off + 2)
    backend.upload_into(d, off, data)
    back = backend.download_device(d, off, n)
    edges = backend.download_device(d, 0, n + off + 2)
    backend.free_device(d)
    assert (back == data).all()
    assert not edges[:off].any() and not edges[off + n:].any()


def test_host_combination_staged_upload(backend, oracle):
    """The host row combination (volta_cuda_pcs_combine_rows) with 64 MiB of
    i16 weights and pads: the weights' upload goes through the staging."""
    rows, cols, pad, comb = 16384, 2048, 8, 2
    w = rand_i16(9200, rows * cols)
    pads = rand_fp(9201, rows * pad)
    co = rand_fp(9202, (comb * rows, 2))
    got = backend.pcs_combine_rows(w, pads, co, rows, cols, pad, comb)
    assert (got == oracle.pcs_combine_rows(w, pads, co, rows, cols, pad, comb)).all()


def test_resident_round_trip_from_pinned_host_memory(backend):
    """A 40 MiB upload and download whose host buffers the caller pinned
    (hipHostMalloc from the HIP runtime the library uses): copied directly,
    no staging; the download equals the upload, and a launch after the copies
    reports no stale error."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipHostMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t, ctypes.c_uint]
    hip.hipHostFree.argtypes = [ctypes.c_void_p]
    n = (40 << 20) // 8
    ptrs = [ctypes.c_void_p(), ctypes.c_void_p()]
    for q in ptrs:
        assert hip.hipHostMalloc(ctypes.byref(q), n * 8, 0) == 0
    try:
        src = np.ctypeslib.as_array((ctypes.c_uint64 * n).from_address(ptrs[0].value))
        dst = np.ctypeslib.as_array((ctypes.c_uint64 * n).from_address(ptrs[1].value))
        src[:] = rand_fp(9400, n)
        dst[:] = 0
        d = backend.alloc_device(n, np.uint64)
        assert backend.lib.volta_cuda_resident_upload(backend.raw, d.id, 0, ptrs[0].value, n * 8) == 0, \
            backend.last_error()
        assert backend.lib.volta_cuda_resident_download(backend.raw, d.id, 0, ptrs[1].value, n * 8) == 0, \
            backend.last_error()
        assert (src == dst).all()
        out = backend.ntt_fp_batch_device(d, 1 << 10, 1 << 12)  # launches after the copies
        backend.free_device(out)
        backend.free_device(d)
    finally:
        for q in ptrs:
            hip.hipHostFree(q)
