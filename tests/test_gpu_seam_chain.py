"""The reference's commit chain through its unchanged calls:
pcs_messages_device then ntt_fp_batch_device on the message rows
(finish_resident_commit, rust/volta-pcs/src/ligero.rs:477-496).

The library records the message rows instead of writing them; a forward NTT
of exactly those rows encodes from the weights and pads in one pass, and any
other access writes the rows first.  Every ordering below must give what the
written rows would give: the oracle's messages and codewords."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

P = 0xFFFF_FFFF_0000_0001


def rand_i16(seed, size):
    return np.random.Generator(np.random.PCG64(seed)).integers(-(1 << 15), 1 << 15, size=size, dtype=np.int16)


def rand_fp(seed, shape):
    return np.random.Generator(np.random.PCG64(seed)).integers(0, P, size=shape, dtype=np.uint64)


def setup(backend, rows, cols, pad, seed):
    w = rand_i16(seed, rows * cols)
    pads = rand_fp(seed + 1, rows * pad) if pad else np.zeros(1, np.uint64)
    return w, pads, backend.upload_device(w), backend.upload_device(pads)


@pytest.mark.parametrize("rows,cols,pad,bits", [(64, 2048, 0, 13), (9, 2048, 512, 13), (5, 8192, 512, 15),
                                                (3, 100, 7, 8), (2, 32768, 512, 17)])
def test_chain_encodes_and_rows_materialise_afterwards(backend, oracle, rows, cols, pad, bits):
    n = 1 << bits
    w, pads, dw, dp = setup(backend, rows, cols, pad, rows * bits)
    msgs = backend.pcs_messages_device(dw, 0, dp, 0, rows, cols, pad, n)
    enc = backend.ntt_fp_batch_device(msgs, rows, n)
    got_enc = backend.download_device(enc).reshape(rows, n)
    got_msgs = backend.download_device(msgs).reshape(rows, n)  # written on this first read
    for b in (dw, dp, msgs, enc):
        backend.free_device(b)
    assert (got_enc == oracle.pcs_encode_i16(w, pads, rows, cols, pad, n)).all()
    assert (got_msgs == oracle.pcs_messages(w, pads, rows, cols, pad, n)).all()


def test_rows_read_before_the_transform_are_written(backend, oracle):
    rows, cols, pad, n = 16, 2048, 0, 8192
    w, pads, dw, dp = setup(backend, rows, cols, pad, 7)
    msgs = backend.pcs_messages_device(dw, 0, dp, 0, rows, cols, pad, n)
    part = backend.download_device(msgs, 3 * n, 2 * n).reshape(2, n)
    enc = backend.ntt_fp_batch_device(msgs, rows, n)  # the rows exist now: the plain transform
    got = backend.download_device(enc).reshape(rows, n)
    for b in (dw, dp, msgs, enc):
        backend.free_device(b)
    assert (part == oracle.pcs_messages(w, pads, rows, cols, pad, n)[3:5]).all()
    assert (got == oracle.pcs_encode_i16(w, pads, rows, cols, pad, n)).all()


def test_sources_overwritten_or_freed_after_the_messages_call(backend, oracle):
    """The rows are a function of the sources at the time of the messages
    call: a later upload into the weights, or freeing them, must not change
    what the transform encodes."""
    rows, cols, pad, n = 8, 1000, 24, 4096
    w, pads, dw, dp = setup(backend, rows, cols, pad, 11)
    msgs = backend.pcs_messages_device(dw, 0, dp, 0, rows, cols, pad, n)
    w2, p2 = rand_i16(12, rows * cols), rand_fp(13, rows * pad)
    backend.upload_into(dw, 0, w2)  # new weights after the call
    backend.upload_into(dp, 0, p2)
    enc = backend.ntt_fp_batch_device(msgs, rows, n)
    want = oracle.pcs_encode_i16(w, pads, rows, cols, pad, n)
    assert (backend.download_device(enc).reshape(rows, n) == want).all()
    msgs2 = backend.pcs_messages_device(dw, 0, dp, 0, rows, cols, pad, n)
    backend.free_device(dw)  # frees a source of the recorded rows
    backend.free_device(dp)
    enc2 = backend.ntt_fp_batch_device(msgs2, rows, n)
    got2 = backend.download_device(enc2).reshape(rows, n)
    for b in (msgs, enc, msgs2, enc2):
        backend.free_device(b)
    assert (got2 == oracle.pcs_encode_i16(w2, p2, rows, cols, pad, n)).all()


def test_transforms_that_do_not_match_the_recorded_rows(backend, oracle):
    """A transform of a sub-range of the rows, of another size, or writing
    over the weights, runs on the written rows."""
    rows, cols, pad, n = 12, 2048, 0, 8192
    w, pads, dw, dp = setup(backend, rows, cols, pad, 21)
    want_m = oracle.pcs_messages(w, pads, rows, cols, pad, n)
    msgs = backend.pcs_messages_device(dw, 0, dp, 0, rows, cols, pad, n)
    sub = backend.alloc_device(3 * n, np.uint64)
    assert backend.lib.volta_cuda_ntt_fp_batch_device(backend.raw, msgs.id, 4 * n, 3, n, sub.id, 0) == 0
    assert (backend.download_device(sub).reshape(3, n) == oracle.ntt_forward_batch(want_m[4:7])).all()
    # the rows written by the mismatch stay valid for a later exact transform
    enc = backend.ntt_fp_batch_device(msgs, rows, n)
    assert (backend.download_device(enc).reshape(rows, n) == oracle.ntt_forward_batch(want_m)).all()
    # a D2D read of the rows writes them first
    msgs2 = backend.pcs_messages_device(dw, 0, dp, 0, 1, cols, pad, n)
    row = backend.alloc_device(n, np.uint64)
    backend.copy_device_rows(msgs2, 0, n, row, 0, n, 1, n)
    assert (backend.download_device(row) == want_m[0]).all()
    for b in (dw, dp, msgs, sub, enc, msgs2, row):
        backend.free_device(b)


def test_transform_writing_into_the_weights_buffer(backend, oracle):
    """Codewords written into the buffer that holds the weights (after them):
    the fused read of the weights would race with those stores, so the rows
    are written and the plain transform runs."""
    rows, cols, n = 4, 2048, 8192
    w = rand_i16(41, rows * cols)
    w_u64 = rows * cols * 2 // 8
    buf = backend.alloc_device(4 * (w_u64 + rows * n), np.int16)  # i16 view: weights then codewords
    backend.upload_into(buf, 0, w)
    dp = backend.alloc_device(1, np.uint64)
    msgs = backend.pcs_messages_device(buf, 0, dp, 0, rows, cols, 0, n)
    assert backend.lib.volta_cuda_ntt_fp_batch_device(backend.raw, msgs.id, 0, rows, n, buf.id, w_u64) == 0, \
        backend.last_error()
    got = backend.download_device(buf, 4 * w_u64, 4 * rows * n).view(np.uint64).reshape(rows, n)
    for b in (buf, dp, msgs):
        backend.free_device(b)
    assert (got == oracle.pcs_encode_i16(w, None, rows, cols, 0, n)).all()


def test_stats_of_the_chain_are_those_of_two_calls():
    """One PcsRows call for the messages, one PcsNtt call for the transform,
    the twiddle upload as the only H2D of a cold context (tests/cuda.rs:235-244)."""
    from volta_mi355x import Backend
    rows, cols, n = 32, 2048, 8192
    w = rand_i16(31, rows * cols)
    with Backend() as b:
        dw, dp = b.upload_device(w), b.alloc_device(1, np.uint64)
        b.reset_stats()
        msgs = b.pcs_messages_device(dw, 0, dp, 0, rows, cols, 0, n)
        enc = b.ntt_fp_batch_device(msgs, rows, n)
        b.free_device(msgs)
        s = b.get_stats()
        assert s["calls"]["pcs_rows"] == 1 and s["calls"]["pcs_ntt"] == 1
        assert s["h2d_bytes"] == n // 2 * 8 and s["d2h_bytes"] == 0
        assert s["kernel_ns"]["pcs_ntt"] > 0
        for x in (dw, dp, enc):
            b.free_device(x)


def test_two_recorded_message_calls_and_unrelated_calls_between(backend, oracle):
    """A second messages call into another buffer writes the first rows; calls
    that touch neither the rows' buffer nor their sources leave the rows
    recorded; reading the weights does not write them, overwriting does."""
    rows, cols, pad, n = 6, 2048, 0, 8192
    w, pads, dw, dp = setup(backend, rows, cols, pad, 51)
    want_m = oracle.pcs_messages(w, pads, rows, cols, pad, n)
    want_e = oracle.ntt_forward_batch(want_m)
    m1 = backend.pcs_messages_device(dw, 0, dp, 0, rows, cols, pad, n)
    m2 = backend.pcs_messages_device(dw, 0, dp, 0, rows, cols, pad, n)  # m1 is written now
    c = backend.fp2_powers_device((3, 4), rows)  # unrelated
    u = backend.pcs_combine_rows_device(dw, 0, dp, 0, c, 0, rows, cols, pad, 1)  # reads the weights
    e2 = backend.ntt_fp_batch_device(m2, rows, n)
    e1 = backend.ntt_fp_batch_device(m1, rows, n)
    assert (backend.download_device(m1).reshape(rows, n) == want_m).all()
    assert (backend.download_device(e1).reshape(rows, n) == want_e).all()
    assert (backend.download_device(e2).reshape(rows, n) == want_e).all()
    # the same rows recorded again into the same region replace the record
    assert backend.lib.volta_cuda_pcs_messages_device(backend.raw, dw.id, 0, dp.id, 0, rows, cols, pad, n, m2.id,
                                                      0) == 0
    assert backend.lib.volta_cuda_pcs_messages_device(backend.raw, dw.id, 0, dp.id, 0, rows, cols, pad, n, m2.id,
                                                      0) == 0
    backend.upload_into(dw, 0, np.zeros(rows * cols, np.int16))  # overwriting a source writes the rows first
    assert (backend.download_device(m2).reshape(rows, n) == want_m).all()
    got_u = backend.download_device(u).view(np.uint64).reshape(1, cols, 2)
    co = oracle.fp2_powers((3, 4), rows)
    for b in (dw, dp, m1, m2, c, u, e1, e2):
        backend.free_device(b)
    assert (got_u == oracle.pcs_combine_rows(w, None, co, rows, cols, pad, 1)).all()


def _hip():
    """The HIP runtime the library already loaded, for copies through raw
    device addresses (what a harness's own kernels would do)."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so", mode=ctypes.RTLD_GLOBAL)
    hip.hipMemcpy.restype = ctypes.c_int
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    return hip


HIP_H2D, HIP_D2H = 1, 2


def test_rows_buffer_address_taken_before_the_messages_call(backend, oracle):
    """A harness that holds the rows' device address before the messages call
    can read the rows with its own kernels: the call must write them at once
    (the buffer is marked by the address query), and the transform then runs
    on the written rows."""
    import ctypes
    rows, cols, pad, n = 8, 2048, 0, 8192
    w, pads, dw, dp = setup(backend, rows, cols, pad, 61)
    msgs = backend.alloc_device(rows * n, np.uint64)
    ptr = backend.device_ptr(msgs)
    assert backend.lib.volta_cuda_pcs_messages_device(backend.raw, dw.id, 0, dp.id, 0, rows, cols, pad, n, msgs.id,
                                                      0) == 0, backend.last_error()
    backend.synchronize()
    host = np.empty(rows * n, np.uint64)
    assert _hip().hipMemcpy(host.ctypes.data, ctypes.c_void_p(ptr), host.nbytes, HIP_D2H) == 0
    enc = backend.ntt_fp_batch_device(msgs, rows, n)
    got = backend.download_device(enc).reshape(rows, n)
    for b in (dw, dp, msgs, enc):
        backend.free_device(b)
    assert (host.reshape(rows, n) == oracle.pcs_messages(w, pads, rows, cols, pad, n)).all()
    assert (got == oracle.pcs_encode_i16(w, pads, rows, cols, pad, n)).all()


@pytest.mark.parametrize("pad", [0, 512])
def test_source_address_taken_before_the_messages_call(backend, oracle, pad):
    """The weights (and pads) overwritten through a raw address after the
    messages call: the rows are those of the sources at the time of the call,
    so the call wrote them at once and the transform encodes those rows."""
    import ctypes
    rows, cols, n = 6, 2048, 8192 if pad == 0 else 1 << 15
    w, pads, dw, dp = setup(backend, rows, cols, pad, 71 + pad)
    wptr = backend.device_ptr(dw)
    pptr = backend.device_ptr(dp) if pad else None
    msgs = backend.pcs_messages_device(dw, 0, dp, 0, rows, cols, pad, n)
    backend.synchronize()
    hip = _hip()
    junk = rand_i16(99, rows * cols)
    assert hip.hipMemcpy(ctypes.c_void_p(wptr), junk.ctypes.data, junk.nbytes, HIP_H2D) == 0
    if pad:
        junk_p = rand_fp(98, rows * pad)
        assert hip.hipMemcpy(ctypes.c_void_p(pptr), junk_p.ctypes.data, junk_p.nbytes, HIP_H2D) == 0
    enc = backend.ntt_fp_batch_device(msgs, rows, n)
    got = backend.download_device(enc).reshape(rows, n)
    for b in (dw, dp, msgs, enc):
        backend.free_device(b)
    assert (got == oracle.pcs_encode_i16(w, pads if pad else None, rows, cols, pad, n)).all()


@pytest.mark.parametrize("bits", [13, 15])
def test_transform_writing_into_the_pads_buffer(backend, oracle, bits):
    """Codewords written into the buffer that holds the pads (after them),
    pad > 0: the fused encode would read the pads while its stores land in
    the same buffer, so the rows are written and the plain transform runs."""
    rows, cols, pad, n = 5, 2048, 512, 1 << bits
    w = rand_i16(81 + bits, rows * cols)
    pads = rand_fp(82 + bits, rows * pad)
    dw = backend.upload_device(w)
    buf = backend.alloc_device(rows * pad + rows * n, np.uint64)  # pads, then the codewords
    backend.upload_into(buf, 0, pads)
    msgs = backend.pcs_messages_device(dw, 0, buf, 0, rows, cols, pad, n)
    assert backend.lib.volta_cuda_ntt_fp_batch_device(backend.raw, msgs.id, 0, rows, n, buf.id, rows * pad) == 0, \
        backend.last_error()
    got = backend.download_device(buf, rows * pad, rows * n).reshape(rows, n)
    left = backend.download_device(buf, 0, rows * pad)
    got_m = backend.download_device(msgs).reshape(rows, n)
    for b in (dw, buf, msgs):
        backend.free_device(b)
    assert (left == pads).all()
    assert (got_m == oracle.pcs_messages(w, pads, rows, cols, pad, n)).all()
    assert (got == oracle.pcs_encode_i16(w, pads, rows, cols, pad, n)).all()


@pytest.mark.parametrize("rows,cols,pad,bits", [(16, 2048, 0, 13), (6, 2048, 512, 13), (4, 8192, 512, 15)])
def test_written_rows_transform_and_a_later_write_into_their_tail(backend, oracle, rows, cols, pad, bits):
    """Rows read back before the transform are written by the library, which
    then knows their zero tail and transforms only their nonzero prefix; an
    upload into a tail afterwards (any write to the buffer) ends that
    knowledge, and the next transform reads the whole rows."""
    n = 1 << bits
    w, pads, dw, dp = setup(backend, rows, cols, pad, 90 + bits + pad)
    msgs = backend.pcs_messages_device(dw, 0, dp, 0, rows, cols, pad, n)
    part = backend.download_device(msgs, 0, 8)  # a read: the rows are written now
    enc1 = backend.ntt_fp_batch_device(msgs, rows, n)
    want_m = oracle.pcs_messages(w, pads if pad else None, rows, cols, pad, n)
    tail = rand_fp(91, 5)
    backend.upload_into(msgs, (rows - 1) * n + n - 5, tail)  # into the last row's zero tail
    enc2 = backend.ntt_fp_batch_device(msgs, rows, n)
    got1 = backend.download_device(enc1).reshape(rows, n)
    got2 = backend.download_device(enc2).reshape(rows, n)
    for b in (dw, dp, msgs, enc1, enc2):
        backend.free_device(b)
    assert (part == want_m.reshape(-1)[:8]).all()
    assert (got1 == oracle.ntt_forward_batch(want_m)).all()
    want_m[rows - 1, n - 5:] = tail
    assert (got2 == oracle.ntt_forward_batch(want_m)).all()


@pytest.mark.parametrize("policy", [0, 1])
def test_late_row_write_is_timed_as_the_messages_kernel(policy):
    """Rows written late (here by a read of their buffer) are the messages
    call's kernel: PcsRows gains their kernel time but no second call, under
    the per-primitive timing policy and under the report's wall-only counters
    (which time nothing)."""
    from volta_mi355x import Backend
    rows, cols, n = 64, 2048, 8192
    w = rand_i16(33, rows * cols)
    with Backend(timing_policy=policy) as b:
        dw, dp = b.upload_device(w), b.alloc_device(1, np.uint64)
        b.synchronize()
        b.reset_stats()
        msgs = b.pcs_messages_device(dw, 0, dp, 0, rows, cols, 0, n)
        b.download_device(msgs, 0, 8)  # writes the rows
        s = b.get_stats()
        assert s["calls"]["pcs_rows"] == 1
        if policy == 0:
            assert s["kernel_ns"]["pcs_rows"] > 0
        for x in (dw, dp, msgs):
            b.free_device(x)
