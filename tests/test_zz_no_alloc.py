"""The allocation-free combination entry point
(volta_mi355x_pcs_combine_rows_device_noalloc) against the allocating one
(volta_cuda_pcs_combine_rows_device) and the oracle, through the C ABI.

Two calls in a row, the second smaller, so the second runs over scratch the
first left behind; neither call may allocate (RawStats allocation_calls and
live_device_bytes unchanged); a plan whose partials outgrow the fixed scratch
at the default row chunks runs with larger ones; a plan beyond it even at the
largest chunks is refused."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

P = 0xFFFF_FFFF_0000_0001


def rand_i16(seed, size):
    return np.random.Generator(np.random.PCG64(seed)).integers(-(1 << 15), 1 << 15, size=size, dtype=np.int16)


def rand_fp(seed, shape):
    return np.random.Generator(np.random.PCG64(seed)).integers(0, P, size=shape, dtype=np.uint64)


def call(b, name, w, dp, dc, rows, cols, pad, comb, out):
    fn = getattr(b.lib, name)
    return fn(b.raw, w.id, 0, dp.id, 0, dc.id, 0, rows, cols, pad, comb, out.id, 0)


@pytest.mark.parametrize("shapes", [[(4096, 2048, 512, 2), (300, 100, 7, 3)],
                                    [(1 << 16, 2048, 0, 2), (5, 3, 1, 1)],
                                    [(1 << 17, 2048, 0, 2), (4096, 2048, 512, 2)]])
def test_noalloc_combination_matches_allocating_entry_point(oracle, shapes):
    from volta_mi355x import FP2, Backend
    with Backend() as b:
        for k, (rows, cols, pad, comb) in enumerate(shapes):
            w = rand_i16(rows + k, rows * cols)
            pads = rand_fp(rows * 3 + k, rows * pad) if pad else np.zeros(1, np.uint64)
            co = rand_fp(comb + k, (comb * rows, 2))
            dw, dp = b.upload_device(w), b.upload_device(pads)
            dc = b.upload_device(co, FP2)
            ref_out = b.alloc_device(comb * (cols + pad), FP2)
            out = b.alloc_device(comb * (cols + pad), FP2)
            assert call(b, "volta_cuda_pcs_combine_rows_device", dw, dp, dc, rows, cols, pad, comb, ref_out) == 0
            b.synchronize()
            before = b.get_stats()
            assert call(b, "volta_mi355x_pcs_combine_rows_device_noalloc", dw, dp, dc, rows, cols, pad, comb,
                        out) == 0, b.last_error()
            b.synchronize()
            after = b.get_stats()
            assert after["allocation_calls"] == before["allocation_calls"]
            assert after["live_device_bytes"] == before["live_device_bytes"]
            assert after["calls"]["pcs_rows"] == before["calls"]["pcs_rows"] + 1
            got = b.download_device(out).view(np.uint64).reshape(comb, cols + pad, 2)
            want = b.download_device(ref_out).view(np.uint64).reshape(comb, cols + pad, 2)
            for x in (dw, dp, dc, ref_out, out):
                b.free_device(x)
            assert (got == want).all(), (rows, cols, pad, comb)
            if rows * cols <= 4096 * 2048:
                assert (got == oracle.pcs_combine_rows(w, pads if pad else None, co, rows, cols, pad, comb)).all()


def test_noalloc_combination_refuses_plans_beyond_its_scratch():
    """2^17 rows of 2048 columns in two partial chunks of 2^16 rows (the
    largest the sums stay exact in): 257 combinations need 2 x 257 x 2048
    Fp2 partials, just over the fixed 16 MiB array; the call fails with an
    error and writes nothing.  (At 512-row chunks, 2^17 rows and two
    combinations also outgrow the array; that plan runs with larger chunks,
    checked above.)"""
    from volta_mi355x import FP2, Backend
    rows, cols, comb = 1 << 17, 2048, 257
    with Backend() as b:
        dw = b.alloc_device(rows * cols, np.int16)
        dp = b.alloc_device(1, np.uint64)
        dc = b.alloc_device(comb * rows, FP2)
        out = b.alloc_device(comb * cols, FP2)
        b.zero_device(out, 0, comb * cols)
        assert call(b, "volta_mi355x_pcs_combine_rows_device_noalloc", dw, dp, dc, rows, cols, 0, comb, out) != 0
        assert "scratch" in b.last_error() and "16777216" in b.last_error()
        assert not b.download_device(out).view(np.uint64).any()
        for x in (dw, dp, dc, out):
            b.free_device(x)


def test_noalloc_combination_two_contexts_back_to_back(oracle):
    """Two contexts on one GPU share the fixed array: calls from both, issued
    back to back with no host synchronisation between them, must each give
    the oracle's combination (the library orders their uses on the device)."""
    from volta_mi355x import FP2, Backend
    shapes = [(4096, 2048, 512, 2), (4096, 2048, 0, 2), (2048, 1000, 3, 3)]
    with Backend() as a, Backend() as b:
        jobs = []
        for k, (rows, cols, pad, comb) in enumerate(shapes * 2):
            ctx = a if k % 2 == 0 else b
            w = rand_i16(700 + k, rows * cols)
            pads = rand_fp(710 + k, rows * pad) if pad else np.zeros(1, np.uint64)
            co = rand_fp(720 + k, (comb * rows, 2))
            dw, dp, dc = ctx.upload_device(w), ctx.upload_device(pads), ctx.upload_device(co, FP2)
            out = ctx.alloc_device(comb * (cols + pad), FP2)
            jobs.append((ctx, w, pads, co, (rows, cols, pad, comb), (dw, dp, dc, out)))
        a.synchronize()
        b.synchronize()
        for ctx, _, _, _, (rows, cols, pad, comb), (dw, dp, dc, out) in jobs:
            assert call(ctx, "volta_mi355x_pcs_combine_rows_device_noalloc", dw, dp, dc, rows, cols, pad, comb,
                        out) == 0, ctx.last_error()
        for ctx, w, pads, co, (rows, cols, pad, comb), bufs in jobs:
            got = ctx.download_device(bufs[3]).view(np.uint64).reshape(comb, cols + pad, 2)
            for x in bufs:
                ctx.free_device(x)
            assert (got == oracle.pcs_combine_rows(w, pads if pad else None, co, rows, cols, pad, comb)).all(), \
                (rows, cols, pad, comb)


def test_noalloc_combination_refused_during_stream_capture():
    """While the context stream is being captured the entry point refuses
    with an error and enqueues nothing (the capture ends with an empty graph)."""
    import ctypes
    from volta_mi355x import FP2, Backend
    hip = ctypes.CDLL("libamdhip64.so", mode=ctypes.RTLD_GLOBAL)
    hip.hipStreamBeginCapture.argtypes = [ctypes.c_void_p, ctypes.c_int]
    hip.hipStreamEndCapture.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]
    hip.hipGraphDestroy.argtypes = [ctypes.c_void_p]
    rows, cols, comb = 64, 256, 1
    with Backend() as b:
        dw = b.upload_device(rand_i16(5, rows * cols))
        dp = b.alloc_device(1, np.uint64)
        dc = b.upload_device(rand_fp(6, (comb * rows, 2)), FP2)
        out = b.alloc_device(comb * cols, FP2)
        b.synchronize()
        s = ctypes.c_void_p(b.stream())
        assert hip.hipStreamBeginCapture(s, 2) == 0  # hipStreamCaptureModeRelaxed
        rc = call(b, "volta_mi355x_pcs_combine_rows_device_noalloc", dw, dp, dc, rows, cols, 0, comb, out)
        err = b.last_error()
        graph = ctypes.c_void_p()
        assert hip.hipStreamEndCapture(s, ctypes.byref(graph)) == 0
        if graph.value:
            hip.hipGraphDestroy(graph)
        assert rc != 0 and "stream capture" in err
        # the context works as before once the capture has ended
        assert call(b, "volta_mi355x_pcs_combine_rows_device_noalloc", dw, dp, dc, rows, cols, 0, comb, out) == 0
        b.synchronize()
        for x in (dw, dp, dc, out):
            b.free_device(x)
