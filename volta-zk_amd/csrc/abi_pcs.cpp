// abi_pcs.cpp -- the PCS entry points of the volta_cuda_* C ABI (ABI 37) plus
// the MI355X extensions (volta_mi355x_*).
//
// Each reference entry point keeps its signature, unit conventions (element
// offsets for compute calls, byte offsets for raw storage), geometry checks,
// error strings and RawStats side effects; the reference implementation
// each replaces is cited at the function.  Compute runs on the context's
// single HIP stream; only entry points that return host data synchronise.
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstring>
#include <vector>

#include "context.hpp"
#include "gl64.hpp"
#include "kernels.hpp"

using namespace vmx;
using gl::Fp2;

namespace {

bool pow2(size_t n) { return n >= 2 && (n & (n - 1)) == 0; }

// Base-field transforms: p - 1 = 2^32 (2^32 - 1) bounds the root order at
// 2^32, and a 2^32-point twiddle table alone would be 16 GiB; sizes above
// 2^31 are refused as invalid geometry before any table is built.
constexpr size_t MAX_BASE_NTT = size_t{1} << 31;
bool base_ntt_size(size_t n) { return pow2(n) && n <= MAX_BASE_NTT; }

template <class F>
int guarded(Context* c, const char* what, F&& f) noexcept {
    try {
        return f();
    } catch (const std::exception&) {
        std::string m = std::string(what) + " threw a C++ exception";
        return fail_msg(c, m.c_str());
    } catch (...) {
        std::string m = std::string(what) + " threw an unknown exception";
        return fail_msg(c, m.c_str());
    }
}

// Resident forward NTT with the per-size twiddle upload accounted as H2D.
int resident_ntt(Context* c, const uint64_t* in, size_t in_stride, size_t msg_len, size_t rows, size_t n,
                 uint64_t* out, bool inverse) {
    uint64_t h2d = 0;
    TwiddleSet* t = nullptr;
    if (ensure_twiddles(c, n, &h2d, &t)) return -1;
    // the pass engine (t->reg) computes the inverse from the forward tables
    if (inverse && !t->reg && ensure_inverse_twiddles(c, n, &h2d, &t)) return -1;
    if (begin_op(c) || mark_op(c, 1)) return -1;
    if (ntt_fp_rows(c, in, in_stride, msg_len, rows, n, out, t, inverse)) return -1;
    if (mark_op(c, 2)) return -1;
    return finish_op(c, OP_PCS_NTT, h2d, 0);
}

}  // namespace

// ---------------------------------------------------------------------------
// Resident NTTs
// ---------------------------------------------------------------------------

// The fused encode of deferred message rows: codewords NTT(lift(w) || pads || 0)
// read from the i16 weights and the pads, the same result as the transform of
// the written rows.  `pm` stays pending: its rows are still unwritten.
static int encode_pending(Context* c, const PendingMessages& pm, uint64_t* out) {
    uint64_t h2d = 0;
    TwiddleSet* t = nullptr;
    if (ensure_twiddles(c, pm.code_len, &h2d, &t)) return -1;
    if (begin_op(c) || mark_op(c, 1)) return -1;
    int rc = 1;
    if (pm.pad == 0) rc = encode_i16_fast(c, pm.w, pm.rows, pm.cols, pm.code_len, out, t);
    if (rc < 0) return -1;
    if (rc == 1 && ntt_msg_i16_rows(c, pm.w, pm.pads, pm.rows, pm.cols, pm.pad, pm.code_len, out, t)) return -1;
    if (mark_op(c, 2)) return -1;
    return finish_op(c, OP_PCS_NTT, h2d, 0);
}

// Replaces volta_cuda_ntt_fp_batch_device (cuda/volta_cuda_backend.cu:6545-6561):
// out-of-place batched forward NTT of pre-padded rows; input is preserved.
// When the input is exactly the region of deferred message rows (the
// reference's commit chain), the codewords are encoded from their sources in
// one pass; the rows stay deferred.
VMX_API int volta_cuda_ntt_fp_batch_device(void* raw, uint64_t in_id, size_t in_off, size_t rows, size_t n,
                                              uint64_t out_id, size_t out_off) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !rows || !base_ntt_size(n)) return fail_msg(c, "invalid resident Fp NTT geometry");
    return guarded(c, "resident Fp NTT", [&] {
        size_t total = 0;
        if (!mul_ok(rows, n, &total)) return fail_msg(c, "resident Fp NTT geometry overflows size_t");
        const PendingMessages& pm = c->pending;
        if (c->has_pending && pm.out_id == in_id && pm.out_off == in_off && pm.rows == rows && pm.code_len == n &&
            out_id != pm.w_id && (!pm.pad || out_id != pm.pads_id)) {
            c->bypass_settle = true;
            void *in = nullptr, *out = nullptr;
            const int rc = region_elems(c, in_id, in_off, total, 8, &in) ||
                           region_elems(c, out_id, out_off, total, 8, &out);
            c->bypass_settle = false;
            if (rc) return -1;
            if (in_id == out_id && in_off < out_off + total && out_off < in_off + total)
                return fail_msg(c, "resident Fp NTT input and output overlap");
            return encode_pending(c, pm, static_cast<uint64_t*>(out));
        }
        void *in = nullptr, *out = nullptr;
        if (region_elems(c, in_id, in_off, total, 8, &in, true)) return -1;
        // Rows the library wrote as messages (and nothing has touched since
        // but reads) are zero from cols + pad on: the transform reads only
        // that prefix of each row.
        size_t len = n;
        if (const Resident* rr = find_resident(c, in_id); rr && rr->msg_rows && rr->msg_off == in_off &&
                                                          rr->msg_count == rows && rr->msg_row_len == n)
            len = rr->msg_nonzero;
        if (region_elems(c, out_id, out_off, total, 8, &out)) return -1;
        if (in_id == out_id && in_off < out_off + total && out_off < in_off + total)
            return fail_msg(c, "resident Fp NTT input and output overlap");
        return resident_ntt(c, static_cast<const uint64_t*>(in), n, len, rows, n, static_cast<uint64_t*>(out),
                            false);
    });
}

// Replaces volta_cuda_ntt_fp2_batch_device (.cu:6563-6579): componentwise Fp2
// NTT with base-field twiddles.
VMX_API int volta_cuda_ntt_fp2_batch_device(void* raw, uint64_t in_id, size_t in_off, size_t rows, size_t n,
                                               uint64_t out_id, size_t out_off) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !rows || !base_ntt_size(n)) return fail_msg(c, "invalid resident Fp2 NTT geometry");
    return guarded(c, "resident Fp2 NTT", [&] {
        size_t total = 0;
        if (!mul_ok(rows, n, &total)) return fail_msg(c, "resident Fp2 NTT geometry overflows size_t");
        void *in = nullptr, *out = nullptr;
        if (region_elems(c, in_id, in_off, total, 16, &in, true) || region_elems(c, out_id, out_off, total, 16, &out))
            return -1;
        if (in_id == out_id && in_off < out_off + total && out_off < in_off + total)
            return fail_msg(c, "resident Fp2 NTT input and output overlap");
        uint64_t h2d = 0;
        TwiddleSet* t = nullptr;
        if (ensure_twiddles(c, n, &h2d, &t)) return -1;
        if (begin_op(c) || mark_op(c, 1)) return -1;
        if (ntt_fp2_rows(c, static_cast<const uint64_t*>(in), rows, n, static_cast<uint64_t*>(out), t))
            return -1;
        if (mark_op(c, 2)) return -1;
        return finish_op(c, OP_PCS_NTT, h2d, 0);
    });
}

// ---------------------------------------------------------------------------
// Host-pointer NTTs (staged through workspaces; synchronous)
// ---------------------------------------------------------------------------

namespace {
int host_ntt(Context* c, const uint64_t* msgs, size_t rows, size_t msg_len, size_t n, uint64_t* out) {
    size_t total = 0, bytes = 0, in_bytes = 0;
    if (!mul_ok(rows, n, &total) || !mul_ok(total, 8, &bytes) || !mul3_ok(rows, msg_len, 8, &in_bytes))
        return fail_msg(c, "Fp NTT geometry overflows size_t");
    if (ensure_ws(c, WS_IN, std::max<size_t>(in_bytes, 8)) || ensure_ws(c, WS_OUT, bytes)) return -1;
    uint64_t h2d = 0;
    TwiddleSet* t = nullptr;
    if (ensure_twiddles(c, n, &h2d, &t)) return -1;
    if (begin_op_h2d(c)) return -1;
    // Compact rows cross PCIe once; zero padding happens in the kernel load.
    if (in_bytes && staged_copy(c, ws<uint64_t>(c, WS_IN), msgs, in_bytes, hipMemcpyHostToDevice)) return -1;
    h2d += in_bytes;
    if (mark_op(c, 1)) return -1;
    if (ntt_fp_rows(c, ws<uint64_t>(c, WS_IN), msg_len, msg_len, rows, n, ws<uint64_t>(c, WS_OUT), t, false))
        return -1;
    if (mark_op(c, 2)) return -1;
    if (staged_copy(c, out, ws<uint64_t>(c, WS_OUT), bytes, hipMemcpyDeviceToHost)) return -1;
    return finish_op(c, OP_PCS_NTT, h2d, bytes);
}
}  // namespace

// Replaces volta_cuda_ntt_fp (.cu:5534-5544).
VMX_API int volta_cuda_ntt_fp(void* raw, const uint64_t* msg, size_t msg_len, size_t n, uint64_t* out) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !msg || !out || !base_ntt_size(n) || msg_len > n) return fail_msg(c, "invalid Fp NTT geometry");
    return guarded(c, "Fp NTT", [&] { return host_ntt(c, msg, 1, msg_len, n, out); });
}

// Replaces volta_cuda_ntt_fp_batch (.cu:5546-5559): compact rows of msg_len.
VMX_API int volta_cuda_ntt_fp_batch(void* raw, const uint64_t* msgs, size_t rows, size_t msg_len, size_t n,
                                       uint64_t* out) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !msgs || !out || !rows || !base_ntt_size(n) || msg_len > n) return fail_msg(c, "invalid Fp NTT batch geometry");
    return guarded(c, "Fp NTT batch", [&] { return host_ntt(c, msgs, rows, msg_len, n, out); });
}

// Replaces volta_cuda_ntt_fp2 (.cu:5561-5571).
VMX_API int volta_cuda_ntt_fp2(void* raw, const Fp2* msg, size_t msg_len, size_t n, Fp2* out) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !msg || !out || !base_ntt_size(n) || msg_len > n) return fail_msg(c, "invalid Fp2 NTT geometry");
    return guarded(c, "Fp2 NTT", [&] {
        const size_t bytes = n * sizeof(Fp2), in_bytes = msg_len * sizeof(Fp2);
        if (ensure_ws(c, WS_IN, bytes) || ensure_ws(c, WS_OUT, bytes)) return -1;
        uint64_t h2d = 0;
        TwiddleSet* t = nullptr;
        if (ensure_twiddles(c, n, &h2d, &t)) return -1;
        if (begin_op_h2d(c)) return -1;
        if (in_bytes && staged_copy(c, ws<Fp2>(c, WS_IN), msg, in_bytes, hipMemcpyHostToDevice)) return -1;
        if (bytes > in_bytes && zero_bytes(c, ws<unsigned char>(c, WS_IN) + in_bytes, bytes - in_bytes)) return -1;
        h2d += bytes;
        if (mark_op(c, 1)) return -1;
        if (ntt_fp2_rows(c, ws<uint64_t>(c, WS_IN), 1, n, ws<uint64_t>(c, WS_OUT), t)) return -1;
        if (mark_op(c, 2)) return -1;
        if (staged_copy(c, out, ws<Fp2>(c, WS_OUT), bytes, hipMemcpyDeviceToHost)) return -1;
        return finish_op(c, OP_PCS_NTT, h2d, bytes);
    });
}

// ---------------------------------------------------------------------------
// PCS rows
// ---------------------------------------------------------------------------

// Replaces volta_cuda_pcs_messages_device (.cu:7064-7079): msg = lift(w) || pads || 0.
VMX_API int volta_cuda_pcs_messages_device(void* raw, uint64_t w_id, size_t w_off, uint64_t pads_id,
                                              size_t pads_off, size_t rows, size_t cols, size_t pad, size_t code_len,
                                              uint64_t out_id, size_t out_off) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !rows || !cols || !code_len || cols + pad > code_len || cols + pad < cols)
        return fail_msg(c, "invalid resident PCS message geometry");
    return guarded(c, "resident PCS messages", [&] {
        size_t wn = 0, pn = 0, on = 0;
        if (!mul_ok(rows, cols, &wn) || !mul_ok(rows, pad, &pn) || !mul_ok(rows, code_len, &on))
            return fail_msg(c, "resident PCS message geometry overflows size_t");
        void *w = nullptr, *pads = nullptr, *out = nullptr;
        if (region_elems(c, w_id, w_off, wn, 2, &w, true) ||
            (pad && region_elems(c, pads_id, pads_off, pn, 8, &pads, true)))
            return -1;
        // Deferred rows of exactly this region are replaced by this call's.
        if (c->has_pending && c->pending.out_id == out_id && c->pending.out_off == out_off &&
            c->pending.rows * c->pending.code_len == on)
            c->has_pending = false;
        if (region_elems(c, out_id, out_off, on, 8, &out)) return -1;
        // The rows are recorded, not written, when their buffer is separate
        // from the sources: a following forward NTT of exactly these rows
        // (finish_resident_commit, rust/volta-pcs/src/ligero.rs:477-496) then
        // encodes straight from the weights and pads, and any other access
        // writes them first (settle_pending).  They are written at once when
        // the caller holds the device address of the rows' buffer or of a
        // source (volta_mi355x_resident_device_ptr), since its own kernels
        // could read the rows or change a source behind the library.  The
        // stats are those of a messages call either way; a call that only
        // records its rows runs nothing on the device and so has no timing
        // record of its own (its kernel time is the later write's, or the
        // fused encode's).
        const bool exposed = find_resident(c, out_id)->exposed || find_resident(c, w_id)->exposed ||
                             (pad && find_resident(c, pads_id)->exposed);
        const bool defer = !exposed && out_id != w_id && (!pad || out_id != pads_id);
        const PendingMessages rec{out_id, out_off, static_cast<uint64_t*>(out), w_id, pad ? pads_id : 0,
                                  static_cast<const int16_t*>(w), static_cast<const uint64_t*>(pads),
                                  rows, cols, pad, code_len};
        if (defer && !c->has_pending) {
            c->pending = rec;
            c->has_pending = true;
            return empty_op(c, OP_PCS_ROWS);
        }
        if (begin_op(c) || mark_op(c, 1)) return -1;
        if (defer) {
            if (settle_pending(c)) return -1;  // one record at a time
            c->pending = rec;
            c->has_pending = true;
        } else {
            if (pcs_messages(c, static_cast<const int16_t*>(w), static_cast<const uint64_t*>(pads), rows, cols, pad,
                             code_len, static_cast<uint64_t*>(out)))
                return -1;
            if (out_id != w_id && (!pad || out_id != pads_id))
                note_message_rows(c, out_id, out_off, rows, code_len, cols + pad);
        }
        if (mark_op(c, 2)) return -1;
        return finish_op(c, OP_PCS_ROWS, 0, 0);
    });
}

namespace {
int combine_device(Context* c, uint64_t w_id, size_t w_off, uint64_t pads_id, size_t pads_off, uint64_t co_id,
                   size_t co_off, size_t rows, size_t cols, size_t pad, size_t combinations, uint64_t out_id,
                   size_t out_off, bool noalloc = false) {
    size_t wn = 0, pn = 0, cn = 0, msg_len = 0, on = 0;
    if (!mul_ok(rows, cols, &wn) || !mul_ok(rows, pad, &pn) || !mul_ok(combinations, rows, &cn) ||
        !add_ok(cols, pad, &msg_len) || !mul_ok(combinations, msg_len, &on))
        return fail_msg(c, "resident PCS combination geometry overflows size_t");
    void *w = nullptr, *pads = nullptr, *co = nullptr, *out = nullptr;
    if (region_elems(c, w_id, w_off, wn, 2, &w, true) || (pad && region_elems(c, pads_id, pads_off, pn, 8, &pads, true)) ||
        region_elems(c, co_id, co_off, cn, 16, &co, true) || region_elems(c, out_id, out_off, on, 16, &out))
        return -1;
    if (begin_op(c) || mark_op(c, 1)) return -1;
    const auto combine = noalloc ? pcs_combine_rows_noalloc : pcs_combine_rows;
    if (combine(c, static_cast<const int16_t*>(w), static_cast<const uint64_t*>(pads), static_cast<const Fp2*>(co),
                rows, cols, pad, combinations, static_cast<Fp2*>(out)))
        return -1;
    if (mark_op(c, 2)) return -1;
    return finish_op(c, OP_PCS_ROWS, 0, 0);
}
}  // namespace

// Replaces volta_cuda_pcs_combine_rows_device (.cu:7081-7099).
VMX_API int volta_cuda_pcs_combine_rows_device(void* raw, uint64_t w_id, size_t w_off, uint64_t pads_id,
                                                  size_t pads_off, uint64_t co_id, size_t co_off, size_t rows,
                                                  size_t cols, size_t pad, size_t combinations, uint64_t out_id,
                                                  size_t out_off) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !rows || !cols || !combinations) return fail_msg(c, "invalid resident PCS combination geometry");
    return guarded(c, "resident PCS combination", [&] {
        return combine_device(c, w_id, w_off, pads_id, pads_off, co_id, co_off, rows, cols, pad, combinations,
                              out_id, out_off);
    });
}

// volta_cuda_pcs_combine_rows_device without allocation, for callers that
// cannot allocate (serving loops, harnesses that forbid hipMalloc): the
// partials and coefficient sums live in a fixed 16 MiB device array per GPU
// instead of the context's grow-only workspaces, and a plan that needs more is
// refused with an error.  All contexts on one GPU share that array; their uses
// are ordered on the device by a per-device event (each use waits for the
// previous one), and each call rewrites every scratch word it reads.  It is
// refused while the context stream is being captured into a graph: its timing
// may synchronise the stream and its ordering event comes from outside the
// capture.  Same arguments, results and stats.
VMX_API int volta_mi355x_pcs_combine_rows_device_noalloc(void* raw, uint64_t w_id, size_t w_off, uint64_t pads_id,
                                                          size_t pads_off, uint64_t co_id, size_t co_off, size_t rows,
                                                          size_t cols, size_t pad, size_t combinations,
                                                          uint64_t out_id, size_t out_off) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !rows || !cols || !combinations) return fail_msg(c, "invalid resident PCS combination geometry");
    return guarded(c, "allocation-free resident PCS combination", [&] {
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        VMX_HIP(c, hipStreamIsCapturing(c->stream, &cap));
        if (cap != hipStreamCaptureStatusNone)
            return fail_msg(c, "allocation-free PCS combination is refused during stream capture");
        return combine_device(c, w_id, w_off, pads_id, pads_off, co_id, co_off, rows, cols, pad, combinations,
                              out_id, out_off, true);
    });
}

// Replaces volta_cuda_pcs_combine_rows (.cu:7228-7241): host buffers in/out.
VMX_API int volta_cuda_pcs_combine_rows(void* raw, const int16_t* weights, const uint64_t* pads, const Fp2* coeffs,
                                           size_t rows, size_t cols, size_t pad, size_t combinations, Fp2* out) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !weights || !coeffs || !out || !rows || !cols || !combinations || (pad && !pads))
        return fail_msg(c, "invalid PCS row-combination geometry");
    return guarded(c, "PCS row combination", [&] {
        size_t wb = 0, pb = 0, cb = 0, ob = 0;
        if (!mul3_ok(rows, cols, 2, &wb) || !mul3_ok(rows, pad, 8, &pb) || !mul3_ok(combinations, rows, 16, &cb) ||
            cols + pad < cols || !mul3_ok(combinations, cols + pad, 16, &ob))
            return fail_msg(c, "PCS row-combination geometry overflows size_t");
        if (ensure_ws(c, WS_IN, wb) || ensure_ws(c, WS_AUX0, std::max<size_t>(pb, 8)) || ensure_ws(c, WS_AUX1, cb) ||
            ensure_ws(c, WS_OUT, ob))
            return -1;
        if (begin_op_h2d(c)) return -1;
        if (staged_copy(c, ws<void>(c, WS_IN), weights, wb, hipMemcpyHostToDevice) ||
            (pb && staged_copy(c, ws<void>(c, WS_AUX0), pads, pb, hipMemcpyHostToDevice)) ||
            staged_copy(c, ws<void>(c, WS_AUX1), coeffs, cb, hipMemcpyHostToDevice))
            return -1;
        if (mark_op(c, 1)) return -1;
        if (pcs_combine_rows(c, ws<int16_t>(c, WS_IN), ws<uint64_t>(c, WS_AUX0), ws<Fp2>(c, WS_AUX1), rows, cols, pad,
                             combinations, ws<Fp2>(c, WS_OUT)))
            return -1;
        if (mark_op(c, 2)) return -1;
        if (staged_copy(c, out, ws<void>(c, WS_OUT), ob, hipMemcpyDeviceToHost)) return -1;
        return finish_op(c, OP_PCS_ROWS, wb + pb + cb, ob);
    });
}

// Replaces volta_cuda_fp2_powers_device (.cu:4107-4126): [c^1 .. c^count].
VMX_API int volta_cuda_fp2_powers_device(void* raw, uint64_t c0, uint64_t c1, uint64_t out_id, size_t out_off,
                                            size_t count) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !count || c0 >= gl::P || c1 >= gl::P) return fail_msg(c, "invalid Fp2 powers input");
    return guarded(c, "Fp2 powers", [&] {
        void* out = nullptr;
        if (region_elems(c, out_id, out_off, count, 16, &out)) return -1;
        if (begin_op(c) || mark_op(c, 1)) return -1;
        if (fp2_powers(c, Fp2{c0, c1}, static_cast<Fp2*>(out), count)) return -1;
        if (mark_op(c, 2)) return -1;
        return finish_op(c, OP_PCS_ROWS, 0, 0, 0, 0, count * sizeof(Fp2));
    });
}

// Replaces volta_cuda_fp2_add_inplace_device (.cu:7101-7112).
VMX_API int volta_cuda_fp2_add_inplace_device(void* raw, uint64_t t_id, size_t t_off, uint64_t a_id, size_t a_off,
                                                 size_t n) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !n) return fail_msg(c, "invalid resident Fp2 add");
    return guarded(c, "resident Fp2 add", [&] {
        void *t = nullptr, *a = nullptr;
        if (region_elems(c, t_id, t_off, n, 16, &t) || region_elems(c, a_id, a_off, n, 16, &a, true)) return -1;
        if (begin_op(c) || mark_op(c, 1)) return -1;
        if (fp2_add_inplace(c, static_cast<Fp2*>(t), static_cast<const Fp2*>(a), n)) return -1;
        if (mark_op(c, 2)) return -1;
        return finish_op(c, OP_PCS_ROWS, 0, 0);
    });
}

// Replaces volta_cuda_pcs_gather_columns_device (.cu:7243-7254).
VMX_API int volta_cuda_pcs_gather_columns_device(void* raw, uint64_t m_id, size_t m_off, size_t rows, size_t cols,
                                                    uint64_t idx_id, size_t idx_off, size_t queries, uint64_t out_id,
                                                    size_t out_off, int fp2) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !rows || !cols || !queries) return fail_msg(c, "invalid resident PCS gather geometry");
    return guarded(c, "resident PCS gather", [&] {
        const size_t elem = fp2 ? 16 : 8;
        size_t mn = 0, on = 0;
        if (!mul_ok(rows, cols, &mn) || !mul_ok(rows, queries, &on))
            return fail_msg(c, "resident PCS gather geometry overflows size_t");
        void *m = nullptr, *idx = nullptr, *out = nullptr;
        if (region_elems(c, m_id, m_off, mn, elem, &m, true) || region_elems(c, idx_id, idx_off, queries, 4, &idx, true) ||
            region_elems(c, out_id, out_off, on, elem, &out))
            return -1;
        // Indices live on the device and are validated by the Rust seam before
        // upload (rust/volta-accel/src/lib.rs:6773-6827); the kernel reads an
        // out-of-range index as a zero column rather than faulting.
        if (begin_op(c) || mark_op(c, 1)) return -1;
        if (gather_columns(c, static_cast<const uint64_t*>(m), static_cast<const uint32_t*>(idx),
                           static_cast<uint64_t*>(out), rows, cols, queries, fp2 != 0))
            return -1;
        if (mark_op(c, 2)) return -1;
        return finish_op(c, OP_PCS_ROWS, 0, 0);
    });
}

// Replaces volta_cuda_pcs_gather_columns (.cu:7243-7254 host form).
VMX_API int volta_cuda_pcs_gather_columns(void* raw, const uint64_t* matrix, size_t rows, size_t cols,
                                             const uint32_t* idx, size_t queries, uint64_t* out) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !matrix || !idx || !out || !rows || !cols || !queries)
        return fail_msg(c, "invalid PCS column-gather geometry");
    for (size_t q = 0; q < queries; ++q)
        if (idx[q] >= cols) return fail_msg(c, "PCS column-gather index out of range");
    return guarded(c, "PCS column gather", [&] {
        size_t mb = 0, ob = 0;
        if (!mul3_ok(rows, cols, 8, &mb) || !mul3_ok(rows, queries, 8, &ob))
            return fail_msg(c, "PCS column-gather geometry overflows size_t");
        const size_t ib = queries * 4;
        if (ensure_ws(c, WS_IN, mb) || ensure_ws(c, WS_AUX0, ib) || ensure_ws(c, WS_OUT, ob)) return -1;
        if (begin_op_h2d(c)) return -1;
        if (staged_copy(c, ws<void>(c, WS_IN), matrix, mb, hipMemcpyHostToDevice) ||
            staged_copy(c, ws<void>(c, WS_AUX0), idx, ib, hipMemcpyHostToDevice))
            return -1;
        if (mark_op(c, 1)) return -1;
        if (gather_columns(c, ws<uint64_t>(c, WS_IN), ws<uint32_t>(c, WS_AUX0), ws<uint64_t>(c, WS_OUT), rows, cols,
                           queries, false))
            return -1;
        if (mark_op(c, 2)) return -1;
        if (staged_copy(c, out, ws<void>(c, WS_OUT), ob, hipMemcpyDeviceToHost)) return -1;
        return finish_op(c, OP_PCS_ROWS, mb + ib, ob);
    });
}

// ---------------------------------------------------------------------------
// ChaCha8 FpStream rows
// ---------------------------------------------------------------------------

namespace {
constexpr uint64_t RESERVED_MOCK_BITS = (uint64_t{1} << 63) | (uint64_t{1} << 62) | (uint64_t{1} << 61);

int fp_rows_impl(Context* c, uint64_t out_id, size_t out_off_bytes, const uint8_t* seed, uint64_t base, size_t rows,
                 size_t count, int op) {
    if (!c || !seed || !rows || !count) return fail_msg(c, "invalid ChaCha8 Fp row generation: rows and count must be non-zero");
    if (rows - 1 > UINT64_MAX - base) return fail_msg(c, "ChaCha8 Fp row domain overflows u64");
    const uint64_t last = base + static_cast<uint64_t>(rows - 1);
    if (op == OP_AUTH_MASKS && ((base | last) & RESERVED_MOCK_BITS))
        return fail_msg(c, "mock correlation mask domain sets reserved correlation bits");
    size_t elems = 0, bytes = 0;
    if (!mul_ok(rows, count, &elems) || !mul_ok(elems, 8, &bytes))
        return fail_msg(c, "ChaCha8 Fp row geometry overflows size_t");
    void* out = nullptr;
    if (region(c, out_id, out_off_bytes, bytes, &out)) return -1;
    if (begin_op(c) || mark_op(c, 1)) return -1;
    if (chacha8_fp_rows(c, seed, base, rows, count, static_cast<uint64_t*>(out))) return -1;
    if (mark_op(c, 2)) return -1;
    return finish_op(c, op, 0, 0, 0, 0, bytes);
}
}  // namespace

// Replaces volta_cuda_chacha8_prover_secret_fp_rows_device (.cu:3991-4047):
// row r = FpStream::domain_separated(seed, base + r), `count` draws each.
VMX_API int volta_cuda_chacha8_prover_secret_fp_rows_device(void* raw, uint64_t out_id, size_t out_off_bytes,
                                                               const uint8_t* seed, uint64_t base, size_t rows,
                                                               size_t count) {
    Context* c = static_cast<Context*>(raw);
    return guarded(c, "ChaCha8 Fp rows", [&] { return fp_rows_impl(c, out_id, out_off_bytes, seed, base, rows, count, OP_PCS_ROWS); });
}

// Replaces volta_cuda_mock_correlation_sub_masks_device (.cu:4049-4058).
VMX_API int volta_cuda_mock_correlation_sub_masks_device(void* raw, uint64_t out_id, size_t out_off_bytes,
                                                            const uint8_t* seed, uint64_t base, size_t rows,
                                                            size_t cols) {
    Context* c = static_cast<Context*>(raw);
    return guarded(c, "mock correlation masks", [&] { return fp_rows_impl(c, out_id, out_off_bytes, seed, base, rows, cols, OP_AUTH_MASKS); });
}

// Replaces volta_cuda_chacha8_prover_secret_fp2_rows_padded_device (.cu:4060-4098).
VMX_API int volta_cuda_chacha8_prover_secret_fp2_rows_padded_device(void* raw, uint64_t out_id,
                                                                       size_t out_off_bytes, const uint8_t* seed,
                                                                       uint64_t base, size_t rows, size_t count,
                                                                       size_t padded) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !seed || !rows || !count || count > padded)
        return fail_msg(c, "invalid prover-secret padded Fp2 row generation");
    return guarded(c, "ChaCha8 Fp2 rows", [&] {
        if (rows - 1 > UINT64_MAX - base) return fail_msg(c, "prover-secret Fp2 row domain overflows u64");
        size_t out_elems = 0, out_bytes = 0, gen = 0, zero = 0;
        if (!mul_ok(rows, padded, &out_elems) || !mul_ok(out_elems, 16, &out_bytes) || !mul_ok(rows * count, 16, &gen) ||
            !mul_ok(rows * (padded - count), 16, &zero))
            return fail_msg(c, "prover-secret Fp2 row geometry overflows size_t");
        void* out = nullptr;
        if (region(c, out_id, out_off_bytes, out_bytes, &out)) return -1;
        if (begin_op(c) || mark_op(c, 1)) return -1;
        if (chacha8_fp2_rows_padded(c, seed, base, rows, count, padded, static_cast<Fp2*>(out))) return -1;
        if (mark_op(c, 2)) return -1;
        return finish_op(c, OP_PCS_ROWS, 0, 0, 0, zero, gen);
    });
}

// ---------------------------------------------------------------------------
// MI355X extensions (no counterpart in the reference ABI)
// ---------------------------------------------------------------------------

// Inverse NTT of pre-padded rows: a_i = n^-1 sum_j A_j w^-ij.  The reference
// has no inverse transform; the large-transform configuration needs one.
VMX_API int volta_mi355x_ntt_fp_inverse_batch_device(void* raw, uint64_t in_id, size_t in_off, size_t rows,
                                                        size_t n, uint64_t out_id, size_t out_off) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !rows || !base_ntt_size(n)) return fail_msg(c, "invalid resident inverse Fp NTT geometry");
    return guarded(c, "resident inverse Fp NTT", [&] {
        size_t total = 0;
        if (!mul_ok(rows, n, &total)) return fail_msg(c, "resident inverse Fp NTT geometry overflows size_t");
        void *in = nullptr, *out = nullptr;
        if (region_elems(c, in_id, in_off, total, 8, &in, true) || region_elems(c, out_id, out_off, total, 8, &out))
            return -1;
        if (in_id == out_id && in_off < out_off + total && out_off < in_off + total)
            return fail_msg(c, "resident inverse Fp NTT input and output overlap");
        return resident_ntt(c, static_cast<const uint64_t*>(in), n, n, rows, n, static_cast<uint64_t*>(out), true);
    });
}

// RS-encode of compact resident u64 rows (msg_len per row) into rows x n
// codewords, zero padding in the load: the resident form of the host
// volta_cuda_ntt_fp_batch without a padded input copy in HBM.
VMX_API int volta_mi355x_ntt_fp_encode_device(void* raw, uint64_t in_id, size_t in_off, size_t rows,
                                                 size_t msg_len, size_t n, uint64_t out_id, size_t out_off) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !rows || !base_ntt_size(n) || msg_len > n) return fail_msg(c, "invalid resident Fp encode geometry");
    return guarded(c, "resident Fp encode", [&] {
        size_t in_n = 0, out_n = 0;
        if (!mul_ok(rows, msg_len, &in_n) || !mul_ok(rows, n, &out_n))
            return fail_msg(c, "resident Fp encode geometry overflows size_t");
        void *in = nullptr, *out = nullptr;
        if (region_elems(c, in_id, in_off, std::max<size_t>(in_n, 1), 8, &in, true) ||
            region_elems(c, out_id, out_off, out_n, 8, &out))
            return -1;
        if (in_id == out_id) return fail_msg(c, "resident Fp encode input and output must be distinct buffers");
        return resident_ntt(c, static_cast<const uint64_t*>(in), msg_len, msg_len, rows, n,
                            static_cast<uint64_t*>(out), false);
    });
}

// Fused Ligero encode: codeword rows NTT(lift(w) || pads || 0) straight from
// the i16 weights, without the rows x code_len message buffer that
// volta_cuda_pcs_messages_device + volta_cuda_ntt_fp_batch_device materialise.
// Same result as that pair; stats: one PcsNtt call (+ the twiddle upload).
VMX_API int volta_mi355x_pcs_encode_device(void* raw, uint64_t w_id, size_t w_off, uint64_t pads_id,
                                              size_t pads_off, size_t rows, size_t cols, size_t pad, size_t code_len,
                                              uint64_t out_id, size_t out_off) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !rows || !cols || !base_ntt_size(code_len) || cols + pad > code_len || cols + pad < cols)
        return fail_msg(c, "invalid resident PCS encode geometry");
    return guarded(c, "resident PCS encode", [&] {
        size_t wn = 0, pn = 0, on = 0;
        if (!mul_ok(rows, cols, &wn) || !mul_ok(rows, pad, &pn) || !mul_ok(rows, code_len, &on))
            return fail_msg(c, "resident PCS encode geometry overflows size_t");
        void *w = nullptr, *pads = nullptr, *out = nullptr;
        if (region_elems(c, w_id, w_off, wn, 2, &w, true) || (pad && region_elems(c, pads_id, pads_off, pn, 8, &pads, true)) ||
            region_elems(c, out_id, out_off, on, 8, &out))
            return -1;
        uint64_t h2d = 0;
        TwiddleSet* t = nullptr;
        if (ensure_twiddles(c, code_len, &h2d, &t)) return -1;
        if (begin_op(c) || mark_op(c, 1)) return -1;
        int rc = 1;
        if (pad == 0)
            rc = encode_i16_fast(c, static_cast<const int16_t*>(w), rows, cols, code_len, static_cast<uint64_t*>(out),
                                 t);
        if (rc < 0) return -1;
        if (rc == 1 && ntt_msg_i16_rows(c, static_cast<const int16_t*>(w), static_cast<const uint64_t*>(pads), rows,
                                        cols, pad, code_len, static_cast<uint64_t*>(out), t))
            return -1;
        if (mark_op(c, 2)) return -1;
        return finish_op(c, OP_PCS_NTT, h2d, 0);
    });
}

// Row combination over dense resident u64 (Fp) rows: out[comb][j] =
// sum_i coeffs[comb*rows + i] * m[i*cols + j].  The reference ABI only combines
// i16 message rows; its own arithmetic benchmark combines u64 rows
// (cuda/p7_pcs_arithmetic.cu:275-288).
VMX_API int volta_mi355x_combine_rows_fp_device(void* raw, uint64_t m_id, size_t m_off, size_t rows, size_t cols,
                                                   uint64_t co_id, size_t co_off, size_t combinations,
                                                   uint64_t out_id, size_t out_off) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !rows || !cols || !combinations) return fail_msg(c, "invalid resident Fp combination geometry");
    return guarded(c, "resident Fp combination", [&] {
        size_t mn = 0, cn = 0, on = 0;
        if (!mul_ok(rows, cols, &mn) || !mul_ok(combinations, rows, &cn) || !mul_ok(combinations, cols, &on))
            return fail_msg(c, "resident Fp combination geometry overflows size_t");
        void *m = nullptr, *co = nullptr, *out = nullptr;
        if (region_elems(c, m_id, m_off, mn, 8, &m, true) || region_elems(c, co_id, co_off, cn, 16, &co, true) ||
            region_elems(c, out_id, out_off, on, 16, &out))
            return -1;
        if (begin_op(c) || mark_op(c, 1)) return -1;
        if (combine_rows_fp(c, static_cast<const uint64_t*>(m), rows, cols, static_cast<const Fp2*>(co), combinations,
                            static_cast<Fp2*>(out)))
            return -1;
        if (mark_op(c, 2)) return -1;
        return finish_op(c, OP_PCS_ROWS, 0, 0);
    });
}

// Raw device address of a resident region, for measurement harnesses that
// time kernels with their own events on the context stream.  Deferred message
// rows that involve the buffer are written first (region), and the buffer is
// marked exposed for the rest of its allocation: no later messages call defers
// rows that live in it or are made from it.
VMX_API int volta_mi355x_resident_device_ptr(void* raw, uint64_t id, size_t off_bytes, size_t bytes, void** out) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !out) return fail_msg(c, "invalid device-pointer query");
    if (region(c, id, off_bytes, bytes, out)) return -1;
    find_resident(c, id)->exposed = true;
    return 0;
}

// The context's HIP stream (hipStream_t), for event timing by a harness.
VMX_API int volta_mi355x_stream(void* raw, void** out) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !out) return fail_msg(c, "invalid stream query");
    *out = c->stream;
    return 0;
}

// The output checksum of the reference's arithmetic benchmarks
// (cuda/p7_pcs_arithmetic.cu:160-176): h ^= x; h *= 0x100000001B3 over u64
// words, a host loop over a host array (the words are read in order).
VMX_API uint64_t volta_mi355x_fnv64_host(const uint64_t* v, size_t n, uint64_t h) {
    if (!v) return h;
    for (size_t i = 0; i < n; ++i) {
        h ^= v[i];
        h *= 0x00000100000001B3ull;
    }
    return h;
}

// Measurement probes: streaming copy (achievable HBM bandwidth) and the
// reference's Fp2-multiply stream/chain roofline kernels.
VMX_API int volta_mi355x_probe_copy_device(void* raw, uint64_t src_id, uint64_t dst_id, size_t bytes) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !bytes || bytes % 16) return fail_msg(c, "invalid copy probe geometry (bytes must be a multiple of 16)");
    void *s = nullptr, *d = nullptr;
    if (region(c, src_id, 0, bytes, &s, true) || region(c, dst_id, 0, bytes, &d)) return -1;
    stream_touched(c);  // no timing record: outside any primitive's markers
    return probe_copy(c, s, d, bytes);
}

VMX_API int volta_mi355x_probe_expand_device(void* raw, uint64_t src_id, uint64_t dst_id, size_t src_bytes) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !src_bytes || src_bytes % 256) return fail_msg(c, "invalid expand probe geometry (a multiple of 256 bytes)");
    size_t dst_bytes = 0;
    if (!mul_ok(src_bytes, 16, &dst_bytes)) return fail_msg(c, "expand probe geometry overflows size_t");
    void *s = nullptr, *d = nullptr;
    if (region(c, src_id, 0, src_bytes, &s, true) || region(c, dst_id, 0, dst_bytes, &d)) return -1;
    stream_touched(c);  // no timing record: outside any primitive's markers
    return probe_expand(c, s, d, src_bytes);
}

VMX_API int volta_mi355x_probe_fp2_device(void* raw, uint64_t a_id, uint64_t b_id, uint64_t out_id, size_t n,
                                             int rounds) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !n || rounds < 0) return fail_msg(c, "invalid Fp2 probe geometry");
    void *a = nullptr, *b = nullptr, *o = nullptr;
    if (region_elems(c, a_id, 0, n, 16, &a, true) || region_elems(c, b_id, 0, n, 16, &b, true) ||
        region_elems(c, out_id, 0, n, 16, &o))
        return -1;
    stream_touched(c);  // no timing record: outside any primitive's markers
    if (rounds == 0)
        return probe_fp2_stream(c, static_cast<const Fp2*>(a), static_cast<const Fp2*>(b), static_cast<Fp2*>(o), n);
    return probe_fp2_chain(c, static_cast<const Fp2*>(a), static_cast<const Fp2*>(b), static_cast<Fp2*>(o), n, rounds);
}

VMX_API int volta_mi355x_synchronize(void* raw) {
    Context* c = static_cast<Context*>(raw);
    if (!c) return -1;
    return sync_stream(c, SyncReason::HostOutput);
}

// ---------------------------------------------------------------------------
// BLAKE3 column leaves, Merkle tree and paths
// ---------------------------------------------------------------------------

namespace {

bool pow2_or_one(size_t n) { return n >= 1 && (n & (n - 1)) == 0; }

// The hash kernels move 32-byte hashes with 16-byte vector accesses.
int hash_aligned(Context* c, const void* p, const char* what) {
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0) {
        std::string m = std::string(what) + " region must be 16-byte aligned";
        return fail_msg(c, m.c_str());
    }
    return 0;
}

int hash_tree_device(Context* c, uint64_t m_id, size_t m_off, size_t rows, size_t cols, uint64_t tree_id,
                     size_t tree_off_bytes, bool fp2) {
    size_t mn = 0, tb = 0;
    if (!mul_ok(rows, cols, &mn) || !mul_ok(2 * cols - 1, 32, &tb))
        return fail_msg(c, "resident Merkle geometry overflows size_t");
    void *m = nullptr, *tree = nullptr;
    if (region_elems(c, m_id, m_off, mn, fp2 ? 16 : 8, &m, true) || region_elems(c, tree_id, tree_off_bytes, tb, 1, &tree))
        return -1;
    if (hash_aligned(c, tree, "Merkle tree")) return -1;
    if (begin_op(c) || mark_op(c, 1)) return -1;
    uint32_t* t = static_cast<uint32_t*>(tree);
    if (merkle_column_leaves(c, static_cast<const uint64_t*>(m), rows, cols, fp2, t) ||
        merkle_tree_levels(c, t, cols))
        return -1;
    if (mark_op(c, 2)) return -1;
    return finish_op(c, OP_PCS_MERKLE, 0, 0);
}

}  // namespace

// Replaces volta_cuda_hash_fp_tree_device (.cu:7166-7175, hash_tree_device_impl
// .cu:7151-7164): leaves = blake3 of each column of the rows x cols Fp matrix,
// then the Merkle levels; (2 cols - 1) hashes at the tree's byte offset.
VMX_API int volta_cuda_hash_fp_tree_device(void* raw, uint64_t matrix_id, size_t matrix_off, size_t rows, size_t cols,
                                              uint64_t tree_id, size_t tree_off_bytes) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !rows || !pow2_or_one(cols)) return fail_msg(c, "invalid resident Fp Merkle geometry");
    return guarded(c, "resident Fp Merkle tree",
                   [&] { return hash_tree_device(c, matrix_id, matrix_off, rows, cols, tree_id, tree_off_bytes, false); });
}

// Replaces volta_cuda_hash_fp2_tree_device (.cu:7177-7186): the same over an
// Fp2 matrix, each element hashed as c0 then c1.
VMX_API int volta_cuda_hash_fp2_tree_device(void* raw, uint64_t matrix_id, size_t matrix_off, size_t rows,
                                               size_t cols, uint64_t tree_id, size_t tree_off_bytes) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !rows || !pow2_or_one(cols)) return fail_msg(c, "invalid resident Fp2 Merkle geometry");
    return guarded(c, "resident Fp2 Merkle tree",
                   [&] { return hash_tree_device(c, matrix_id, matrix_off, rows, cols, tree_id, tree_off_bytes, true); });
}

// Replaces volta_cuda_merkle_paths_device (.cu:7188-7204): for each query the
// log2(leaves) sibling hashes from the leaf level up (MerkleTree::open,
// rust/volta-pcs/src/merkle.rs:43-51).  Indices are validated by the Rust seam
// (rust/volta-accel/src/lib.rs:6735-6760); an out-of-range index yields zero
// hashes instead of reading outside the tree.
VMX_API int volta_cuda_merkle_paths_device(void* raw, uint64_t tree_id, size_t tree_off_bytes, size_t leaves,
                                              uint64_t idx_id, size_t idx_off, size_t queries, uint64_t paths_id,
                                              size_t paths_off_bytes) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !pow2(leaves) || !queries) return fail_msg(c, "invalid resident Merkle path geometry");
    return guarded(c, "resident Merkle paths", [&] {
        size_t bits = 0;
        while ((size_t{1} << bits) < leaves) ++bits;
        size_t tb = 0, pb = 0;
        if (leaves > SIZE_MAX / 2 || !mul_ok(2 * leaves - 1, 32, &tb) || !mul3_ok(queries, bits, 32, &pb))
            return fail_msg(c, "resident Merkle path geometry overflows size_t");
        void *tree = nullptr, *idx = nullptr, *paths = nullptr;
        if (region_elems(c, tree_id, tree_off_bytes, tb, 1, &tree, true) ||
            region_elems(c, idx_id, idx_off, queries, 4, &idx, true) ||
            region_elems(c, paths_id, paths_off_bytes, pb, 1, &paths))
            return -1;
        if (hash_aligned(c, tree, "Merkle tree") || hash_aligned(c, paths, "Merkle path")) return -1;
        if (begin_op(c) || mark_op(c, 1)) return -1;
        if (merkle_paths(c, static_cast<const uint32_t*>(tree), leaves, static_cast<const uint32_t*>(idx), queries,
                         static_cast<uint32_t*>(paths)))
            return -1;
        if (mark_op(c, 2)) return -1;
        return finish_op(c, OP_PCS_MERKLE, 0, 0);
    });
}

// Replaces volta_cuda_hash_fp_columns (.cu:7256-7265; caller
// Backend::hash_fp_columns, rust/volta-accel/src/lib.rs:6380-6405): host
// rows x cols Fp matrix in, cols x 32 leaf bytes out.  Same geometry rule:
// rows >= 8, rows % 8 == 0, cols a power of two.
VMX_API int volta_cuda_hash_fp_columns(void* raw, const uint64_t* matrix, size_t rows, size_t cols, uint8_t* leaves) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !matrix || !leaves || rows < 8 || rows % 8 || !pow2_or_one(cols))
        return fail_msg(c, "invalid PCS hash matrix geometry");
    return guarded(c, "PCS column hashes", [&] {
        size_t mb = 0, hb = 0;
        if (!mul3_ok(rows, cols, 8, &mb) || !mul_ok(cols, 32, &hb))
            return fail_msg(c, "PCS hash matrix geometry overflows size_t");
        if (ensure_ws(c, WS_IN, mb) || ensure_ws(c, WS_OUT, hb)) return -1;
        if (begin_op_h2d(c)) return -1;
        if (staged_copy(c, ws<void>(c, WS_IN), matrix, mb, hipMemcpyHostToDevice)) return -1;
        if (mark_op(c, 1)) return -1;
        if (merkle_column_leaves(c, ws<uint64_t>(c, WS_IN), rows, cols, false, ws<uint32_t>(c, WS_OUT))) return -1;
        if (mark_op(c, 2)) return -1;
        VMX_HIP(c, hipMemcpyAsync(leaves, ws<void>(c, WS_OUT), hb, hipMemcpyDeviceToHost, c->stream));
        return finish_op(c, OP_PCS_MERKLE, mb, hb);
    });
}

// ---------------------------------------------------------------------------
// Opening-path helpers
// ---------------------------------------------------------------------------

// Replaces volta_cuda_logup_eq_rows_device (.cu:6884-6911; callers
// Backend::logup_eq_rows_device and equality_weights_device,
// rust/volta-accel/src/lib.rs:6167-6205, 3037-3053): rows x 2^dims Fp2,
// out[r][x] = prod_k (bit k of x ? p[r][k] : 1 - p[r][k]).  dims = 0 writes
// one 1 per row and reads no points.
VMX_API int volta_cuda_logup_eq_rows_device(void* raw, uint64_t points_id, size_t points_off, size_t rows,
                                               size_t dims, uint64_t out_id, size_t out_off) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !rows || dims >= 63 || (dims && !points_id)) return fail_msg(c, "invalid resident eq-row geometry");
    return guarded(c, "resident eq rows", [&] {
        const size_t width = size_t{1} << dims;
        size_t total = 0, pn = 0;
        if (!mul_ok(rows, width, &total) || !mul_ok(rows, dims, &pn))
            return fail_msg(c, "resident eq-row geometry overflows size_t");
        void *points = nullptr, *out = nullptr;
        if ((dims && region_elems(c, points_id, points_off, pn, 16, &points, true)) ||
            region_elems(c, out_id, out_off, total, 16, &out))
            return -1;
        if (begin_op(c) || mark_op(c, 1)) return -1;
        if (eq_rows(c, static_cast<const Fp2*>(points), rows, dims, static_cast<Fp2*>(out))) return -1;
        if (mark_op(c, 2)) return -1;
        return finish_op(c, OP_LOGUP, 0, 0);
    });
}

// Replaces volta_cuda_fp2_row_dots_device (.cu:4049-4103; caller
// Backend::fp2_row_dots_device, rust/volta-accel/src/lib.rs:1873-1908):
// out[r] = sum_{j < len} a[r a_stride + j] b[r b_stride + j], element offsets
// and strides; the output may not overlap either input.
VMX_API int volta_cuda_fp2_row_dots_device(void* raw, uint64_t a_id, size_t a_off, size_t a_stride, uint64_t b_id,
                                              size_t b_off, size_t b_stride, uint64_t out_id, size_t out_off,
                                              size_t rows, size_t len) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !rows || !len || a_stride < len || b_stride < len) return fail_msg(c, "invalid Fp2 row-dot geometry");
    return guarded(c, "Fp2 row dots", [&] {
        size_t aob = 0, asb = 0, bob = 0, bsb = 0, rowb = 0;
        if (!mul_ok(a_off, 16, &aob) || !mul_ok(a_stride, 16, &asb) || !mul_ok(b_off, 16, &bob) ||
            !mul_ok(b_stride, 16, &bsb) || !mul_ok(len, 16, &rowb))
            return fail_msg(c, "Fp2 row-dot geometry overflows size_t");
        void *a = nullptr, *b = nullptr, *out = nullptr;
        size_t a_span = 0, b_span = 0;
        if (strided_region(c, a_id, aob, asb, rowb, rows, &a, &a_span, true) ||
            strided_region(c, b_id, bob, bsb, rowb, rows, &b, &b_span, true) ||
            region_elems(c, out_id, out_off, rows, 16, &out))
            return -1;
        auto overlaps = [&](const void* p, size_t n) {
            const char *o = static_cast<const char*>(out), *q = static_cast<const char*>(p);
            return o < q + n && q < o + rows * 16;
        };
        if (overlaps(a, a_span) || overlaps(b, b_span)) return fail_msg(c, "Fp2 row-dot output overlaps an input");
        if (begin_op(c) || mark_op(c, 1)) return -1;
        if (fp2_row_dots(c, static_cast<const Fp2*>(a), a_stride, static_cast<const Fp2*>(b), b_stride,
                         static_cast<Fp2*>(out), rows, len))
            return -1;
        if (mark_op(c, 2)) return -1;
        return finish_op(c, OP_PCS_ROWS, 0, 0);
    });
}

// ---------------------------------------------------------------------------
// X4 extension-field transforms
// ---------------------------------------------------------------------------

namespace {

constexpr size_t X4_MAX_N = size_t{1} << 33;

int log2_of(size_t n) {
    int b = 0;
    while ((size_t{1} << b) < n) ++b;
    return b;
}

bool x4_fold_geometry(size_t input_len, uint64_t c0, uint64_t c1) {
    return pow2(input_len) && input_len <= X4_MAX_N && c0 < gl::P && c1 < gl::P;
}

}  // namespace

// Replaces volta_cuda_x4b_ntt_fp2 (cuda/volta_cuda_backend.cu:5577-5634): the
// n-point NTT of the coefficients (zero beyond coefficient_len) with the X4
// root of order n (rust/volta-pcs/src/x4/ntt.rs:49-122), natural order.  The
// coefficient tail is zero-filled inside the transform's first pass (the
// stats still report it as zeroed bytes, as the reference's memset does); the
// X4 tables are uploaded once per size and counted as H2D bytes.
VMX_API int volta_cuda_x4b_ntt_fp2(void* raw, const Fp2* coefficients, size_t coefficient_len, size_t n,
                                   Fp2* output) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !coefficients || !output || !coefficient_len || coefficient_len > n || !pow2(n) || n > X4_MAX_N)
        return fail_msg(c, "invalid X4b Fp2 NTT geometry");
    return guarded(c, "X4b Fp2 NTT", [&] {
        size_t total = 0, in_bytes = 0;
        if (!mul_ok(n, sizeof(Fp2), &total) || !mul_ok(coefficient_len, sizeof(Fp2), &in_bytes))
            return fail_msg(c, "X4b Fp2 NTT byte geometry overflows size_t");
        if (ensure_ws(c, WS_IN, in_bytes) || ensure_ws(c, WS_OUT, total)) return -1;
        uint64_t h2d = 0;
        X4Tables tb;
        if (x4_tables(c, log2_of(n), &h2d, &tb)) return -1;
        if (begin_op_h2d(c)) return -1;
        if (staged_copy(c, ws<Fp2>(c, WS_IN), coefficients, in_bytes, hipMemcpyHostToDevice)) return -1;
        h2d += in_bytes;
        if (mark_op(c, 1)) return -1;
        if (x4_ntt(c, tb, ws<Fp2>(c, WS_IN), coefficient_len, ws<Fp2>(c, WS_OUT))) return -1;
        if (mark_op(c, 2)) return -1;
        if (staged_copy(c, output, ws<Fp2>(c, WS_OUT), total, hipMemcpyDeviceToHost)) return -1;
        return finish_op(c, OP_PCS_NTT, h2d, total, 0, total - in_bytes);
    });
}

// MI355X extension: the same X4 NTT on resident buffers (element offsets):
// in[in_off .. in_off + len) -> out[out_off .. out_off + n).  The regions must
// not overlap; the input is left unchanged.
VMX_API int volta_mi355x_x4_ntt_fp2_device(void* raw, uint64_t in_id, size_t in_off, size_t len, size_t n,
                                           uint64_t out_id, size_t out_off) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !len || len > n || !pow2(n) || n > X4_MAX_N) return fail_msg(c, "invalid resident X4 NTT geometry");
    return guarded(c, "resident X4 NTT", [&] {
        void *in = nullptr, *out = nullptr;
        if (region_elems(c, in_id, in_off, len, sizeof(Fp2), &in, true) ||
            region_elems(c, out_id, out_off, n, sizeof(Fp2), &out))
            return -1;
        const auto a = reinterpret_cast<uintptr_t>(in), b = reinterpret_cast<uintptr_t>(out);
        if (a < b + n * sizeof(Fp2) && b < a + len * sizeof(Fp2))
            return fail_msg(c, "resident X4 NTT input and output overlap");
        uint64_t h2d = 0;
        X4Tables tb;
        if (x4_tables(c, log2_of(n), &h2d, &tb)) return -1;
        if (begin_op(c) || mark_op(c, 1)) return -1;
        if (x4_ntt(c, tb, static_cast<const Fp2*>(in), len, static_cast<Fp2*>(out))) return -1;
        if (mark_op(c, 2)) return -1;
        return finish_op(c, OP_PCS_NTT, h2d, 0);
    });
}

// Replaces volta_cuda_x4c_direct_fold_arena (.cu:5925-5972): the codeword of
// input_len Fp2 at input_offset_bytes of the arena (a resident buffer) folds
// into input_len/2 Fp2 at output_offset_bytes (fold_codeword,
// rust/volta-pcs/src/x4/ntt.rs:238-256).
VMX_API int volta_cuda_x4c_direct_fold_arena(void* raw, uint64_t arena_id, size_t input_offset_bytes,
                                             size_t input_len, size_t output_offset_bytes, uint64_t challenge_c0,
                                             uint64_t challenge_c1) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !x4_fold_geometry(input_len, challenge_c0, challenge_c1))
        return fail_msg(c, "invalid X4c arena direct-fold geometry");
    return guarded(c, "X4c arena direct fold", [&] {
        const size_t half = input_len / 2;
        size_t in_bytes = 0, out_bytes = 0;
        if (!mul_ok(input_len, sizeof(Fp2), &in_bytes) || !mul_ok(half, sizeof(Fp2), &out_bytes))
            return fail_msg(c, "X4c arena direct-fold byte geometry overflows size_t");
        // 16 bytes: the reference's alignof(volta_x4b::Fp2)
        if ((input_offset_bytes | output_offset_bytes) % 16 != 0)
            return fail_msg(c, "misaligned X4c arena direct-fold region");
        void *in = nullptr, *out = nullptr;
        if (region(c, arena_id, input_offset_bytes, in_bytes, &in) ||
            region(c, arena_id, output_offset_bytes, out_bytes, &out))
            return -1;
        if (input_offset_bytes < output_offset_bytes + out_bytes && output_offset_bytes < input_offset_bytes + in_bytes)
            return fail_msg(c, "X4c arena direct-fold input/output overlap");
        uint64_t h2d = 0;
        X4Tables tb;
        if (x4_tables(c, log2_of(input_len), &h2d, &tb)) return -1;
        if (begin_op(c) || mark_op(c, 1)) return -1;
        const Fp2* pos = static_cast<const Fp2*>(in);
        if (x4_fold(c, tb, pos, pos + half, static_cast<Fp2*>(out), 0, half, Fp2{challenge_c0, challenge_c1}))
            return -1;
        ++c->stats.x4c_kernel_launches;
        if (mark_op(c, 2)) return -1;
        return finish_op(c, OP_PCS_ROWS, h2d, 0, 0, 0, out_bytes);
    });
}

// Replaces volta_cuda_x4c_upload_pinned (.cu:5808-5837): bytes from a pinned
// host region to a resident region.  The pinned source is in flight until the
// copy completes; another pinned upload from it is refused meanwhile.
VMX_API int volta_cuda_x4c_upload_pinned(void* raw, uint64_t pinned_id, size_t pinned_offset_bytes, uint64_t arena_id,
                                         size_t arena_offset_bytes, size_t bytes) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !bytes) return fail_msg(c, "invalid X4c pinned upload");
    return guarded(c, "X4c pinned upload", [&] {
        void *src = nullptr, *dst = nullptr;
        Pinned* owner = nullptr;
        if (pinned_region(c, pinned_id, pinned_offset_bytes, bytes, &src, &owner) ||
            region(c, arena_id, arena_offset_bytes, bytes, &dst))
            return -1;
        bool ready = false;
        if (pinned_ready(c, owner, &ready)) return -1;
        if (!ready) return reject(c, "X4c pinned upload source is still in flight");
        if (begin_transfer(c)) return -1;
        const auto t0 = std::chrono::steady_clock::now();
        const hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream);
        const auto t1 = std::chrono::steady_clock::now();
        if (e != hipSuccess) return fail_hip(c, "hipMemcpyAsync(X4c pinned upload)", e);
        if (pinned_mark_in_flight(c, owner)) return -1;
        ++c->stats.resident_h2d_host_calls;
        c->stats.resident_h2d_host_call_ns += std::chrono::duration_cast<std::chrono::nanoseconds>(t1 - t0).count();
        return finish_transfer(c, bytes, true);
    });
}

// Replaces volta_cuda_x4c_direct_fold_pinned_tile (.cu:5839-5923): outputs
// output_start .. output_start + output_count of the fold of an input_len
// codeword whose needed halves sit in a pinned tile (output_count positive
// values v[j], then output_count negative values v[j + input_len/2]).  The
// tile is staged through scratch (tile bytes at scratch_offset_bytes of the
// arena) and the outputs land at output_offset_bytes + 16 output_start.
VMX_API int volta_cuda_x4c_direct_fold_pinned_tile(void* raw, uint64_t pinned_id, size_t pinned_offset_bytes,
                                                   uint64_t arena_id, size_t output_offset_bytes,
                                                   size_t scratch_offset_bytes, size_t input_len, size_t output_start,
                                                   size_t output_count, uint64_t challenge_c0,
                                                   uint64_t challenge_c1) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !x4_fold_geometry(input_len, challenge_c0, challenge_c1) || !output_count ||
        output_start > input_len / 2 || output_count > input_len / 2 - output_start)
        return fail_msg(c, "invalid X4c pinned direct-fold geometry");
    return guarded(c, "X4c pinned direct fold", [&] {
        size_t tile_elems = 0, tile_bytes = 0, start_bytes = 0, tile_out_bytes = 0, out_bytes = 0;
        if (!mul_ok(output_count, 2, &tile_elems) || !mul_ok(tile_elems, sizeof(Fp2), &tile_bytes) ||
            !mul_ok(output_start, sizeof(Fp2), &start_bytes) || !mul_ok(output_count, sizeof(Fp2), &tile_out_bytes) ||
            !mul_ok(input_len / 2, sizeof(Fp2), &out_bytes))
            return fail_msg(c, "X4c pinned direct-fold byte geometry overflows size_t");
        if ((pinned_offset_bytes | output_offset_bytes | scratch_offset_bytes) % 16 != 0)
            return fail_msg(c, "misaligned X4c pinned direct-fold region");
        void *src = nullptr, *scratch = nullptr, *out = nullptr;
        Pinned* owner = nullptr;
        if (pinned_region(c, pinned_id, pinned_offset_bytes, tile_bytes, &src, &owner) ||
            region(c, arena_id, scratch_offset_bytes, tile_bytes, &scratch) ||
            region(c, arena_id, output_offset_bytes, out_bytes, &out))
            return -1;
        if (scratch_offset_bytes < output_offset_bytes + out_bytes &&
            output_offset_bytes < scratch_offset_bytes + tile_bytes)
            return fail_msg(c, "X4c pinned direct-fold scratch/output overlap");
        bool ready = false;
        if (pinned_ready(c, owner, &ready)) return -1;
        if (!ready) return reject(c, "X4c direct-fold pinned tile is still in flight");
        uint64_t h2d = 0;
        X4Tables tb;
        if (x4_tables(c, log2_of(input_len), &h2d, &tb)) return -1;
        if (begin_op_h2d(c)) return -1;
        const auto t0 = std::chrono::steady_clock::now();
        const hipError_t e = hipMemcpyAsync(scratch, src, tile_bytes, hipMemcpyHostToDevice, c->stream);
        const auto t1 = std::chrono::steady_clock::now();
        if (e != hipSuccess) return fail_hip(c, "hipMemcpyAsync(X4c direct-fold tile)", e);
        if (pinned_mark_in_flight(c, owner)) return -1;
        ++c->stats.resident_h2d_host_calls;
        c->stats.resident_h2d_host_call_ns += std::chrono::duration_cast<std::chrono::nanoseconds>(t1 - t0).count();
        if (mark_op(c, 1)) return -1;
        const Fp2* pos = static_cast<const Fp2*>(scratch);
        Fp2* dst = reinterpret_cast<Fp2*>(static_cast<unsigned char*>(out) + start_bytes);
        if (x4_fold(c, tb, pos, pos + output_count, dst, output_start, output_count, Fp2{challenge_c0, challenge_c1}))
            return -1;
        ++c->stats.x4c_kernel_launches;
        if (mark_op(c, 2)) return -1;
        return finish_op(c, OP_PCS_ROWS, h2d + tile_bytes, 0, 0, 0, tile_out_bytes);
    });
}

// Replaces volta_cuda_fp2_mobius_inverse_inplace_device (.cu:2965-2972,
// 7114-7130): for every bit of the index, upper += lower, over n = 2^k Fp2 at
// values_offset (elements) of the resident buffer.
VMX_API int volta_cuda_fp2_mobius_inverse_inplace_device(void* raw, uint64_t values_id, size_t values_offset,
                                                         size_t n) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !n || (n & (n - 1))) return fail_msg(c, "invalid resident Fp2 Mobius inverse");
    return guarded(c, "resident Fp2 Mobius inverse", [&] {
        void* v = nullptr;
        if (region_elems(c, values_id, values_offset, n, sizeof(Fp2), &v)) return -1;
        if (begin_op(c) || mark_op(c, 1)) return -1;
        if (fp2_mobius(c, static_cast<Fp2*>(v), n, true)) return -1;
        if (mark_op(c, 2)) return -1;
        return finish_op(c, OP_PCS_ROWS, 0, 0);
    });
}
