// context.cpp -- lifecycle, resident memory, pinned memory, stats and timing
// exports of the volta_cuda_* C ABI (ABI 37), written for HIP on gfx950.
//
// Behavioural contract (not code) follows the reference backend:
//   ids/regions           cuda/volta_cuda_backend.cu:296-345
//   create/destroy/error  :3150-3206          timing policy/coarse scopes :3208-3330
//   stats/memory          :3332-3470          resident alloc/free/copies  :3733-3950
//   pinned pool           :3560-3730
// Every entry point returns 0 on success and -1 (or a HIP status) on failure
// with a message for volta_cuda_last_error; nothing throws across the ABI.
#include "context.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <new>
#include <thread>

#include "gl64.hpp"

namespace vmx {

int fail_msg(Context* c, const char* msg) noexcept;

static void abort_record(Context* c) noexcept {
    if (!c) return;
    if (c->coarse_accounted) c->poisoned = true;
    if (c->record_active && c->timing_mode == TIMING_EVENTS_DEFERRED) c->ring[c->active_slot].mask = 0;
    c->reuse_slot = -1;  // a failed primitive may have enqueued work after the last marker
    c->record_active = false;
    c->coarse_active = false;
    c->coarse_inner = false;
    c->counter_active = false;
    c->coarse_accounted = false;
    c->coarse_op = -1;
}

int fail_msg(Context* c, const char* msg) noexcept {
    abort_record(c);
    if (c) {
        try {
            c->error = msg;
        } catch (...) {
        }
    }
    return -1;
}

int fail_hip(Context* c, const char* what, hipError_t e) noexcept {
    abort_record(c);
    if (c) {
        try {
            c->error = std::string(what) + ": " + hipGetErrorString(e);
        } catch (...) {
        }
    }
    return e == hipSuccess ? -1 : static_cast<int>(e);
}

int reject(Context* c, const char* msg) noexcept {
    if (c) {
        try {
            c->error = msg;
        } catch (...) {
        }
    }
    return -1;
}

bool mul_ok(size_t a, size_t b, size_t* out) {
    if (a != 0 && b > std::numeric_limits<size_t>::max() / a) return false;
    *out = a * b;
    return true;
}

bool mul3_ok(size_t a, size_t b, size_t c, size_t* out) {
    size_t ab = 0;
    return mul_ok(a, b, &ab) && mul_ok(ab, c, out);
}

bool add_ok(size_t a, size_t b, size_t* out) {
    if (b > std::numeric_limits<size_t>::max() - a) return false;
    *out = a + b;
    return true;
}

static uint64_t make_id(size_t slot, uint32_t gen) { return (static_cast<uint64_t>(gen) << 32) | (slot + 1); }

Resident* find_resident(Context* c, uint64_t id) {
    if (!c || !id) return nullptr;
    const uint64_t s = id & 0xFFFFFFFFull;
    const uint32_t gen = static_cast<uint32_t>(id >> 32);
    if (!s || !gen || s - 1 >= c->resident.size()) return nullptr;
    Resident& r = c->resident[s - 1];
    return (r.active && r.generation == gen) ? &r : nullptr;
}

void note_message_rows(Context* c, uint64_t id, size_t off, size_t rows, size_t row_len, size_t nonzero) {
    Resident* r = find_resident(c, id);
    if (!r || r->exposed) return;
    r->msg_rows = true;
    r->msg_off = off;
    r->msg_count = rows;
    r->msg_row_len = row_len;
    r->msg_nonzero = nonzero;
}

int settle_pending(Context* c) {
    if (!c->has_pending) return 0;
    const PendingMessages m = c->pending;
    c->has_pending = false;
    // The late write is the messages call's kernel: its time goes to PcsRows
    // (the call itself was counted when it was made).  Inside another
    // primitive's record or a coarse scope that window already times it.
    const bool timed = !c->record_active && !c->coarse_active && !c->counter_active &&
                       c->timing_mode != TIMING_WALL_ONLY_COUNTERS;
    if (timed && (begin_op(c) || mark_op(c, 1))) return -1;
    if (pcs_messages(c, m.w, m.pads, m.rows, m.cols, m.pad, m.code_len, m.out)) return -1;
    if (timed) {
        if (mark_op(c, 2)) return -1;
        c->uncounted = true;
        const int rc = finish_op(c, OP_PCS_ROWS, 0, 0);
        c->uncounted = false;
        if (rc) return -1;
    }
    note_message_rows(c, m.out_id, m.out_off, m.rows, m.code_len, m.cols + m.pad);
    return 0;
}

// Every entry point reaches resident memory through region(), so deferred
// message rows are written here before anything can read them or overwrite
// their sources (freeing a source writes them too, resident_free).
static bool touches_pending(const Context* c, uint64_t id, bool read_only) {
    const PendingMessages& m = c->pending;
    if (id == m.out_id) return true;
    return !read_only && (id == m.w_id || (m.pad && id == m.pads_id));
}

int region(Context* c, uint64_t id, size_t offset_bytes, size_t bytes, void** out, bool read_only) {
    if (c && c->has_pending && !c->bypass_settle && touches_pending(c, id, read_only) && settle_pending(c))
        return -1;
    Resident* r = find_resident(c, id);
    if (!r) return fail_msg(c, "unknown resident buffer id");
    if (offset_bytes > r->logical || bytes > r->logical - offset_bytes)
        return fail_msg(c, "resident buffer region is out of bounds");
    if (!read_only) r->msg_rows = false;  // anything but a read may change the recorded rows
    *out = static_cast<unsigned char*>(r->ptr) + offset_bytes;
    return 0;
}

int region_elems(Context* c, uint64_t id, size_t offset, size_t count, size_t elem, void** out, bool read_only) {
    size_t ob = 0, nb = 0;
    if (!mul_ok(offset, elem, &ob) || !mul_ok(count, elem, &nb))
        return fail_msg(c, "resident region geometry overflows size_t");
    return region(c, id, ob, nb, out, read_only);
}

int strided_region(Context* c, uint64_t id, size_t offset, size_t stride, size_t row_bytes,
                   size_t rows, void** out, size_t* span, bool read_only) {
    if (!rows || !row_bytes || stride < row_bytes)
        return fail_msg(c, "invalid resident strided-row geometry");
    size_t prefix = 0;
    if (!mul_ok(rows - 1, stride, &prefix) || !add_ok(prefix, row_bytes, span))
        return fail_msg(c, "resident strided-row geometry overflows size_t");
    return region(c, id, offset, *span, out, read_only);
}

// ---- synchronisation ---------------------------------------------------------

static uint64_t& reason_counter(RawStats& s, SyncReason r) {
    switch (r) {
        case SyncReason::HostOutput: return s.sync_host_output;
        case SyncReason::UploadLifetime: return s.sync_upload_lifetime;
        case SyncReason::TimingFlush: return s.sync_timing_flush;
        case SyncReason::ProfilingLegacy: return s.sync_profiling_legacy;
        case SyncReason::AllocatorFlush: return s.sync_allocator_flush;
    }
    return s.sync_profiling_legacy;
}

int sync_stream(Context* c, SyncReason reason) {
    const auto t0 = std::chrono::steady_clock::now();
    VMX_HIP(c, hipStreamSynchronize(c->stream));
    const auto t1 = std::chrono::steady_clock::now();
    ++c->stats.synchronizations;
    ++reason_counter(c->stats, reason);
    c->stats.synchronization_ns +=
        std::chrono::duration_cast<std::chrono::nanoseconds>(t1 - t0).count();
    c->outstanding = 0;
    c->counter_pending = false;
    for (auto& p : c->pinned) p.in_flight = false;
    stream_touched(c);
    return 0;
}

// ---- host <-> device copies of the host-pointer entry points ---------------------
// A plain hipMemcpyAsync between pageable host memory and the device moved
// 4 GiB of codewords at about 18 GB/s and 1 GiB of messages at about 30 GB/s.
// Staged, thread t of the copy's threads moves chunks t, t + T, t + 2T, ... of
// STAGE_SLOT_BYTES through its own pinned buffer and event, so the host-side
// copies of up to T chunks run at once while the DMA engine works through the
// stream:
//   download: queue the chunk's DMA into the buffer, wait for its event, copy
//     the buffer to the caller's memory;
//   upload: wait for the buffer's previous DMA, copy the caller's chunk into
//     it, queue its DMA.
// The threads' DMAs interleave on the one stream, after the work queued before
// the copy; each thread touches only its own buffer and event.

static bool stage_setup(Context* c) {
    if (c->stage_ready) return true;
    for (size_t t = 0; t < c->stage_buf.size(); ++t) {
        if (!c->stage_buf[t] && hipHostMalloc(&c->stage_buf[t], STAGE_SLOT_BYTES, hipHostMallocDefault) != hipSuccess) {
            c->stage_buf[t] = nullptr;
            return false;
        }
        if (!c->stage_ev[t]) {
            // recorded once here, so an upload's first wait on it has a
            // recorded event to wait for
            if (hipEventCreateWithFlags(&c->stage_ev[t], hipEventDisableTiming) != hipSuccess) {
                c->stage_ev[t] = nullptr;
                return false;
            }
            if (hipEventRecord(c->stage_ev[t], c->stream) != hipSuccess) return false;
        }
    }
    c->stage_ready = true;
    return true;
}

int staged_copy(Context* c, void* dst, const void* src, size_t bytes, hipMemcpyKind kind) {
    if (kind != hipMemcpyDeviceToHost && kind != hipMemcpyHostToDevice) return fail_msg(c, "staged copy: bad kind");
    stream_touched(c);
    // A host buffer the caller pinned needs no staging.  For pageable memory
    // the query fails (hipErrorInvalidValue); its error is cleared at once so
    // that no later hipGetLastError reports it.
    bool pinned = false;
    if (bytes >= STAGE_MIN_BYTES) {
        hipPointerAttribute_t attr{};
        if (hipPointerGetAttributes(&attr, kind == hipMemcpyDeviceToHost ? dst : src) == hipSuccess)
            pinned = attr.type == hipMemoryTypeHost;
        else
            (void)hipGetLastError();
    }
    if (bytes < STAGE_MIN_BYTES || pinned || !stage_setup(c)) {
        VMX_HIP(c, hipMemcpyAsync(dst, src, bytes, kind, c->stream));
        return 0;
    }
    const size_t chunks = (bytes + STAGE_SLOT_BYTES - 1) / STAGE_SLOT_BYTES;
    const size_t threads = std::min(chunks, c->stage_buf.size());
    const bool down = kind == hipMemcpyDeviceToHost;
    unsigned char* d = static_cast<unsigned char*>(dst);
    const unsigned char* s = static_cast<const unsigned char*>(src);
    std::vector<hipError_t> err(threads, hipSuccess);
    auto work = [&](size_t t) {
        // a new thread's current device is the default one: use the context's
        hipError_t e = t ? hipSetDevice(c->device) : hipSuccess;
        void* buf = c->stage_buf[t];
        hipEvent_t ev = c->stage_ev[t];
        for (size_t k = t; k < chunks && e == hipSuccess; k += threads) {
            const size_t off = k * STAGE_SLOT_BYTES, len = std::min(STAGE_SLOT_BYTES, bytes - off);
            if (down) {
                e = hipMemcpyAsync(buf, s + off, len, hipMemcpyDeviceToHost, c->stream);
                if (e == hipSuccess) e = hipEventRecord(ev, c->stream);
                if (e == hipSuccess) e = hipEventSynchronize(ev);
                if (e == hipSuccess) std::memcpy(d + off, buf, len);
            } else {
                e = hipEventSynchronize(ev);  // the buffer's previous DMA (none: returns at once)
                if (e == hipSuccess) std::memcpy(buf, s + off, len);
                if (e == hipSuccess) e = hipMemcpyAsync(d + off, buf, len, hipMemcpyHostToDevice, c->stream);
                if (e == hipSuccess) e = hipEventRecord(ev, c->stream);
            }
        }
        err[t] = e;
    };
    std::vector<std::thread> pool;
    pool.reserve(threads - 1);
    try {
        for (size_t t = 1; t < threads; ++t) pool.emplace_back(work, t);
    } catch (...) {
        for (auto& th : pool) th.join();
        return fail_msg(c, "staged copy: could not start its threads");
    }
    work(0);
    for (auto& th : pool) th.join();
    for (hipError_t e : err)
        if (e != hipSuccess) return fail_hip(c, down ? "staged copy (device to host)" : "staged copy (host to device)", e);
    return 0;
}

// ---- workspaces and twiddles -----------------------------------------------------

int ensure_ws(Context* c, int slot, size_t bytes) {
    if (slot < 0 || slot >= WS_COUNT) return fail_msg(c, "invalid workspace slot");
    Workspace& w = c->ws[slot];
    if (w.capacity >= bytes) return 0;
    if (c->coarse_active) return reject(c, "workspace growth is forbidden inside a coarse timing scope");
    if (w.ptr) {
        if (sync_stream(c, SyncReason::AllocatorFlush)) return -1;
        VMX_HIP(c, hipFree(w.ptr));
        ++c->stats.physical_free_calls;
        c->stats.live_device_bytes -= w.capacity;
        w = Workspace{};
    }
    VMX_HIP(c, hipMalloc(&w.ptr, bytes));
    w.capacity = bytes;
    ++c->stats.allocation_calls;
    c->stats.live_device_bytes += bytes;
    c->stats.peak_device_bytes = std::max(c->stats.peak_device_bytes, c->stats.live_device_bytes);
    return 0;
}

static int upload_table(Context* c, const std::vector<uint64_t>& host, uint64_t** out,
                        uint64_t* h2d) {
    const size_t bytes = host.size() * sizeof(uint64_t);
    void* p = nullptr;
    VMX_HIP(c, hipMalloc(&p, bytes));
    ++c->stats.allocation_calls;
    c->stats.live_device_bytes += bytes;
    c->stats.peak_device_bytes = std::max(c->stats.peak_device_bytes, c->stats.live_device_bytes);
    // The host vector dies on return: the copy must complete first.
    VMX_HIP(c, hipMemcpyAsync(p, host.data(), bytes, hipMemcpyHostToDevice, c->stream));
    if (sync_stream(c, SyncReason::UploadLifetime)) return -1;
    *h2d += bytes;
    *out = static_cast<uint64_t*>(p);
    return 0;
}

static int tw_log2(size_t n) {
    int b = 0;
    while ((size_t{1} << b) < n) ++b;
    return b;
}

int ensure_twiddles(Context* c, size_t n, uint64_t* h2d, TwiddleSet** out) {
    TwiddleSet& t = c->twiddles[n];
    t.n = n;
    if (!t.fwd) {
        if (c->coarse_active) return reject(c, "twiddle upload is forbidden inside a coarse timing scope");
        std::vector<uint64_t> host(std::max<size_t>(n / 2, 1));
        const uint64_t w = gl::root_of_unity(static_cast<unsigned>(tw_log2(n)));
        uint64_t acc = 1;
        for (size_t i = 0; i < n / 2; ++i) {
            host[i] = acc;
            acc = gl::mul(acc, w);
        }
        if (upload_table(c, host, &t.fwd, h2d)) return -1;
    }
    // the pass engine's tables come from fwd on the device: no further H2D
    if (!t.reg && n <= (size_t{1} << 31) && reg_ntt_covers(n)) {
        stream_touched(c);  // the tables' kernels run outside any primitive's markers
        if (derive_reg_tables(c, &t)) return -1;
    }
    *out = &t;
    return 0;
}

int ensure_split_twiddles(Context* c, size_t n, uint64_t* h2d, TwiddleSet** out) {
    TwiddleSet& t = c->twiddles[n];
    t.n = n;
    if (!t.split) {
        if (c->coarse_active) return reject(c, "twiddle upload is forbidden inside a coarse timing scope");
        const int bits = tw_log2(n);
        const int h = (bits + 1) / 2;
        const size_t lo = size_t{1} << h, hi = n >> h;
        std::vector<uint64_t> host(lo + hi);
        const uint64_t w = gl::root_of_unity(static_cast<unsigned>(bits));
        uint64_t acc = 1;
        for (size_t i = 0; i < lo; ++i) {
            host[i] = acc;
            acc = gl::mul(acc, w);
        }
        // acc = w^(2^h) now
        const uint64_t step = acc;
        acc = 1;
        for (size_t i = 0; i < hi; ++i) {
            host[lo + i] = acc;
            acc = gl::mul(acc, step);
        }
        if (upload_table(c, host, &t.split, h2d)) return -1;
        t.split_h = h;
        t.split_bytes = host.size() * sizeof(uint64_t);
    }
    *out = &t;
    return 0;
}

int ensure_inverse_twiddles(Context* c, size_t n, uint64_t* h2d, TwiddleSet** out) {
    TwiddleSet* t = nullptr;
    if (ensure_twiddles(c, n, h2d, &t)) return -1;
    if (!t->inv) {
        if (c->coarse_active) return reject(c, "twiddle upload is forbidden inside a coarse timing scope");
        std::vector<uint64_t> host(std::max<size_t>(n / 2, 1));
        const uint64_t w = gl::inv_host(gl::root_of_unity(static_cast<unsigned>(tw_log2(n))));
        uint64_t acc = 1;
        for (size_t i = 0; i < n / 2; ++i) {
            host[i] = acc;
            acc = gl::mul(acc, w);
        }
        if (upload_table(c, host, &t->inv, h2d)) return -1;
    }
    *out = t;
    return 0;
}

int ensure_grid_twiddles(Context* c, TwiddleSet* t, size_t bytes, int (*build)(Context*, TwiddleSet*)) {
    if (t->grid) return 0;
    if (c->coarse_active) return reject(c, "twiddle table growth is forbidden inside a coarse timing scope");
    void* p = nullptr;
    VMX_HIP(c, hipMalloc(&p, bytes));
    ++c->stats.allocation_calls;
    c->stats.live_device_bytes += bytes;
    c->stats.peak_device_bytes = std::max(c->stats.peak_device_bytes, c->stats.live_device_bytes);
    t->grid = static_cast<uint64_t*>(p);
    t->grid_bytes = bytes;
    return build(c, t);
}

// ---- events --------------------------------------------------------------------------

// Timing events only measure: nothing reads device memory on the strength of
// their completion (downloads and pinned buffers synchronise by other means),
// so they skip the system-scope release, which writes back and invalidates the
// caches at every record and left ~15 us of idle GPU between primitives.
static hipError_t ev_create(Context* c, hipEvent_t* e) {
    ++c->stats.timing_event_api_calls;
    return hipEventCreateWithFlags(e, hipEventDisableSystemFence);
}

static hipError_t ev_record(Context* c, hipEvent_t e) {
    ++c->stats.timing_event_api_calls;
    stream_touched(c);
    return hipEventRecord(e, c->stream);
}

// One elapsed-time query; *ok is false when the runtime reports success but
// no finite duration (counted as a no-write, never as zero time).
static int ev_elapsed(Context* c, hipEvent_t a, hipEvent_t b, uint64_t* ns, bool* ok) {
    ++c->stats.timing_elapsed_query_attempts;
    if (c->inject_no_write) {
        --c->inject_no_write;
        ++c->stats.timing_elapsed_no_write;
        *ok = false;
        return 0;
    }
    float ms = -1.0f;
    ++c->stats.timing_event_api_calls;
    const hipError_t e = hipEventElapsedTime(&ms, a, b);
    if (e != hipSuccess) return fail_hip(c, "hipEventElapsedTime", e);
    if (std::isfinite(ms) && ms >= 0.0f) {
        *ns = static_cast<uint64_t>(static_cast<double>(ms) * 1.0e6);
        ++c->stats.timing_event_queries;
        *ok = true;
    } else {
        ++c->stats.timing_elapsed_no_write;
        *ok = false;
    }
    return 0;
}

// Bounded retry: a duration that is never reported is an error, not zero.
static int ev_ns(Context* c, hipEvent_t a, hipEvent_t b, uint64_t* ns) {
    for (int attempt = 0; attempt < 3; ++attempt) {
        bool ok = false;
        if (ev_elapsed(c, a, b, ns, &ok)) return -1;
        if (ok) return 0;
    }
    return fail_msg(c, "event elapsed time was never reported");
}

static int ring_take(Context* c, size_t* slot) {
    if (c->ring_pending == TIMING_RING_SIZE && flush_deferred(c, SyncReason::TimingFlush)) return -1;
    *slot = (c->ring_begin + c->ring_pending) % TIMING_RING_SIZE;
    TimingRecord& r = c->ring[*slot];
    for (auto& e : r.ev)
        if (!e) VMX_HIP(c, ev_create(c, &e));
    r.mask = 0;
    r.start = nullptr;
    r.op = -1;
    r.coarse = r.transfer_h2d = r.transfer_d2h = false;
    r.h2d = r.d2h = r.d2d = r.zeroed = r.generated = 0;
    return 0;
}

static void ring_commit(Context* c) {
    ++c->ring_pending;
    c->stats.timing_pending_high_water =
        std::max<uint64_t>(c->stats.timing_pending_high_water, c->ring_pending);
    c->record_active = false;
}

int flush_deferred(Context* c, SyncReason reason) {
    if (c->timing_mode != TIMING_EVENTS_DEFERRED || c->ring_pending == 0) return 0;
    if (sync_stream(c, reason)) return -1;
    while (c->ring_pending) {
        TimingRecord& r = c->ring[c->ring_begin];
        uint64_t ns = 0;
        if (r.coarse) {
            if (ev_ns(c, r.ev[0], r.ev[1], &ns)) return -1;
            c->stats.coarse_timing_ns += ns;
            c->stats.kernel_ns[r.op] += ns;
        } else if (r.transfer_h2d || r.transfer_d2h) {
            if (ev_ns(c, r.ev[0], r.ev[1], &ns)) return -1;
            if (r.transfer_h2d) c->stats.h2d_ns += ns;
            else c->stats.d2h_ns += ns;
        } else {
            if (r.h2d) {
                if (ev_ns(c, r.ev[0], r.ev[1], &ns)) return -1;
                c->stats.h2d_ns += ns;
            }
            if (ev_ns(c, r.start ? r.start : r.ev[1], r.ev[2], &ns)) return -1;
            c->stats.kernel_ns[r.op] += ns;
            if (r.d2h) {
                if (ev_ns(c, r.ev[2], r.ev[3], &ns)) return -1;
                c->stats.d2h_ns += ns;
            }
        }
        ++c->stats.timing_records;
        c->ring_begin = (c->ring_begin + 1) % TIMING_RING_SIZE;
        --c->ring_pending;
    }
    ++c->stats.timing_flush_count;
    return 0;
}

// ---- primitive accounting ----------------------------------------------------------

int begin_op(Context* c) {
    std::fill(std::begin(c->phase_ns), std::end(c->phase_ns), 0);
    if (c->coarse_active) {
        if (c->coarse_inner) return reject(c, "nested primitive timing inside a coarse timing scope");
        c->coarse_inner = true;
        return 0;
    }
    switch (c->timing_mode) {
        case TIMING_WALL_ONLY_COUNTERS:
            if (c->counter_active) return reject(c, "nested counter-only timing record");
            c->counter_active = true;
            return 0;
        case TIMING_EVENTS_DEFERRED: {
            // The record's opening event is only needed to time a host upload
            // before marker 1 (begin_op_h2d); a device-only primitive records
            // markers 1 and 2 alone, two event records per call instead of four.
            size_t slot = 0;
            if (ring_take(c, &slot)) return -1;
            c->active_slot = slot;
            c->record_active = true;
            return 0;
        }
        case TIMING_EVENTS:
            c->record_active = true;
            VMX_HIP(c, ev_record(c, c->events[0]));
            return 0;
        default:
            c->record_active = true;
            c->phase_start = std::chrono::steady_clock::now();
            return 0;
    }
}

int begin_op_h2d(Context* c) {
    if (begin_op(c)) return -1;
    if (c->timing_mode == TIMING_EVENTS_DEFERRED && !c->coarse_active) {
        VMX_HIP(c, ev_record(c, c->ring[c->active_slot].ev[0]));
        c->ring[c->active_slot].mask |= 1;
    }
    return 0;
}

// Marker 1 of a device-only record can be the previous record's marker 2 when
// that marker is still the last thing enqueued on the stream and the device
// has not reached it: the kernels that follow then start as soon as it
// completes, exactly as they would after a marker of their own, and the stream
// runs one marker fewer.  Each marker costs the device about 3 us between
// kernels on this runtime (the next dispatch is only processed after it), a
// third of a small configuration's step.  A marker the device has already
// passed is not borrowed: the stream may have gone idle since, and that gap is
// no kernel's time.  The window between this query and the next launch is the
// only slack (host microseconds, and only when the device catches up within it).
static int borrow_start(Context* c, TimingRecord* r) {
    const long prev = c->reuse_slot;
    c->reuse_slot = -1;
    if (prev < 0) return 0;
    hipEvent_t e = c->ring[static_cast<size_t>(prev)].ev[2];
    ++c->stats.timing_event_api_calls;
    const hipError_t q = hipEventQuery(e);
    if (q == hipSuccess) return 0;
    if (q != hipErrorNotReady) return fail_hip(c, "hipEventQuery", q);
    (void)hipGetLastError();  // not-ready is a state: keep it out of the next launch check
    r->start = e;
    return 1;
}

int mark_op(Context* c, int which) {
    if (which != 1 && which != 2) return fail_msg(c, "invalid timing marker");
    if (c->coarse_active) return c->coarse_inner ? 0 : fail_msg(c, "coarse marker without primitive");
    switch (c->timing_mode) {
        case TIMING_WALL_ONLY_COUNTERS:
            return c->counter_active ? 0 : fail_msg(c, "counter marker without primitive");
        case TIMING_EVENTS_DEFERRED: {
            if (!c->record_active) return fail_msg(c, "deferred marker without record");
            TimingRecord& r = c->ring[c->active_slot];
            if (which == 1 && !(r.mask & 1)) {
                const int shared = borrow_start(c, &r);
                if (shared < 0) return -1;
                if (shared) {
                    r.mask |= 2;
                    return 0;
                }
            }
            VMX_HIP(c, ev_record(c, r.ev[which]));
            r.mask |= static_cast<uint8_t>(1u << which);
            return 0;
        }
        case TIMING_EVENTS:
            VMX_HIP(c, ev_record(c, c->events[which]));
            return 0;
        default: {
            // Host-barrier wall mode: each phase ends at a barrier.
            VMX_HIP(c, hipStreamSynchronize(c->stream));
            const auto now = std::chrono::steady_clock::now();
            c->phase_ns[which - 1] =
                std::chrono::duration_cast<std::chrono::nanoseconds>(now - c->phase_start).count();
            c->phase_start = now;
            return 0;
        }
    }
}

static void account(Context* c, int op, uint64_t h2d, uint64_t d2h, uint64_t d2d, uint64_t zeroed,
                    uint64_t generated) {
    if (!c->uncounted) ++c->stats.calls[op];
    c->stats.h2d_bytes += h2d;
    c->stats.d2h_bytes += d2h;
    c->stats.d2d_bytes += d2d;
    c->stats.device_zeroed_bytes += zeroed;
    c->stats.device_generated_bytes += generated;
}

int finish_op(Context* c, int op, uint64_t h2d, uint64_t d2h, uint64_t d2d, uint64_t zeroed,
              uint64_t generated) {
    ++c->outstanding;
    if (c->coarse_active) {
        if (!c->coarse_inner) return fail_msg(c, "coarse finish without primitive");
        if (op != c->coarse_op) return fail_msg(c, "coarse timing scope received a different operation kind");
        if (h2d || d2h) {
            if (sync_stream(c, d2h ? SyncReason::HostOutput : SyncReason::UploadLifetime)) return -1;
            return fail_msg(c, "host transfer is forbidden inside a coarse timing scope");
        }
        account(c, op, 0, 0, d2d, zeroed, generated);
        c->coarse_accounted = true;
        if (c->timing_mode == TIMING_WALL_ONLY_COUNTERS) c->counter_pending = true;
        c->coarse_inner = false;
        return 0;
    }
    switch (c->timing_mode) {
        case TIMING_WALL_ONLY_COUNTERS:
            if (!c->counter_active) return fail_msg(c, "counter finish without primitive");
            c->counter_active = false;
            c->counter_pending = true;
            if (d2h && sync_stream(c, SyncReason::HostOutput)) return -1;
            account(c, op, h2d, d2h, d2d, zeroed, generated);
            return 0;
        case TIMING_EVENTS_DEFERRED: {
            if (!c->record_active) return fail_msg(c, "deferred finish without record");
            TimingRecord& r = c->ring[c->active_slot];
            if (d2h) {  // the closing event only times a download after marker 2
                VMX_HIP(c, ev_record(c, r.ev[3]));
                r.mask |= 8;
            }
            r.op = op;
            // upload time is measured when the primitive opened with
            // begin_op_h2d (twiddle tables uploaded before the record count
            // their bytes only)
            r.h2d = (r.mask & 1) ? h2d : 0;
            r.d2h = d2h;
            ring_commit(c);
            // marker 2 is the stream's last item unless a download followed it
            if (!d2h && (r.mask & 4)) c->reuse_slot = static_cast<long>(c->active_slot);
            account(c, op, h2d, d2h, d2d, zeroed, generated);
            return d2h ? flush_deferred(c, SyncReason::HostOutput) : 0;
        }
        case TIMING_EVENTS: {
            VMX_HIP(c, ev_record(c, c->events[3]));
            c->record_active = false;
            const SyncReason why = d2h ? SyncReason::HostOutput
                                       : (h2d ? SyncReason::UploadLifetime : SyncReason::ProfilingLegacy);
            if (sync_stream(c, why)) return -1;
            uint64_t a = 0, k = 0, b = 0;
            if (ev_ns(c, c->events[0], c->events[1], &a) || ev_ns(c, c->events[1], c->events[2], &k) ||
                ev_ns(c, c->events[2], c->events[3], &b))
                return -1;
            account(c, op, h2d, d2h, d2d, zeroed, generated);
            if (h2d) c->stats.h2d_ns += a;
            c->stats.kernel_ns[op] += k;
            if (d2h) c->stats.d2h_ns += b;
            return 0;
        }
        default: {
            c->record_active = false;
            VMX_HIP(c, hipStreamSynchronize(c->stream));
            c->phase_ns[2] = std::chrono::duration_cast<std::chrono::nanoseconds>(
                                 std::chrono::steady_clock::now() - c->phase_start)
                                 .count();
            // Three barriers per primitive in this mode, classified by cause.
            c->stats.synchronizations += 3;
            if (h2d) ++c->stats.sync_upload_lifetime;
            if (d2h) ++c->stats.sync_host_output;
            c->stats.sync_profiling_legacy += 3 - (h2d ? 1 : 0) - (d2h ? 1 : 0);
            account(c, op, h2d, d2h, d2d, zeroed, generated);
            if (h2d) c->stats.h2d_ns += c->phase_ns[0];
            c->stats.kernel_ns[op] += c->phase_ns[1];
            if (d2h) c->stats.d2h_ns += c->phase_ns[2];
            return 0;
        }
    }
}

int empty_op(Context* c, int op) {
    if (c->timing_mode != TIMING_EVENTS_DEFERRED || c->coarse_active)
        return (begin_op(c) || mark_op(c, 1) || mark_op(c, 2)) ? -1 : finish_op(c, op, 0, 0);
    if (c->record_active) return fail_msg(c, "empty primitive inside a timing record");
    ++c->outstanding;
    account(c, op, 0, 0, 0, 0, 0);
    return 0;
}

int begin_transfer(Context* c) {
    if (c->coarse_active) return reject(c, "host transfer is forbidden inside a coarse timing scope");
    switch (c->timing_mode) {
        case TIMING_WALL_ONLY_COUNTERS:
            if (c->counter_active) return reject(c, "nested counter-only timing record");
            c->counter_active = true;
            return 0;
        case TIMING_EVENTS_DEFERRED: {
            size_t slot = 0;
            if (ring_take(c, &slot)) return -1;
            c->active_slot = slot;
            c->record_active = true;
            VMX_HIP(c, ev_record(c, c->ring[slot].ev[0]));
            c->ring[slot].mask |= 1;
            return 0;
        }
        case TIMING_EVENTS:
            c->record_active = true;
            VMX_HIP(c, ev_record(c, c->events[0]));
            return 0;
        default:
            c->record_active = true;
            c->phase_start = std::chrono::steady_clock::now();
            return 0;
    }
}

int finish_transfer(Context* c, size_t bytes, bool h2d) {
    ++c->outstanding;
    switch (c->timing_mode) {
        case TIMING_WALL_ONLY_COUNTERS:
            if (!c->counter_active) return fail_msg(c, "counter transfer finish without transfer");
            c->counter_active = false;
            c->counter_pending = true;
            if (!h2d && sync_stream(c, SyncReason::HostOutput)) return -1;
            (h2d ? c->stats.h2d_bytes : c->stats.d2h_bytes) += bytes;
            return 0;
        case TIMING_EVENTS_DEFERRED: {
            if (!c->record_active) return fail_msg(c, "deferred transfer finish without record");
            TimingRecord& r = c->ring[c->active_slot];
            VMX_HIP(c, ev_record(c, r.ev[1]));
            r.mask |= 2;
            r.transfer_h2d = h2d;
            r.transfer_d2h = !h2d;
            ring_commit(c);
            (h2d ? c->stats.h2d_bytes : c->stats.d2h_bytes) += bytes;
            return h2d ? 0 : flush_deferred(c, SyncReason::HostOutput);
        }
        case TIMING_EVENTS: {
            VMX_HIP(c, ev_record(c, c->events[1]));
            c->record_active = false;
            if (sync_stream(c, h2d ? SyncReason::UploadLifetime : SyncReason::HostOutput)) return -1;
            uint64_t ns = 0;
            if (ev_ns(c, c->events[0], c->events[1], &ns)) return -1;
            if (h2d) {
                c->stats.h2d_bytes += bytes;
                c->stats.h2d_ns += ns;
            } else {
                c->stats.d2h_bytes += bytes;
                c->stats.d2h_ns += ns;
            }
            return 0;
        }
        default: {
            c->record_active = false;
            if (sync_stream(c, h2d ? SyncReason::UploadLifetime : SyncReason::HostOutput)) return -1;
            const uint64_t ns = std::chrono::duration_cast<std::chrono::nanoseconds>(
                                    std::chrono::steady_clock::now() - c->phase_start)
                                    .count();
            if (h2d) {
                c->stats.h2d_bytes += bytes;
                c->stats.h2d_ns += ns;
            } else {
                c->stats.d2h_bytes += bytes;
                c->stats.d2h_ns += ns;
            }
            return 0;
        }
    }
}

// ---- resident pool ----------------------------------------------------------------------

static int trim_resident(Context* c) {
    bool any = false;
    for (size_t s : c->free_slots)
        if (c->resident[s].ptr) any = true;
    if (!any) return 0;
    if (sync_stream(c, SyncReason::AllocatorFlush)) return -1;
    for (size_t s : c->free_slots) {
        Resident& r = c->resident[s];
        if (!r.ptr) continue;
        VMX_HIP(c, hipFree(r.ptr));
        ++c->stats.physical_free_calls;
        c->stats.live_device_bytes -= r.capacity;
        r.ptr = nullptr;
        r.capacity = 0;
    }
    return 0;
}

static int trim_pinned(Context* c) {
    bool any = false;
    for (size_t s : c->free_pinned)
        if (c->pinned[s].ptr) any = true;
    if (!any) return 0;
    if (sync_stream(c, SyncReason::AllocatorFlush)) return -1;
    for (size_t s : c->free_pinned) {
        Pinned& p = c->pinned[s];
        if (!p.ptr) continue;
        if (p.ready) (void)hipEventDestroy(p.ready);
        p.ready = nullptr;
        VMX_HIP(c, hipHostFree(p.ptr));
        ++c->stats.pinned_physical_free_calls;
        c->stats.live_pinned_bytes -= p.capacity;
        p.ptr = nullptr;
        p.capacity = 0;
    }
    return 0;
}

static Pinned* find_pinned(Context* c, uint64_t id) {
    if (!c || !id) return nullptr;
    const uint64_t s = id & 0xFFFFFFFFull;
    const uint32_t gen = static_cast<uint32_t>(id >> 32);
    if (!s || !gen || s - 1 >= c->pinned.size()) return nullptr;
    Pinned& p = c->pinned[s - 1];
    return (p.active && p.generation == gen) ? &p : nullptr;
}

int pinned_region(Context* c, uint64_t id, size_t offset_bytes, size_t bytes, void** out, Pinned** owner) {
    Pinned* p = find_pinned(c, id);
    if (!p) return fail_msg(c, "unknown or stale pinned buffer id");
    if (offset_bytes > p->logical || bytes > p->logical - offset_bytes)
        return fail_msg(c, "pinned buffer region is out of bounds");
    *out = static_cast<unsigned char*>(p->ptr) + offset_bytes;
    if (owner) *owner = p;
    return 0;
}

int pinned_ready(Context* c, Pinned* p, bool* ready) {
    if (!p->in_flight) {
        *ready = true;
        return 0;
    }
    const hipError_t e = hipEventQuery(p->ready);
    if (e == hipSuccess) {
        p->in_flight = false;
        *ready = true;
        return 0;
    }
    if (e == hipErrorNotReady) {
        *ready = false;
        return 0;
    }
    return fail_hip(c, "hipEventQuery(pinned ready)", e);
}

int pinned_mark_in_flight(Context* c, Pinned* p) {
    if (!p->ready) return fail_msg(c, "pinned buffer has no ready event");
    stream_touched(c);
    VMX_HIP(c, hipEventRecord(p->ready, c->stream));
    p->in_flight = true;
    return 0;
}

}  // namespace vmx

using namespace vmx;

#define VMX_GUARD_BEGIN try {
#define VMX_GUARD_END(c, what)                                   \
    }                                                            \
    catch (const std::exception&) {                              \
        return fail_msg((c), what " threw a C++ exception");     \
    }                                                            \
    catch (...) {                                                \
        return fail_msg((c), what " threw an unknown exception"); \
    }

VMX_API uint32_t volta_cuda_abi_version(void) { return ABI_VERSION; }

VMX_API int volta_cuda_create(void** out) {
    if (!out) return -1;
    *out = nullptr;
    Context* c = new (std::nothrow) Context;
    if (!c) return -1;
    *out = c;
    VMX_GUARD_BEGIN
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess) return fail_hip(c, "hipGetDeviceCount", e);
    if (count < 1) return fail_msg(c, "no HIP device is available");
    VMX_HIP(c, hipGetDevice(&c->device));
    VMX_HIP(c, hipDeviceGetAttribute(&c->cu_count, hipDeviceAttributeMultiprocessorCount, c->device));
    // Default-priority non-blocking stream: all context work is ordered on it.
    VMX_HIP(c, hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
    for (auto& ev : c->events) VMX_HIP(c, ev_create(c, &ev));
    // Probe event timing once; fall back to host barriers if unusable.
    VMX_HIP(c, ev_record(c, c->events[0]));
    VMX_HIP(c, ev_record(c, c->events[1]));
    VMX_HIP(c, hipStreamSynchronize(c->stream));
    float ms = -1.0f;
    e = hipEventElapsedTime(&ms, c->events[0], c->events[1]);
    ++c->stats.timing_event_api_calls;
    if (e == hipSuccess && ms >= 0.0f) {
        c->timing_mode = TIMING_EVENTS;
    } else {
        (void)hipGetLastError();
        c->timing_mode = TIMING_HOST_BARRIER_WALL;
    }
    c->stats.timing_mode = c->timing_mode;
    // Resolve this device's scratch array of the allocation-free combination.
    // A failure only disables that entry point, which then reports it.
    (void)combine_scratch_attach(c);
    return 0;
    VMX_GUARD_END(c, "context construction")
}

VMX_API void volta_cuda_destroy(void* raw) {
    Context* c = static_cast<Context*>(raw);
    if (!c) return;
    try {
        if (c->coarse_active) abort_record(c);
        if (c->timing_mode == TIMING_EVENTS_DEFERRED) (void)flush_deferred(c, SyncReason::TimingFlush);
        if (c->stream) (void)hipStreamSynchronize(c->stream);
        for (auto& w : c->ws)
            if (w.ptr) (void)hipFree(w.ptr);
        for (auto& r : c->resident)
            if (r.ptr) (void)hipFree(r.ptr);
        for (auto& kv : c->twiddles) {
            if (kv.second.fwd) (void)hipFree(kv.second.fwd);
            if (kv.second.inv) (void)hipFree(kv.second.inv);
            if (kv.second.grid) (void)hipFree(kv.second.grid);
            if (kv.second.split) (void)hipFree(kv.second.split);
            if (kv.second.reg) (void)hipFree(kv.second.reg);
            for (uint64_t* t : kv.second.col)
                if (t) (void)hipFree(t);
            for (uint64_t* t : kv.second.col_scaled)
                if (t) (void)hipFree(t);
        }
        for (auto& p : c->pinned) {
            if (p.ready) (void)hipEventDestroy(p.ready);
            if (p.ptr) (void)hipHostFree(p.ptr);
        }
        for (auto& r : c->ring)
            for (auto e : r.ev)
                if (e) (void)hipEventDestroy(e);
        for (auto e : c->events)
            if (e) (void)hipEventDestroy(e);
        for (auto e : c->stage_ev)
            if (e) (void)hipEventDestroy(e);
        for (void* b : c->stage_buf)
            if (b) (void)hipHostFree(b);
        if (c->stream) (void)hipStreamDestroy(c->stream);
    } catch (...) {
    }
    delete c;
}

VMX_API const char* volta_cuda_last_error(void* raw) {
    Context* c = static_cast<Context*>(raw);
    return c ? c->error.c_str() : "null context";
}

VMX_API int volta_cuda_set_resident_timing_policy(void* raw, int policy) {
    Context* c = static_cast<Context*>(raw);
    if (!c) return -1;
    if (c->record_active || c->coarse_active || c->counter_active || c->ring_pending || c->counter_pending)
        return reject(c, "cannot change resident timing policy after work has started");
    if (policy == 0) {
        if (c->timing_mode == TIMING_EVENTS) c->timing_mode = TIMING_EVENTS_DEFERRED;
    } else if (policy == 1) {
        c->timing_mode = TIMING_WALL_ONLY_COUNTERS;
    } else {
        return reject(c, "unknown resident timing policy");
    }
    // The construction-time event probe is outside every measurement window.
    c->stats.timing_elapsed_query_attempts = 0;
    c->stats.timing_elapsed_no_write = 0;
    c->stats.timing_event_queries = 0;
    c->stats.timing_event_api_calls = 0;
    c->stats.timing_mode = c->timing_mode;
    return 0;
}

VMX_API int volta_cuda_test_inject_elapsed_no_write_once(void* raw) {
    Context* c = static_cast<Context*>(raw);
    if (!c) return -1;
    if (c->record_active) return reject(c, "cannot inject elapsed no-write during an active record");
    c->inject_no_write = 1;
    return 0;
}

static bool resident_observation(Context* c) {
    return c->timing_mode == TIMING_EVENTS_DEFERRED || c->timing_mode == TIMING_WALL_ONLY_COUNTERS;
}

VMX_API int volta_cuda_begin_coarse_timing(void* raw, int op) {
    Context* c = static_cast<Context*>(raw);
    if (!c) return -1;
    if (!resident_observation(c)) return reject(c, "coarse timing requires a resident observation mode");
    if (c->poisoned) return reject(c, "measurement timing is poisoned; reset stats before continuing");
    if (op < 0 || op >= OP_COUNT) return reject(c, "invalid coarse timing operation");
    if (c->coarse_active || c->record_active || c->counter_active) return reject(c, "nested coarse timing scope");
    if (c->timing_mode == TIMING_EVENTS_DEFERRED) {
        size_t slot = 0;
        if (ring_take(c, &slot)) return -1;
        c->coarse_slot = slot;
        VMX_HIP(c, ev_record(c, c->ring[slot].ev[0]));
        c->ring[slot].mask |= 1;
        c->ring[slot].coarse = true;
        c->ring[slot].op = op;
    }
    c->coarse_op = op;
    c->coarse_active = true;
    c->coarse_inner = false;
    c->coarse_accounted = false;
    return 0;
}

VMX_API int volta_cuda_end_coarse_timing(void* raw) {
    Context* c = static_cast<Context*>(raw);
    if (!c) return -1;
    if (!resident_observation(c)) return reject(c, "coarse timing requires a resident observation mode");
    if (!c->coarse_active) return reject(c, "no active coarse timing scope");
    if (c->coarse_inner) return reject(c, "cannot end coarse timing during an active primitive");
    if (c->timing_mode == TIMING_EVENTS_DEFERRED) {
        TimingRecord& r = c->ring[c->coarse_slot];
        VMX_HIP(c, ev_record(c, r.ev[1]));
        r.mask |= 2;
        c->active_slot = c->coarse_slot;
        ring_commit(c);
    }
    c->coarse_active = false;
    c->coarse_op = -1;
    c->coarse_accounted = false;
    ++c->stats.coarse_timing_scopes;
    return 0;
}

VMX_API int volta_cuda_abort_coarse_timing(void* raw) {
    Context* c = static_cast<Context*>(raw);
    if (!c) return -1;
    if (!resident_observation(c)) return reject(c, "coarse timing requires a resident observation mode");
    if (c->coarse_active) abort_record(c);
    return 0;
}

VMX_API int volta_cuda_ensure_timing_capacity(void* raw, size_t bound, size_t* before, size_t* after,
                                                 int* flushed) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !before || !after || !flushed) return reject(c, "invalid timing-capacity output");
    if (!resident_observation(c))
        return reject(c, "timing-capacity preflight requires a resident observation mode");
    if (c->record_active || c->counter_active)
        return reject(c, "cannot preflight timing capacity during an active record");
    if (bound > TIMING_RING_SIZE) return reject(c, "deferred timing cohort bound exceeds ring capacity");
    *flushed = 0;
    *before = c->timing_mode == TIMING_EVENTS_DEFERRED ? c->ring_pending : 0;
    if (c->timing_mode == TIMING_WALL_ONLY_COUNTERS) {
        *after = 0;
        return 0;
    }
    if (c->ring_pending > TIMING_RING_SIZE - bound) {
        if (flush_deferred(c, SyncReason::TimingFlush)) return -1;
        *flushed = 1;
    }
    *after = c->ring_pending;
    return 0;
}

VMX_API int volta_cuda_flush_profiling(void* raw) {
    Context* c = static_cast<Context*>(raw);
    if (!c) return -1;
    if (c->poisoned) return reject(c, "measurement timing is poisoned; reset stats before reading it");
    if (c->record_active || c->counter_active) return reject(c, "cannot flush an active timing record");
    if (c->timing_mode == TIMING_WALL_ONLY_COUNTERS && c->counter_pending)
        return sync_stream(c, SyncReason::TimingFlush);
    return flush_deferred(c, SyncReason::TimingFlush);
}

VMX_API int volta_cuda_reset_stats(void* raw) {
    Context* c = static_cast<Context*>(raw);
    if (!c) return -1;
    if (c->record_active || c->counter_active) return reject(c, "cannot reset stats during an active timing record");
    VMX_GUARD_BEGIN
    // Pending work finishes before its counters are discarded.
    if (c->ring_pending || c->counter_pending || c->poisoned || c->outstanding) {
        if (sync_stream(c, SyncReason::TimingFlush)) return -1;
    }
    c->ring_begin = 0;
    c->ring_pending = 0;
    stream_touched(c);  // no record is left to lend its marker
    const uint64_t live = c->stats.live_device_bytes;
    const uint64_t live_pinned = c->stats.live_pinned_bytes;
    c->stats = RawStats{};
    c->stats.live_device_bytes = live;
    c->stats.peak_device_bytes = live;
    c->stats.live_pinned_bytes = live_pinned;
    c->stats.peak_pinned_bytes = live_pinned;
    c->stats.timing_mode = c->timing_mode;
    c->poisoned = false;
    c->coarse_accounted = false;
    c->counter_pending = false;
    return 0;
    VMX_GUARD_END(c, "stats reset")
}

VMX_API int volta_cuda_get_stats(void* raw, RawStats* out) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !out) return -1;
    if (c->poisoned) return reject(c, "measurement timing is poisoned; reset stats before reading it");
    if (c->record_active || c->counter_active) return reject(c, "cannot read stats during an active timing record");
    if (volta_cuda_flush_profiling(raw)) return -1;
    const RawStats& s = c->stats;
    if (s.sync_host_output + s.sync_upload_lifetime + s.sync_timing_flush + s.sync_profiling_legacy +
            s.sync_allocator_flush !=
        s.synchronizations)
        return fail_msg(c, "synchronization reason accounting mismatch");
    if (s.timing_elapsed_query_attempts != s.timing_event_queries + s.timing_elapsed_no_write)
        return fail_msg(c, "elapsed timing query accounting mismatch");
    if (c->timing_mode == TIMING_WALL_ONLY_COUNTERS) {
        uint64_t k = 0;
        for (auto v : s.kernel_ns) k += v;
        if (s.timing_records || s.timing_elapsed_query_attempts || s.timing_event_api_calls || s.h2d_ns ||
            s.d2h_ns || s.coarse_timing_ns || k)
            return fail_msg(c, "wall-only counter mode emitted event attribution");
    }
    *out = s;
    return 0;
}

VMX_API int volta_cuda_memory_breakdown(void* raw, uint64_t* workspace, uint64_t* resident,
                                           uint64_t* cached) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !workspace || !resident || !cached) return fail_msg(c, "invalid memory-breakdown output");
    uint64_t w = 0, r = 0, k = 0;
    for (const auto& b : c->ws) w += b.capacity;
    for (const auto& kv : c->twiddles) {
        const size_t half = std::max<size_t>(kv.first / 2, 1) * sizeof(uint64_t);
        if (kv.second.fwd) w += half;
        if (kv.second.inv) w += half;
        w += kv.second.grid_bytes + kv.second.split_bytes + kv.second.reg_bytes + kv.second.col_bytes;
    }
    for (const auto& b : c->resident) {
        if (!b.ptr) continue;
        (b.active ? r : k) += b.capacity;
    }
    if (w + r + k != c->stats.live_device_bytes) return fail_msg(c, "device-memory accounting mismatch");
    *workspace = w;
    *resident = r;
    *cached = k;
    return 0;
}

VMX_API int volta_cuda_trim_resident_cache(void* raw) {
    Context* c = static_cast<Context*>(raw);
    if (!c) return fail_msg(c, "invalid resident-cache trim context");
    if (c->coarse_active) return reject(c, "resident-cache trim is forbidden inside a coarse timing scope");
    VMX_GUARD_BEGIN
    return trim_resident(c);
    VMX_GUARD_END(c, "resident-cache trim")
}

VMX_API int volta_cuda_resident_alloc(void* raw, size_t bytes, uint64_t* out_id) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !bytes || !out_id) return fail_msg(c, "invalid resident allocation");
    if (c->coarse_active) return reject(c, "resident allocation is forbidden inside a coarse timing scope");
    VMX_GUARD_BEGIN
    ++c->stats.resident_alloc_requests;
    // Best fit among freed slots that still hold storage.
    size_t best = SIZE_MAX;
    size_t best_pos = SIZE_MAX;
    for (size_t i = 0; i < c->free_slots.size(); ++i) {
        const Resident& r = c->resident[c->free_slots[i]];
        if (r.ptr && r.capacity >= bytes && r.generation != UINT32_MAX &&
            (best == SIZE_MAX || r.capacity < c->resident[best].capacity)) {
            best = c->free_slots[i];
            best_pos = i;
        }
    }
    if (best != SIZE_MAX) {
        Resident& r = c->resident[best];
        c->free_slots.erase(c->free_slots.begin() + static_cast<ptrdiff_t>(best_pos));
        ++r.generation;
        r.logical = bytes;
        r.active = true;
        r.exposed = false;   // a new allocation: nothing is known of its contents
        r.msg_rows = false;
        ++c->stats.resident_reuse_hits;
        *out_id = make_id(best, r.generation);
        return 0;
    }
    void* ptr = nullptr;
    hipError_t e = hipMalloc(&ptr, bytes);
    if (e == hipErrorOutOfMemory) {
        (void)hipGetLastError();
        if (trim_resident(c)) return -1;
        e = hipMalloc(&ptr, bytes);
    }
    if (e != hipSuccess) return fail_hip(c, "hipMalloc(resident)", e);
    ++c->stats.allocation_calls;
    c->stats.live_device_bytes += bytes;
    c->stats.peak_device_bytes = std::max(c->stats.peak_device_bytes, c->stats.live_device_bytes);
    // Reuse an empty slot (no storage) if one exists, else append.
    size_t slot = SIZE_MAX;
    for (size_t i = 0; i < c->free_slots.size(); ++i) {
        const Resident& r = c->resident[c->free_slots[i]];
        if (!r.ptr && r.generation != UINT32_MAX) {
            slot = c->free_slots[i];
            c->free_slots.erase(c->free_slots.begin() + static_cast<ptrdiff_t>(i));
            break;
        }
    }
    if (slot == SIZE_MAX) {
        if (c->resident.size() >= 0xFFFFFFFEull) {
            (void)hipFree(ptr);
            ++c->stats.physical_free_calls;
            c->stats.live_device_bytes -= bytes;
            return fail_msg(c, "resident slot space exhausted");
        }
        c->resident.emplace_back();
        slot = c->resident.size() - 1;
    }
    Resident& r = c->resident[slot];
    ++r.generation;
    r.ptr = ptr;
    r.capacity = bytes;
    r.logical = bytes;
    r.active = true;
    r.exposed = false;
    r.msg_rows = false;
    *out_id = make_id(slot, r.generation);
    return 0;
    VMX_GUARD_END(c, "resident allocation")
}

VMX_API int volta_cuda_resident_free(void* raw, uint64_t id) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !id) return fail_msg(c, "invalid resident free");
    if (c->coarse_active) return reject(c, "resident free is forbidden inside a coarse timing scope");
    VMX_GUARD_BEGIN
    ++c->stats.resident_free_requests;
    Resident* r = find_resident(c, id);
    if (!r) return fail_msg(c, "unknown or stale resident buffer id");
    // Freeing the buffer that holds deferred message rows discards them;
    // freeing one of their sources writes them first.
    if (c->has_pending) {
        if (c->pending.out_id == id) c->has_pending = false;
        else if ((c->pending.w_id == id || (c->pending.pad && c->pending.pads_id == id)) && settle_pending(c))
            return -1;
    }
    // Storage stays cached for reuse; single-stream ordering makes a later
    // user of the same storage run after every earlier user.
    c->free_slots.push_back(static_cast<size_t>((id & 0xFFFFFFFFull) - 1));
    r->logical = 0;
    r->active = false;
    r->exposed = false;
    r->msg_rows = false;
    return 0;
    VMX_GUARD_END(c, "resident free")
}

VMX_API int volta_cuda_resident_upload(void* raw, uint64_t id, size_t off, const void* src, size_t bytes) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !src || !bytes) return fail_msg(c, "invalid resident upload");
    void* dst = nullptr;
    if (region(c, id, off, bytes, &dst)) return -1;
    if (begin_transfer(c)) return -1;
    const auto t0 = std::chrono::steady_clock::now();
    const int rc = staged_copy(c, dst, src, bytes, hipMemcpyHostToDevice);
    const auto t1 = std::chrono::steady_clock::now();
    if (rc) return -1;
    ++c->stats.resident_h2d_host_calls;
    c->stats.resident_h2d_host_call_ns += std::chrono::duration_cast<std::chrono::nanoseconds>(t1 - t0).count();
    return finish_transfer(c, bytes, true);
}

VMX_API int volta_cuda_resident_download(void* raw, uint64_t id, size_t off, void* dst, size_t bytes) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !dst || !bytes) return fail_msg(c, "invalid resident download");
    void* src = nullptr;
    if (region(c, id, off, bytes, &src, true)) return -1;
    if (begin_transfer(c)) return -1;
    const auto t0 = std::chrono::steady_clock::now();
    const int rc = staged_copy(c, dst, src, bytes, hipMemcpyDeviceToHost);
    const auto t1 = std::chrono::steady_clock::now();
    if (rc) return -1;
    ++c->stats.resident_d2h_host_calls;
    c->stats.resident_d2h_host_call_ns += std::chrono::duration_cast<std::chrono::nanoseconds>(t1 - t0).count();
    return finish_transfer(c, bytes, false);
}

// Device-side zero fill (a plain kernel rather than a memset node, so a
// caller may capture it in a graph).
__global__ void vmx_zero_kernel(uint4* dst, size_t n16, unsigned char* tail, size_t tail_bytes) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += stride)
        dst[i] = make_uint4(0, 0, 0, 0);
    if (blockIdx.x == 0)
        for (size_t i = threadIdx.x; i < tail_bytes; i += blockDim.x) tail[i] = 0;
}

namespace vmx {
// Zero `bytes` at `dst` on the context stream.
int zero_bytes(Context* c, void* dst, size_t bytes) {
    stream_touched(c);
    unsigned char* p = static_cast<unsigned char*>(dst);
    // Leading bytes until 16-byte alignment, handled with the tail path.
    size_t head = (16 - (reinterpret_cast<uintptr_t>(p) & 15)) & 15;
    head = std::min(head, bytes);
    if (head) {
        hipLaunchKernelGGL(vmx_zero_kernel, dim3(1), dim3(64), 0, c->stream, static_cast<uint4*>(nullptr),
                           size_t{0}, p, head);
        VMX_HIP(c, hipGetLastError());
    }
    p += head;
    bytes -= head;
    const size_t n16 = bytes / 16;
    const size_t tail = bytes - n16 * 16;
    if (n16 || tail) {
        const size_t blocks = std::min<size_t>((n16 + 255) / 256 + 1, 4096);
        hipLaunchKernelGGL(vmx_zero_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, c->stream,
                           reinterpret_cast<uint4*>(p), n16, p + n16 * 16, tail);
        VMX_HIP(c, hipGetLastError());
    }
    return 0;
}
}  // namespace vmx

VMX_API int volta_cuda_resident_zero(void* raw, uint64_t id, size_t off, size_t bytes) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !bytes) return fail_msg(c, "invalid resident zero");
    void* dst = nullptr;
    if (region(c, id, off, bytes, &dst)) return -1;
    if (begin_op(c) || mark_op(c, 1)) return -1;
    if (zero_bytes(c, dst, bytes)) return -1;
    if (mark_op(c, 2)) return -1;
    return finish_op(c, OP_PCS_ROWS, 0, 0, 0, bytes, 0);
}

static int copy_rows_impl(Context* c, uint64_t src_id, size_t src_off, size_t src_stride, uint64_t dst_id,
                          size_t dst_off, size_t dst_stride, size_t rows, size_t row_bytes, int op) {
    if (!c) return -1;
    void *src = nullptr, *dst = nullptr;
    size_t src_span = 0, dst_span = 0;
    if (strided_region(c, src_id, src_off, src_stride, row_bytes, rows, &src, &src_span, true) ||
        strided_region(c, dst_id, dst_off, dst_stride, row_bytes, rows, &dst, &dst_span))
        return -1;
    if (src_id == dst_id) {
        size_t se = 0, de = 0;
        if (!add_ok(src_off, src_span, &se) || !add_ok(dst_off, dst_span, &de))
            return fail_msg(c, "resident D2D copy envelope overflows size_t");
        if (src_off < de && dst_off < se) return fail_msg(c, "resident D2D copy source and destination overlap");
    }
    size_t total = 0;
    if (!mul_ok(rows, row_bytes, &total)) return fail_msg(c, "resident D2D byte count overflows size_t");
    if (begin_op(c) || mark_op(c, 1)) return -1;
    VMX_HIP(c, hipMemcpy2DAsync(dst, dst_stride, src, src_stride, row_bytes, rows, hipMemcpyDeviceToDevice,
                                c->stream));
    if (mark_op(c, 2)) return -1;
    return finish_op(c, op, 0, 0, total, 0, 0);
}

VMX_API int volta_cuda_resident_copy_rows(void* raw, uint64_t src_id, size_t src_off, size_t src_stride,
                                             uint64_t dst_id, size_t dst_off, size_t dst_stride, size_t rows,
                                             size_t row_bytes) {
    return copy_rows_impl(static_cast<Context*>(raw), src_id, src_off, src_stride, dst_id, dst_off, dst_stride,
                          rows, row_bytes, OP_PCS_ROWS);
}

VMX_API int volta_cuda_resident_mailbox_copy_rows(void* raw, uint64_t src_id, size_t src_off,
                                                     size_t src_stride, uint64_t dst_id, size_t dst_off,
                                                     size_t dst_stride, size_t rows, size_t row_bytes) {
    return copy_rows_impl(static_cast<Context*>(raw), src_id, src_off, src_stride, dst_id, dst_off, dst_stride,
                          rows, row_bytes, OP_MAILBOX);
}

// ---- pinned host pool -------------------------------------------------------------

VMX_API int volta_cuda_pinned_alloc(void* raw, size_t bytes, uint64_t* out_id) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !bytes || !out_id) return fail_msg(c, "invalid pinned allocation");
    if (c->coarse_active) return reject(c, "pinned allocation is forbidden inside a coarse timing scope");
    VMX_GUARD_BEGIN
    ++c->stats.pinned_alloc_requests;
    size_t best = SIZE_MAX, best_pos = SIZE_MAX;
    for (size_t i = 0; i < c->free_pinned.size(); ++i) {
        const Pinned& p = c->pinned[c->free_pinned[i]];
        if (p.ptr && p.capacity >= bytes && p.generation != UINT32_MAX &&
            (best == SIZE_MAX || p.capacity < c->pinned[best].capacity)) {
            best = c->free_pinned[i];
            best_pos = i;
        }
    }
    if (best != SIZE_MAX) {
        Pinned& p = c->pinned[best];
        c->free_pinned.erase(c->free_pinned.begin() + static_cast<ptrdiff_t>(best_pos));
        ++p.generation;
        p.logical = bytes;
        p.active = true;
        ++c->stats.pinned_reuse_hits;
        *out_id = make_id(best, p.generation);
        return 0;
    }
    void* ptr = nullptr;
    hipEvent_t ready = nullptr;
    VMX_HIP(c, hipEventCreateWithFlags(&ready, hipEventDisableTiming));
    const hipError_t e = hipHostMalloc(&ptr, bytes, hipHostMallocDefault);
    if (e != hipSuccess) {
        (void)hipEventDestroy(ready);
        return fail_hip(c, "hipHostMalloc(pinned)", e);
    }
    ++c->stats.pinned_allocation_calls;
    c->stats.live_pinned_bytes += bytes;
    c->stats.peak_pinned_bytes = std::max(c->stats.peak_pinned_bytes, c->stats.live_pinned_bytes);
    c->pinned.emplace_back();
    const size_t slot = c->pinned.size() - 1;
    Pinned& p = c->pinned[slot];
    p.ptr = ptr;
    p.ready = ready;
    p.capacity = bytes;
    p.logical = bytes;
    p.generation = 1;
    p.active = true;
    *out_id = make_id(slot, p.generation);
    return 0;
    VMX_GUARD_END(c, "pinned allocation")
}

VMX_API int volta_cuda_pinned_write(void* raw, uint64_t id, size_t off, const void* src, size_t bytes) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !src || !bytes) return fail_msg(c, "invalid pinned write");
    Pinned* p = find_pinned(c, id);
    if (!p) return fail_msg(c, "unknown or stale pinned buffer id");
    if (off > p->logical || bytes > p->logical - off) return fail_msg(c, "pinned buffer region is out of bounds");
    if (p->in_flight && p->ready) {
        VMX_HIP(c, hipEventSynchronize(p->ready));
        p->in_flight = false;
    }
    std::memcpy(static_cast<unsigned char*>(p->ptr) + off, src, bytes);
    ++c->stats.pinned_host_write_calls;
    c->stats.pinned_host_write_bytes += bytes;
    return 0;
}

VMX_API int volta_cuda_pinned_wait_ready(void* raw, uint64_t id) {
    Context* c = static_cast<Context*>(raw);
    if (!c) return -1;
    Pinned* p = find_pinned(c, id);
    if (!p) return fail_msg(c, "unknown or stale pinned buffer id");
    if (p->in_flight && p->ready) VMX_HIP(c, hipEventSynchronize(p->ready));
    p->in_flight = false;
    return 0;
}

VMX_API int volta_cuda_pinned_free(void* raw, uint64_t id) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !id) return fail_msg(c, "invalid pinned free");
    if (c->coarse_active) return reject(c, "pinned free is forbidden inside a coarse timing scope");
    VMX_GUARD_BEGIN
    Pinned* p = find_pinned(c, id);
    if (!p) return fail_msg(c, "unknown or stale pinned buffer id");
    ++c->stats.pinned_free_requests;
    c->free_pinned.push_back(static_cast<size_t>((id & 0xFFFFFFFFull) - 1));
    p->logical = 0;
    p->active = false;
    return 0;
    VMX_GUARD_END(c, "pinned free")
}

VMX_API int volta_cuda_trim_pinned_cache(void* raw) {
    Context* c = static_cast<Context*>(raw);
    if (!c) return fail_msg(c, "invalid pinned-cache trim context");
    if (c->coarse_active) return reject(c, "pinned-cache trim is forbidden inside a coarse timing scope");
    VMX_GUARD_BEGIN
    return trim_pinned(c);
    VMX_GUARD_END(c, "pinned-cache trim")
}

VMX_API int volta_cuda_pinned_memory_stats(void* raw, RawPinnedMemoryStats* out) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !out) return fail_msg(c, "invalid pinned-memory stats output");
    RawPinnedMemoryStats r{};
    for (const auto& p : c->pinned) {
        if (!p.ptr) continue;
        if (p.active) {
            r.active_bytes += p.capacity;
            ++r.active_allocations;
        } else {
            r.cached_bytes += p.capacity;
            ++r.cached_allocations;
        }
        if (p.in_flight) ++r.in_flight_allocations;
    }
    if (r.active_bytes + r.cached_bytes != c->stats.live_pinned_bytes)
        return fail_msg(c, "pinned-memory accounting mismatch");
    r.physical_allocation_calls = c->stats.pinned_allocation_calls;
    r.allocation_requests = c->stats.pinned_alloc_requests;
    r.reuse_hits = c->stats.pinned_reuse_hits;
    r.free_requests = c->stats.pinned_free_requests;
    r.physical_free_calls = c->stats.pinned_physical_free_calls;
    r.host_write_calls = c->stats.pinned_host_write_calls;
    r.host_write_bytes = c->stats.pinned_host_write_bytes;
    r.peak_bytes = c->stats.peak_pinned_bytes;
    *out = r;
    return 0;
}

VMX_API int volta_cuda_x4c_control_state(void* raw, RawX4cControlState* out) {
    Context* c = static_cast<Context*>(raw);
    if (!c || !out) return fail_msg(c, "invalid control-state output");
    ++c->stats.x4c_control_peek_calls;
    const hipError_t q = hipStreamQuery(c->stream);
    uint32_t state = 0;
    if (q == hipSuccess) {
        c->outstanding = 0;
        c->counter_pending = false;
        for (auto& p : c->pinned) p.in_flight = false;
    } else if (q == hipErrorNotReady) {
        state = 1;
        ++c->stats.x4c_control_peek_pending;
    } else {
        return fail_hip(c, "hipStreamQuery(control state)", q);
    }
    RawX4cControlState r{};
    r.stream_state = state;
    r.flags = (c->coarse_active ? 1u : 0u) | ((c->record_active || c->counter_active) ? 2u : 0u) |
              (c->poisoned ? 4u : 0u);
    r.outstanding_cuda_operations = c->outstanding;
    r.pending_timing_records = c->ring_pending;
    for (const auto& b : c->ws) r.workspace_device_bytes += b.capacity;
    for (const auto& kv : c->twiddles) {
        const size_t half = std::max<size_t>(kv.first / 2, 1) * sizeof(uint64_t);
        if (kv.second.fwd) r.workspace_device_bytes += half;
        if (kv.second.inv) r.workspace_device_bytes += half;
        r.workspace_device_bytes +=
            kv.second.grid_bytes + kv.second.split_bytes + kv.second.reg_bytes + kv.second.col_bytes;
    }
    for (const auto& b : c->resident) {
        if (!b.ptr) continue;
        if (b.active) {
            ++r.active_device_allocations;
            r.active_device_bytes += b.capacity;
        } else {
            ++r.cached_device_allocations;
            r.cached_device_bytes += b.capacity;
        }
    }
    for (const auto& p : c->pinned) {
        if (!p.ptr) continue;
        if (p.active) {
            ++r.active_pinned_allocations;
            r.active_pinned_bytes += p.capacity;
        } else {
            ++r.cached_pinned_allocations;
            r.cached_pinned_bytes += p.capacity;
        }
        if (p.in_flight) ++r.in_flight_pinned_allocations;
    }
    *out = r;
    return 0;
}
