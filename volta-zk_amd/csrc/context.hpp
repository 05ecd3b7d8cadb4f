// context.hpp -- per-context state behind the volta_cuda_* C ABI (ABI 37).
//
// One context = one HIP stream on the current device, a generational-id
// resident allocator with best-fit reuse of freed storage, a handful of
// grow-only workspaces for the host-pointer entry points, a per-size twiddle
// cache, and RawStats accounting/timing.  The observable contract follows the
// reference backend (cuda/volta_cuda_backend.cu:55-123 RawStats layout,
// :174-310 ids and buffers, :1035-1262 timing, :3150-3560 control exports).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <array>
#include <chrono>
#include <cstddef>
#include <map>
#include <string>
#include <vector>

// Exported C entry point (the library is built with hidden visibility).
#define VMX_API extern "C" __attribute__((visibility("default")))

namespace vmx {

constexpr uint32_t ABI_VERSION = 37;
constexpr int OP_COUNT = 7;
constexpr int OP_GEMM = 0;
constexpr int OP_LOGUP = 1;
constexpr int OP_PCS_ROWS = 2;
constexpr int OP_PCS_NTT = 3;
constexpr int OP_PCS_MERKLE = 4;
constexpr int OP_AUTH_MASKS = 5;
constexpr int OP_MAILBOX = 6;

// Timing modes reported in RawStats::timing_mode (reference .cu:42-46).
constexpr uint32_t TIMING_EVENTS = 1;           // per-primitive events, read at once
constexpr uint32_t TIMING_HOST_BARRIER_WALL = 2; // events unusable: host barriers
constexpr uint32_t TIMING_EVENTS_DEFERRED = 3;  // events resolved lazily from a ring
constexpr uint32_t TIMING_WALL_ONLY_COUNTERS = 4; // counters only, no events
constexpr size_t TIMING_RING_SIZE = 512;

// Exact field order of the reference's RawStats (504 bytes).
struct RawStats {
    uint64_t calls[OP_COUNT];
    uint64_t kernel_ns[OP_COUNT];
    uint64_t h2d_bytes;
    uint64_t d2h_bytes;
    uint64_t d2d_bytes;
    uint64_t device_zeroed_bytes;
    uint64_t device_generated_bytes;
    uint64_t h2d_ns;
    uint64_t d2h_ns;
    uint64_t resident_h2d_host_calls;
    uint64_t resident_d2h_host_calls;
    uint64_t resident_h2d_host_call_ns;
    uint64_t resident_d2h_host_call_ns;
    uint64_t synchronizations;
    uint64_t synchronization_ns;
    uint64_t sync_host_output;
    uint64_t sync_upload_lifetime;
    uint64_t sync_timing_flush;
    uint64_t sync_profiling_legacy;
    uint64_t sync_allocator_flush;
    uint64_t allocation_calls;
    uint64_t resident_alloc_requests;
    uint64_t resident_reuse_hits;
    uint64_t resident_free_requests;
    uint64_t physical_free_calls;
    uint64_t live_device_bytes;
    uint64_t peak_device_bytes;
    uint64_t pinned_allocation_calls;
    uint64_t pinned_alloc_requests;
    uint64_t pinned_reuse_hits;
    uint64_t pinned_free_requests;
    uint64_t pinned_physical_free_calls;
    uint64_t pinned_host_write_calls;
    uint64_t pinned_host_write_bytes;
    uint64_t live_pinned_bytes;
    uint64_t peak_pinned_bytes;
    uint64_t x4c_arena_reset_calls;
    uint64_t x4c_arena_reset_bytes;
    uint64_t x4c_kernel_launches;
    uint64_t x4c_control_peek_calls;
    uint64_t x4c_control_peek_pending;
    uint64_t timing_records;
    uint64_t timing_elapsed_query_attempts;
    uint64_t timing_elapsed_no_write;
    uint64_t timing_event_queries;
    uint64_t timing_event_api_calls;
    uint64_t timing_pending_high_water;
    uint64_t timing_flush_count;
    uint64_t coarse_timing_scopes;
    uint64_t coarse_timing_ns;
    uint32_t timing_mode;
    uint32_t reserved;
};
static_assert(sizeof(RawStats) == 504, "RawStats must keep the reference's 504-byte layout");

struct RawPinnedMemoryStats {
    uint64_t active_bytes;
    uint64_t cached_bytes;
    uint64_t active_allocations;
    uint64_t cached_allocations;
    uint64_t in_flight_allocations;
    uint64_t physical_allocation_calls;
    uint64_t allocation_requests;
    uint64_t reuse_hits;
    uint64_t free_requests;
    uint64_t physical_free_calls;
    uint64_t host_write_calls;
    uint64_t host_write_bytes;
    uint64_t peak_bytes;
};
static_assert(sizeof(RawPinnedMemoryStats) == 104, "pinned stats layout");

struct RawX4cControlState {
    uint32_t stream_state;
    uint32_t flags;
    uint64_t outstanding_cuda_operations;
    uint64_t pending_timing_records;
    uint64_t active_device_allocations;
    uint64_t cached_device_allocations;
    uint64_t active_pinned_allocations;
    uint64_t cached_pinned_allocations;
    uint64_t in_flight_pinned_allocations;
    uint64_t workspace_device_bytes;
    uint64_t active_device_bytes;
    uint64_t cached_device_bytes;
    uint64_t active_pinned_bytes;
    uint64_t cached_pinned_bytes;
};
static_assert(sizeof(RawX4cControlState) == 104, "control-state layout");

enum class SyncReason { HostOutput, UploadLifetime, TimingFlush, ProfilingLegacy, AllocatorFlush };

// Resident storage addressed by id = (generation << 32) | (slot + 1).
struct Resident {
    void* ptr = nullptr;
    size_t capacity = 0;
    size_t logical = 0;
    uint32_t generation = 0;
    bool active = false;
    // Its device address was handed to the caller (volta_mi355x_resident_device_ptr):
    // the caller's own kernels may read or write it outside the library, so no
    // deferred message rows involve it.
    bool exposed = false;
    // Message rows lift(w) || pads || 0 that the library itself wrote here
    // (rows of row_len elements from element off, zero from element nonzero
    // on in each row), kept until anything other than a read touches the
    // buffer: a forward NTT of exactly those rows then reads only the nonzero
    // part.
    bool msg_rows = false;
    size_t msg_off = 0, msg_count = 0, msg_row_len = 0, msg_nonzero = 0;
};

struct Pinned {
    void* ptr = nullptr;
    size_t capacity = 0;
    size_t logical = 0;
    hipEvent_t ready = nullptr;
    uint32_t generation = 0;
    bool active = false;
    bool in_flight = false;
};

struct Workspace {
    void* ptr = nullptr;
    size_t capacity = 0;
};

// Workspace slots used by host-pointer entry points and internal scratch.
enum WorkspaceSlot : int {
    WS_IN = 0,
    WS_OUT = 1,
    WS_AUX0 = 2,
    WS_AUX1 = 3,
    WS_PARTIALS = 4,  // combination partial sums
    WS_AUX2 = 5,      // combination coefficient sums
    WS_HASH = 6,      // Merkle column-group chaining values
    WS_COUNT = 7,
};

struct TimingRecord {
    hipEvent_t ev[4]{};
    // marker 1 borrowed from the previous record's marker 2 (null: ev[1])
    hipEvent_t start = nullptr;
    int op = -1;
    uint8_t mask = 0;  // which of ev[] were recorded (bit 1 also when marker 1 is borrowed)
    bool coarse = false;
    bool transfer_h2d = false;
    bool transfer_d2h = false;
    uint64_t h2d = 0, d2h = 0, d2d = 0, zeroed = 0, generated = 0;
};

// Device twiddle tables for one transform size n (all tables are uploaded once
// and cached for the life of the context).
struct TwiddleSet {
    uint64_t* fwd = nullptr;  // w^0 .. w^(n/2-1), the reference's table
    uint64_t* inv = nullptr;  // w^0 .. w^-(n/2-1) (inverse transform only)
    uint64_t* grid = nullptr; // w^(i2*j1) laid out for the fast encode (device-built)
    size_t grid_bytes = 0;
    // Two-level table of w^e for any e < n: lo[j] = w^j (j < 2^h), then
    // hi[j] = w^(j 2^h) (j < n / 2^h), h = ceil(log2 n / 2); w^e = lo[e & (2^h-1)] hi[e >> h].
    uint64_t* split = nullptr;
    size_t split_bytes = 0;
    int split_h = 0;
    // The pass engine's tables (n >= 2^13), derived on the device from fwd:
    // [w_4096^j, j < 2048][two-level table of w with h = reg_h].
    uint64_t* reg = nullptr;
    size_t reg_bytes = 0;
    int reg_h = 0;
    // Pre-twiddles of the pass engine's column passes whose columns span n
    // points (derived on the device): col[rb][i 2^(log2 n - rb) + l] = w^(i l),
    // i < 2^rb.  col_bytes sums them.
    uint64_t* col[16] = {};
    // The same tables times n^-1 (n = their span), for the last pass of a
    // batched inverse transform; col_bytes counts them too.
    uint64_t* col_scaled[16] = {};
    size_t col_bytes = 0;
    size_t n = 0;
};

// Message rows msg = lift(w) || pads || 0 that volta_cuda_pcs_messages_device
// recorded but has not written yet (the out region holds them virtually).
// They are written by settle_pending before any other access to any resident
// buffer, unless the next access is a forward NTT of exactly that region,
// which encodes straight from the sources instead.
struct PendingMessages {
    uint64_t out_id = 0;
    size_t out_off = 0;  // elements
    uint64_t* out = nullptr;
    uint64_t w_id = 0, pads_id = 0;
    const int16_t* w = nullptr;
    const uint64_t* pads = nullptr;
    size_t rows = 0, cols = 0, pad = 0, code_len = 0;
};

struct Context {
    int device = 0;
    int cu_count = 0;  // compute units of `device` (sizes persistent grids)
    hipStream_t stream = nullptr;
    hipEvent_t events[4]{};
    std::vector<Resident> resident;
    std::vector<size_t> free_slots;  // inactive slots (may hold storage)
    std::vector<Pinned> pinned;
    std::vector<size_t> free_pinned;
    Workspace ws[WS_COUNT];
    std::map<size_t, TwiddleSet> twiddles;
    RawStats stats{};
    uint32_t timing_mode = TIMING_EVENTS;
    // deferred ring
    std::array<TimingRecord, TIMING_RING_SIZE> ring{};
    size_t ring_begin = 0;
    size_t ring_pending = 0;
    bool record_active = false;  // a ring/legacy record is between begin and finish
    size_t active_slot = 0;
    // The ring slot whose marker 2 is the last thing enqueued on the stream
    // (-1: none, or other work followed it); the next device-only record may
    // open with that marker instead of recording its own.
    long reuse_slot = -1;
    // coarse scopes
    bool coarse_active = false;
    bool coarse_inner = false;
    bool coarse_accounted = false;
    bool poisoned = false;
    int coarse_op = -1;
    size_t coarse_slot = 0;
    // counters-only
    bool counter_active = false;
    // set while a record that adds kernel time without a call is finished
    // (the late write of deferred message rows)
    bool uncounted = false;
    bool counter_pending = false;
    uint64_t outstanding = 0;
    std::chrono::steady_clock::time_point phase_start{};
    uint64_t phase_ns[3]{};
    uint32_t inject_no_write = 0;
    // this device's address of the allocation-free combination's scratch
    // array (null when it could not be resolved)
    void* scratch = nullptr;
    std::string scratch_error;
    // at most one deferred message-row record; `bypass_settle` lets the NTT
    // that consumes it resolve its regions without writing it
    bool has_pending = false;
    PendingMessages pending{};
    bool bypass_settle = false;
    // Pinned staging of the host-pointer transforms' large copies
    // (staged_copy): one buffer and one event per copy thread, allocated on
    // first use and kept for the context's life.
    std::array<void*, 8> stage_buf{};
    std::array<hipEvent_t, 8> stage_ev{};
    bool stage_ready = false;
    std::string error;
};

// ---- error helpers (never throw across the ABI) -----------------------------
int fail_msg(Context* c, const char* msg) noexcept;
int fail_hip(Context* c, const char* what, hipError_t e) noexcept;
int reject(Context* c, const char* msg) noexcept;

#define VMX_HIP(c, call)                                              \
    do {                                                              \
        hipError_t vmx_e_ = (call);                                   \
        if (vmx_e_ != hipSuccess) return ::vmx::fail_hip((c), #call, vmx_e_); \
    } while (0)

// ---- geometry helpers -----------------------------------------------------------
bool mul_ok(size_t a, size_t b, size_t* out);
// a * b * c without overflow (every partial product checked).
bool mul3_ok(size_t a, size_t b, size_t c, size_t* out);
bool add_ok(size_t a, size_t b, size_t* out);
Resident* find_resident(Context* c, uint64_t id);
// Resolve a byte region of a resident buffer; fails if out of bounds.
// `read_only` marks a region the caller only reads: deferred message rows are
// written first only when their own buffer is read, while any other access
// to their buffer or to their sources writes them first.
int region(Context* c, uint64_t id, size_t offset_bytes, size_t bytes, void** out, bool read_only = false);
// Element-offset variant: offset and count in units of elem_bytes.
int region_elems(Context* c, uint64_t id, size_t offset, size_t count, size_t elem_bytes,
                 void** out, bool read_only = false);
int strided_region(Context* c, uint64_t id, size_t offset, size_t stride, size_t row_bytes,
                   size_t rows, void** out, size_t* span, bool read_only = false);

// Pinned host regions (byte offsets) and their transfer state: a pinned
// source stays "in flight" from the copy that reads it until its ready event
// completes (reference .cu:538-575).
int pinned_region(Context* c, uint64_t id, size_t offset_bytes, size_t bytes, void** out, Pinned** owner);
int pinned_ready(Context* c, Pinned* p, bool* ready);
int pinned_mark_in_flight(Context* c, Pinned* p);

// Writes the deferred message rows, if any (one launch on the context stream,
// outside any primitive's timing record).
int settle_pending(Context* c);
// Records that buffer `id` holds message rows the library wrote (Resident::msg_rows);
// nothing is recorded for a buffer whose address the caller holds.
void note_message_rows(Context* c, uint64_t id, size_t off, size_t rows, size_t row_len, size_t nonzero);

// ---- host <-> device copies of the host-pointer entry points ---------------------
// A copy of `bytes` between pageable host memory and the device, on the
// context's stream after the work queued before it; returns once the data is
// on the host (download) or queued for the device (upload: the source may be
// reused at once).  Copies of at least STAGE_MIN_BYTES of pageable host memory
// go through the pinned staging buffers; the rest, copies of host memory the
// caller pinned, and all copies if the buffers cannot be pinned are one
// hipMemcpyAsync.
constexpr size_t STAGE_SLOT_BYTES = size_t{16} << 20;
constexpr size_t STAGE_MIN_BYTES = size_t{32} << 20;
int staged_copy(Context* c, void* dst, const void* src, size_t bytes, hipMemcpyKind kind);

// ---- workspaces and twiddles ---------------------------------------------------
int ensure_ws(Context* c, int slot, size_t bytes);
template <typename T>
T* ws(Context* c, int slot) {
    return static_cast<T*>(c->ws[slot].ptr);
}
// Forward twiddles for size n; uploads n/2 u64 on first use and adds the
// bytes to *h2d (the reference's per-size upload, .cu:2675-2689).
int ensure_twiddles(Context* c, size_t n, uint64_t* h2d, TwiddleSet** out);
int ensure_inverse_twiddles(Context* c, size_t n, uint64_t* h2d, TwiddleSet** out);
// Derives TwiddleSet::reg from t->fwd on the device (ntt_reg.hip); a no-op
// when present.  ensure_twiddles calls it for every size the pass engine runs.
int derive_reg_tables(Context* c, TwiddleSet* t);
bool reg_ntt_covers(uint64_t n);
// Two-level table of w^e for size n (TwiddleSet::split), uploaded once.
int ensure_split_twiddles(Context* c, size_t n, uint64_t* h2d, TwiddleSet** out);
// Device-built table of `bytes` for the fast encode, derived from t->fwd on
// the device (no host upload).  `build` enqueues the kernel that fills it.
int ensure_grid_twiddles(Context* c, TwiddleSet* t, size_t bytes, int (*build)(Context*, TwiddleSet*));

// ---- timing/accounting (one primitive = begin, [mark1], [mark2], finish) ---------
int begin_op(Context* c);
// begin_op for a primitive that uploads host data before marker 1: its upload is timed.
int begin_op_h2d(Context* c);
int mark_op(Context* c, int which);
int finish_op(Context* c, int op, uint64_t h2d, uint64_t d2h, uint64_t d2d = 0,
              uint64_t zeroed = 0, uint64_t generated = 0);
int begin_transfer(Context* c);
int finish_transfer(Context* c, size_t bytes, bool h2d);
int sync_stream(Context* c, SyncReason reason);
int flush_deferred(Context* c, SyncReason reason);
// A primitive that enqueues nothing on the device: counted as a call, with no
// timing record (under deferred events) and so no markers on the stream.
int empty_op(Context* c, int op);
// Work enqueued on the stream outside a primitive's markers: the last record's
// closing marker can no longer open the next one.
inline void stream_touched(Context* c) { c->reuse_slot = -1; }

}  // namespace vmx
