// encode_fast.hip -- the Ligero RS-encode fast path for gfx950.
//
// Shape: codeword length n = 2^13, i16 message rows of cols <= 2^11 (rate
// <= 1/4: the GPT-2 weight commits, configurations c_attn and full GPT-2).
// Output is bit-identical to NttPlan::encode of lift(w) zero-padded
// (rust/volta-pcs/src/ntt.rs:36-70); the factorisation below is exact.
//
// Four-step split n = 128 x 64, input index i = 64*i1 + i2 (i1 < 128, and
// only i1 < 32 is non-zero), output index j = j1 + 128*j2:
//   phase A (wave S = outputs j1 in [32 S, 32 S + 32), all 64 columns):
//       X[j1][i2] = sum_{i1<32} x[64 i1 + i2] * w128^(i1 j1)
//     as an exact int8 matrix product on the matrix cores (enc13_mfma.hpp:
//     the inputs split into two signed bytes, the DFT matrix into balanced
//     base-256 digits, eight position sums folded to one field element), then
//       Y[j1][i2] = X[j1][i2] * w_n^(i2 j1)      (the only 64x64 products)
//   phase B (thread = row j1 x parity h, h alternating per row): the 64-point DFT over
//     i2 (w64 = 2^39) as its first radix-2 DIF stage followed by one 32-point
//     DFT per parity (w32 = 2^78: shifts only); X[2k + h] goes to
//     out[j1 + 128 (2k + h)], so each store instruction writes 64 consecutive u64.
// A persistent grid of 4-wave workgroups walks the rows; Y lives in LDS with a
// padded pitch.
// HBM traffic per row: 4 KiB of i16 read + 64 KiB of u64 written.
#include <hip/hip_runtime.h>

#include "context.hpp"
#include "enc13_mfma.hpp"
#include "enc13_phase_b.hpp"
#include "gl64.hpp"
#include "gl64_shift.hpp"
#include "kernels.hpp"
#include "ntt_rr.hpp"

namespace vmx {

namespace enc13 {

constexpr int LOG_N = 13;
constexpr int N = 1 << LOG_N;
constexpr int N1 = 128;    // j1 range
constexpr int N2 = 64;     // i2 range
constexpr int K = 32;      // non-zero i1 range (cols <= K * N2 = 2048)
constexpr int PITCH = 65;  // u64 per LDS row of Y
constexpr int THREADS = 256;
constexpr size_t LATE_ROWS = 8;  // rows per workgroup up to which phase B takes the late shifts
constexpr size_t LDS_BYTES = size_t{N1} * PITCH * sizeof(uint64_t);
constexpr size_t GRID_BYTES = size_t{N1} * N2 * sizeof(uint64_t);
// The twiddle grid, then phase A's A fragments, then its accumulator init
// words, then (256-byte aligned) the tables of the one-pass u64 transform
// (ntt_rr.hpp, n = 2^13).
constexpr size_t R13_OFF =
    (GRID_BYTES + enc13m::FRAG_BYTES + enc13m::INIT_WORDS * sizeof(int) + 255) & ~size_t{255};
constexpr size_t TABLE_BYTES = R13_OFF + size_t{rr::Shape<3>::TABLE_WORDS} * sizeof(uint64_t);

typedef int v4i __attribute__((ext_vector_type(4)));

// Phase B of one row: the 64-point DFT over i2 of Y's row j1 at output parity
// H, X[2k + H] stored to o[j1 + N1 (2k + H)].  Phase A stored the first
// radix-2 stage's sums S in columns 0..31 of the row and its differences D in
// columns 32..63.  The workgroup's second barrier sits between the LDS reads
// and the DFT: Y is rewritten by the next row's phase A, and once every wave
// holds its row's inputs in registers the workgroup may move on, so the DFTs
// and stores overlap the next phase A of faster waves.  Parity 1's 31 shifts
// (D[q] w64^q) come before the barrier (LATE = false), where the parity-0
// wave's wait is filled by the other workgroup's wave on its SIMD when
// workgroups walk many rows, or after it (LATE = true), so both parities reach
// the barrier together, which pays when each workgroup has only a few rows.
template <bool LATE>
__device__ __forceinline__ void phase_b(const uint64_t* Y, int j1, int H, uint64_t* o) {
    uint64_t v[K];
    if constexpr (LATE) {
        enc13m::phase_b_load<0>(Y + j1 * PITCH + 32 * H, v);
        __syncthreads();
        if (H != 0) enc13m::phase_b_twiddle(v);
    } else {
        if (H == 0) enc13m::phase_b_load<0>(Y + j1 * PITCH, v);
        else enc13m::phase_b_load<1>(Y + j1 * PITCH + 32, v);
        __syncthreads();
    }
    enc13m::phase_b_dft(v);
    o += j1 + N1 * H;
#pragma unroll
    for (int k = 0; k < 32; ++k) __builtin_nontemporal_store(v[k], o + N1 * 2 * k);
}

// The row's inputs as the matrix product's B operand: lane l, column tile t
// holds x[64 i1 + 16 t + (l & 15)] for i1 in [8 (l >> 4), 8 (l >> 4) + 8), two
// per word as the digit pairs x ^ 0x80 (low byte (x & 255) - 128, high byte
// x >> 8).  The raw buffer resource spans exactly the row's cols entries, so
// the tail reads as 0 (an out-of-range buffer load reads zero and touches no
// memory); all 32 loads share one offset register.
__device__ __forceinline__ void load_frags(const int16_t* wr, size_t cols, int lane, v4i* xf) {
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int16_t*>(wr), static_cast<short>(0), static_cast<int>(cols * sizeof(int16_t)), 0x00020000);
    const int off = static_cast<int>(sizeof(int16_t)) * (N2 * 8 * (lane >> 4) + (lane & 15));
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int e0 = N2 * (2 * q) + 16 * t, e1 = N2 * (2 * q + 1) + 16 * t;
            const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b16(rsrc, off + 2 * e0, 0, 0);
            const uint32_t hi = __builtin_amdgcn_raw_buffer_load_b16(rsrc, off + 2 * e1, 0, 0);
            xf[t][q] = static_cast<int>(((lo & 0xFFFFu) | (hi << 16)) ^ 0x00800080u);
        }
}

// One wave's share of every row its workgroup owns.  Wave S runs phase A for
// the output pairs q in [8 S, 8 S + 8) (j1 = 4 q + 0..3) of all 64 columns:
// its 16 A fragments (8 pairs x positions 0-3 and 4-7) stay in registers for
// the kernel's life, and each row takes 64 products.  It then runs phase B for
// rows j1 in [64 (S >> 1), 64 (S >> 1) + 64) and parity H, 1 - (S & 1) on the
// workgroup's first row and flipped on each row after it: parity 1's first
// stage costs about three times parity 0's, and a fixed parity per wave would
// give the same SIMDs the longer share on every row.  S and H are uniform, so
// no lane diverges.  The workgroup walks rows blockIdx.x,
// blockIdx.x + gridDim.x, ..., loading the next row's inputs before phase B of
// the current row.
template <bool LATE>
__device__ __forceinline__ void encode_rows(int S, const int16_t* __restrict__ w, size_t cols, size_t rows,
                                            const uint64_t* __restrict__ grid, const v4i* __restrict__ frags,
                                            const v4i* __restrict__ init, uint64_t* __restrict__ out, uint64_t* Y,
                                            int lane, uint32_t k16, uint32_t keps) {
    constexpr int NP = enc13m::PAIRS;
    int H = 1 - (S & 1);
    const int j1b = (S >> 1) * 64 + lane;
    const int grp = lane >> 4, m = lane & 15;
    const int q0 = NP * S;
    v4i af[NP][2];
#pragma unroll
    for (int P = 0; P < NP; ++P)
#pragma unroll
        for (int h = 0; h < 2; ++h) af[P][h] = frags[((q0 + P) * 2 + h) * 64 + lane];
    // Buffer loads put the pair and tile parts of the twiddle and init addresses
    // in the scalar offset, so no per-load address registers stay live.
    const __amdgpu_buffer_rsrc_t grsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint64_t*>(grid), static_cast<short>(0), static_cast<int>(GRID_BYTES), 0x00020000);
    const __amdgpu_buffer_rsrc_t irsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<v4i*>(init), static_cast<short>(0), static_cast<int>(enc13m::INIT_WORDS * sizeof(int)), 0x00020000);
    const uint32_t g_off = static_cast<uint32_t>(((4 * q0 + grp) * N2 + m) * sizeof(uint64_t));
    const uint32_t i_off = static_cast<uint32_t>((4 * q0 + grp) * 2 * sizeof(v4i));
    auto g_load = [&](int P, int t) {  // w^(i2 j1) for j1 = 4 (q0 + P) + grp, i2 = 16 t + m
        const uint32_t so = static_cast<uint32_t>((4 * P * N2 + 16 * t) * sizeof(uint64_t));
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(grsrc, g_off, so, 0);
        return static_cast<uint64_t>(v[0]) | (static_cast<uint64_t>(v[1]) << 32);
    };
    auto c_load = [&](int P, int h) {  // init words of j1 = 4 (q0 + P) + grp, positions 4 h .. 4 h + 3
        const uint32_t so = static_cast<uint32_t>((4 * P * 2 + h) * sizeof(v4i));
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(irsrc, i_off, so, 0);
        return v4i{static_cast<int>(v[0]), static_cast<int>(v[1]), static_cast<int>(v[2]), static_cast<int>(v[3])};
    };
    // The first two pairs' init words and the first pair's twiddles do not
    // depend on the row: held in registers, so a row's phase A starts without
    // waiting on L2.
    const v4i c00 = c_load(0, 0), c01 = c_load(0, 1), c10 = c_load(1, 0), c11 = c_load(1, 1);
    uint64_t g0[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) g0[t] = g_load(0, t);
    v4i xf[4];
    size_t row = blockIdx.x;  // < rows: the grid never exceeds the row count
    load_frags(w + row * cols, cols, lane, xf);
    for (; row < rows; row += gridDim.x) {
        // A SIMD holds one wave of each of two workgroups.  Phase A issues at a
        // higher wave priority than phase B, so when both waves are ready the
        // one heading for its workgroup's barrier goes first and the other fills
        // its gaps (without the priorities the encode is about 10% slower).
        __builtin_amdgcn_s_setprio(1);
        // Software pipeline over the pairs: pair P + 1's products are issued
        // before pair P's results are folded (the fold waits on the matrix
        // cores otherwise), its init words two pairs ahead and its twiddles one
        // pair ahead.
        uint64_t g[NP][4];
        v4i c[NP][2], d[NP][4][2];
        c[0][0] = c00;
        c[0][1] = c01;
        c[1][0] = c10;
        c[1][1] = c11;
#pragma unroll
        for (int t = 0; t < 4; ++t) g[0][t] = g0[t];
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int h = 0; h < 2; ++h) d[0][t][h] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[0][h], xf[t], c[0][h], 0, 0, 0);
#pragma unroll
        for (int P = 0; P < NP; ++P) {
            if (P + 2 < NP) {
                c[P + 2][0] = c_load(P + 2, 0);
                c[P + 2][1] = c_load(P + 2, 1);
            }
            if (P + 1 < NP) {
#pragma unroll
                for (int t = 0; t < 4; ++t) g[P + 1][t] = g_load(P + 1, t);
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int h = 0; h < 2; ++h)
                        d[P + 1][t][h] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[P + 1][h], xf[t], c[P + 1][h], 0, 0, 0);
            }
            const int j1 = 4 * (q0 + P) + grp;
            uint64_t y[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int a[4] = {d[P][t][0][0], d[P][t][0][1], d[P][t][0][2], d[P][t][0][3]};
                const int b[4] = {d[P][t][1][0], d[P][t][1][1], d[P][t][1][2], d[P][t][1][3]};
                y[t] = gl::mul32x4(enc13m::recombine(a, b, k16, keps), g[P][t]);
            }
            // columns i2 = 16 t + m and i2 + 32 (t + 2) of row j1 are both in
            // this lane: store phase B's first-stage sums and differences
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                Y[j1 * PITCH + 16 * t + m] = gl::add(y[t], y[t + 2]);
                Y[j1 * PITCH + 32 + 16 * t + m] = gl::sub(y[t], y[t + 2]);
            }
            __builtin_amdgcn_sched_barrier(0);  // at most two pairs' products in registers
        }
        const size_t next = row + gridDim.x;
        if (next < rows) load_frags(w + next * cols, cols, lane, xf);
        __syncthreads();
        __builtin_amdgcn_s_setprio(0);
        phase_b<LATE>(Y, j1b, H, out + row * N);
        H ^= 1;
    }
}

template <bool LATE>
__global__ __launch_bounds__(THREADS, 2) void encode13_i16(const int16_t* __restrict__ w, size_t cols, size_t rows,
                                                          const uint64_t* __restrict__ tables,
                                                          uint64_t* __restrict__ out, uint32_t k16, uint32_t keps) {
    extern __shared__ uint64_t Y[];
    const int lane = threadIdx.x & 63;
    const v4i* frags = reinterpret_cast<const v4i*>(reinterpret_cast<const unsigned char*>(tables) + GRID_BYTES);
    const v4i* init = reinterpret_cast<const v4i*>(reinterpret_cast<const unsigned char*>(frags) + enc13m::FRAG_BYTES);
    encode_rows<LATE>(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6), w, cols, rows, tables, frags, init, out, Y, lane, k16,
                keps);
}

// grid[j1 * 64 + i2] = w^(i2 j1) from the half table (w^e = -w^(e - n/2)).
__global__ void build_grid13(const uint64_t* __restrict__ tw, uint64_t* __restrict__ grid) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= N1 * N2) return;
    const int j1 = idx / N2, i2 = idx % N2;
    const int e = i2 * j1;  // < n
    grid[idx] = e < N / 2 ? tw[e] : gl::neg(tw[e - N / 2]);
}

// Phase A's tables after the grid: the A fragments (enc13m::a_fragment, one
// 16-byte fragment per thread) and the accumulator init words.
__global__ void build_phase_a13(const uint64_t* __restrict__ tw, int8_t* __restrict__ frags, int* __restrict__ init) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx < static_cast<int>(enc13m::FRAG_BYTES / 16)) enc13m::a_fragment(tw, idx, frags + 16 * idx);
    if (idx < static_cast<int>(enc13m::INIT_WORDS)) init[idx] = enc13m::init_word(tw, idx >> 3, idx & 7);
}

int build_grid(Context* c, TwiddleSet* t) {
    hipLaunchKernelGGL(build_grid13, dim3((N1 * N2 + 255) / 256), dim3(256), 0, c->stream,
                       static_cast<const uint64_t*>(t->fwd), t->grid);
    VMX_HIP(c, hipGetLastError());
    int8_t* frags = reinterpret_cast<int8_t*>(t->grid) + GRID_BYTES;
    int* init = reinterpret_cast<int*>(frags + enc13m::FRAG_BYTES);
    hipLaunchKernelGGL(build_phase_a13, dim3(static_cast<unsigned>((enc13m::FRAG_BYTES / 16 + 255) / 256)), dim3(256),
                       0, c->stream, static_cast<const uint64_t*>(t->fwd), frags, init);
    VMX_HIP(c, hipGetLastError());
    return build_rr13_table(c, static_cast<const uint64_t*>(t->fwd),
                            reinterpret_cast<uint64_t*>(reinterpret_cast<unsigned char*>(t->grid) + R13_OFF));
}

}  // namespace enc13

const uint64_t* enc13_rr_table(Context* c, TwiddleSet* t) {
    if (ensure_grid_twiddles(c, t, enc13::TABLE_BYTES, enc13::build_grid)) return nullptr;
    return reinterpret_cast<const uint64_t*>(reinterpret_cast<const unsigned char*>(t->grid) + enc13::R13_OFF);
}

int encode_i16_fast(Context* c, const int16_t* w, size_t rows, size_t cols, size_t n, uint64_t* out,
                    TwiddleSet* t) {
    if (n != static_cast<size_t>(enc13::N) || cols == 0 || cols > static_cast<size_t>(enc13::K * enc13::N2))
        return 1;
    if (rows == 0) return 0;
    if (ensure_grid_twiddles(c, t, enc13::TABLE_BYTES, enc13::build_grid)) return -1;
    // Two workgroups fit a CU (LDS); a persistent grid of that many overlaps
    // each row's input loads with the previous row's phase B.
    const size_t per_cu = 2;
    const size_t cus = c->cu_count > 0 ? static_cast<size_t>(c->cu_count) : 256;
    const unsigned blocks = static_cast<unsigned>(std::min(rows, per_cu * cus));
    // Where parity 1's shifts go (phase_b): after the barrier when each
    // workgroup walks at most LATE_ROWS rows.
    const bool late = rows <= enc13::LATE_ROWS * blocks;
    const void* k = late ? reinterpret_cast<const void*>(enc13::encode13_i16<true>)
                         : reinterpret_cast<const void*>(enc13::encode13_i16<false>);
    // The LDS limit is an attribute of the kernel on the current device: set
    // it on every call (a host-side call of about a microsecond), so no flag
    // shared between contexts, threads or devices is needed.
    VMX_HIP(c, hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(enc13::LDS_BYTES)));
    const uint64_t* grid = t->grid;
    if (late)
        hipLaunchKernelGGL(enc13::encode13_i16<true>, dim3(blocks), dim3(enc13::THREADS), enc13::LDS_BYTES, c->stream,
                           w, cols, rows, grid, out, 65536u, 0xFFFFFFFFu);
    else
        hipLaunchKernelGGL(enc13::encode13_i16<false>, dim3(blocks), dim3(enc13::THREADS), enc13::LDS_BYTES, c->stream,
                           w, cols, rows, grid, out, 65536u, 0xFFFFFFFFu);
    VMX_HIP(c, hipGetLastError());
    return 0;
}

}  // namespace vmx
