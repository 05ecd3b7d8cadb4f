// encode_fast.hip -- the Ligero RS-encode fast path for gfx950.
//
// Shape: codeword length n = 2^13, i16 message rows of cols <= 2^11 (rate
// <= 1/4: the GPT-2 weight commits, configurations c_attn and full GPT-2).
// Output is bit-identical to NttPlan::encode of lift(w) zero-padded
// (rust/volta-pcs/src/ntt.rs:36-70); the factorisation below is exact.
//
// Four-step split n = 128 x 64, input index i = 64*i1 + i2 (i1 < 128, and
// only i1 < 32 is non-zero), output index j = j1 + 128*j2:
//   phase A (thread = coset s in 0..3 x column i2 in 0..63, s = wave):
//       X[4 t1 + s] = sum_{i1<32} (x[64 i1 + i2] * w128^(s i1)) * w32^(i1 t1)
//     i.e. the 128-point DFT of a 32-long column as four 32-point DFTs of
//     pre-twiddled inputs.  w128^k is a power of two (or a difference of two)
//     times a 16-bit integer, w32 = 2^78: shifts only.  Then
//       Y[j1][i2] = X[j1] * w_n^(i2 j1)      (the only 64x64 products)
//   phase B (thread = row j1 x parity h, h = 1 - (wave & 1)): the 64-point DFT over
//     i2 (w64 = 2^39) as its first radix-2 DIF stage followed by one 32-point
//     DFT per parity; X[2k + h] goes to out[j1 + 128 (2k + h)], so each store
//     instruction writes 64 consecutive u64.
// A persistent grid of 4-wave workgroups walks the rows; Y lives in LDS with a
// padded pitch.
// HBM traffic per row: 4 KiB of i16 read + 64 KiB of u64 written.
#include <hip/hip_runtime.h>

#include "context.hpp"
#include "gl64.hpp"
#include "gl64_shift.hpp"
#include "kernels.hpp"

namespace vmx {

namespace enc13 {

constexpr int LOG_N = 13;
constexpr int N = 1 << LOG_N;
constexpr int N1 = 128;    // j1 range
constexpr int N2 = 64;     // i2 range
constexpr int K = 32;      // non-zero i1 range (cols <= K * N2 = 2048)
constexpr int PITCH = 65;  // u64 per LDS row of Y
constexpr int THREADS = 256;
constexpr size_t LDS_BYTES = size_t{N1} * PITCH * sizeof(uint64_t);

// The 32 possibly non-zero entries x[64 i1 + i2] (i1 < 32) of one row, zero
// past cols.  A raw buffer resource spanning exactly the row's cols entries
// makes the hardware return 0 for the tail (an out-of-range buffer load reads
// zero and touches no memory), and all 32 loads share one offset register.
__device__ __forceinline__ void load_column(const int16_t* wr, size_t cols, int i2, uint32_t* x) {
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int16_t*>(wr), static_cast<short>(0), static_cast<int>(cols * sizeof(int16_t)), 0x00020000);
    const int off = i2 * static_cast<int>(sizeof(int16_t));
#pragma unroll
    for (int q = 0; q < K / 2; ++q) {  // x[q] = w[2q] | w[2q + 1] << 16 (two i16 per register)
        const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b16(rsrc, off + 2 * q * N2 * static_cast<int>(sizeof(int16_t)), 0, 0);
        const uint32_t hi = __builtin_amdgcn_raw_buffer_load_b16(rsrc, off + (2 * q + 1) * N2 * static_cast<int>(sizeof(int16_t)), 0, 0);
        x[q] = (lo & 0xFFFFu) | (hi << 16);
    }
}

// Phase B's LDS half for row j1 and output parity H: reads Y's row and applies
// the first radix-2 stage; the 32-point DFT over v then gives X[2k + H] in v[k].
template <int H>
__host__ __device__ __forceinline__ void phase_b_first(const uint64_t* Y, int j1, uint64_t* v) {
    const uint64_t* y = Y + j1 * PITCH;
    gl::static_for<0, 32>([&](auto qq) {
        constexpr int q = decltype(qq)::value;
        const uint64_t a = y[q], b = y[q + 32];
        if constexpr (H == 0) v[gl::bitrev_c(q, 5)] = gl::add(a, b);
        else v[gl::bitrev_c(q, 5)] = gl::mul_pow2<gl::E_W64 * q>(gl::sub(a, b));
    });
}

// Coset S's pre-twiddled inputs in bit-reversed order: v[brev(i1)] = x[i1] w128^(S i1)
// (xp: the column's 32 inputs, two i16 per word).
template <int S>
__device__ __forceinline__ void pretwiddle(const uint32_t* xp, uint64_t* v) {
    gl::static_for<0, K>([&](auto ii) {
        constexpr int i1 = decltype(ii)::value;
        const int32_t xi = static_cast<int16_t>(static_cast<uint16_t>(i1 & 1 ? xp[i1 >> 1] >> 16 : xp[i1 >> 1]));
        v[gl::bitrev_c(i1, 5)] = gl::i16_mul_w128<S * i1>(xi);
    });
}

// One wave's share of every row its workgroup owns: wave S runs phase A for
// coset S and phase B for rows j1 in [64 (S >> 1), 64 (S >> 1) + 64) and
// parity H = 1 - (S & 1).  S is uniform, so no lane diverges.  Only the
// pre-twiddles and phase B's first stage depend on the wave; the DFTs and the
// twiddle products are one copy of code for all four waves (43 KB of code
// instead of 136 KB).  The even cosets (pure-shift pre-twiddles) take the
// dearer parity 1 (sub + shift first stage), which evens out the waves' work
// per row.  The workgroup walks rows blockIdx.x, blockIdx.x + gridDim.x, ...,
// loading the next row's inputs while phase B of the current row runs.
__device__ __forceinline__ void encode_rows(int S, const int16_t* __restrict__ w, size_t cols, size_t rows,
                                            const uint64_t* __restrict__ grid, uint64_t* __restrict__ out,
                                            uint64_t* Y, int lane) {
    const int H = 1 - (S & 1);
    const int j1 = (S >> 1) * 64 + lane;
    uint32_t x[K / 2];
    size_t row = blockIdx.x;  // < rows: the grid never exceeds the row count
    load_column(w + row * cols, cols, lane, x);
    for (; row < rows; row += gridDim.x) {
        // A SIMD holds one wave of each of two workgroups.  Phase A issues at a
        // higher wave priority than phase B, so when both waves are ready the
        // one heading for its workgroup's barrier goes first and the other fills
        // its gaps (measured: 2.43 -> 2.27 ms on C3; priority 3 or 2/1 the same).
        __builtin_amdgcn_s_setprio(1);
        // Phase A: the four-step twiddles w_n^(i2 (4 t1 + S)) come from the
        // L2-resident grid, loaded before the DFT so its arithmetic covers them.
        uint64_t g[K];
#pragma unroll
        for (int t1 = 0; t1 < K; ++t1) g[t1] = grid[(4 * t1 + S) * N2 + lane];
        __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the DFT
        uint64_t v[K];
        switch (S) {
            case 0: pretwiddle<0>(x, v); break;
            case 1: pretwiddle<1>(x, v); break;
            case 2: pretwiddle<2>(x, v); break;
            default: pretwiddle<3>(x, v); break;
        }
        gl::dit_pow2<5, gl::E_W32>(v);
#pragma unroll
        for (int t1 = 0; t1 < K; ++t1) Y[(4 * t1 + S) * PITCH + lane] = gl::mul32x4(v[t1], g[t1]);
        const size_t next = row + gridDim.x;
        if (next < rows) load_column(w + next * cols, cols, lane, x);
        __syncthreads();
        __builtin_amdgcn_s_setprio(0);
        if (H == 0) phase_b_first<0>(Y, j1, v);
        else phase_b_first<1>(Y, j1, v);
        // Y is rewritten by the next row's phase A.  Once every wave holds its
        // rows' first stage in registers the workgroup may move on, so the
        // DFTs and stores of phase B overlap the next phase A of faster waves.
        __syncthreads();
        gl::dit_pow2<5, gl::E_W32>(v);
        uint64_t* o = out + row * N + j1 + N1 * H;
#pragma unroll
        for (int k = 0; k < 32; ++k) __builtin_nontemporal_store(v[k], o + N1 * 2 * k);
    }
}

__global__ __launch_bounds__(THREADS, 2) void encode13_i16(const int16_t* __restrict__ w, size_t cols, size_t rows,
                                                          const uint64_t* __restrict__ grid,
                                                          uint64_t* __restrict__ out) {
    extern __shared__ uint64_t Y[];
    const int lane = threadIdx.x & 63;
    encode_rows(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6), w, cols, rows, grid, out, Y, lane);
}

// grid[j1 * 64 + i2] = w^(i2 j1) from the half table (w^e = -w^(e - n/2)).
__global__ void build_grid13(const uint64_t* __restrict__ tw, uint64_t* __restrict__ grid) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= N1 * N2) return;
    const int j1 = idx / N2, i2 = idx % N2;
    const int e = i2 * j1;  // < n
    grid[idx] = e < N / 2 ? tw[e] : gl::neg(tw[e - N / 2]);
}

int build_grid(Context* c, TwiddleSet* t) {
    hipLaunchKernelGGL(build_grid13, dim3((N1 * N2 + 255) / 256), dim3(256), 0, c->stream,
                       static_cast<const uint64_t*>(t->fwd), t->grid);
    VMX_HIP(c, hipGetLastError());
    return 0;
}

}  // namespace enc13

int encode_i16_fast(Context* c, const int16_t* w, size_t rows, size_t cols, size_t n, uint64_t* out,
                    TwiddleSet* t) {
    if (n != static_cast<size_t>(enc13::N) || cols == 0 || cols > static_cast<size_t>(enc13::K * enc13::N2))
        return 1;
    if (rows == 0) return 0;
    if (ensure_grid_twiddles(c, t, size_t{enc13::N1} * enc13::N2 * sizeof(uint64_t), enc13::build_grid)) return -1;
    // The LDS limit is an attribute of the kernel on the current device: set
    // it on every call (a host-side call of about a microsecond), so no flag
    // shared between contexts, threads or devices is needed.
    VMX_HIP(c, hipFuncSetAttribute(reinterpret_cast<const void*>(enc13::encode13_i16),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(enc13::LDS_BYTES)));
    // Two workgroups fit a CU (LDS); a persistent grid of that many overlaps
    // each row's input loads with the previous row's phase B.
    const size_t per_cu = 2;
    const size_t cus = c->cu_count > 0 ? static_cast<size_t>(c->cu_count) : 256;
    const unsigned blocks = static_cast<unsigned>(std::min(rows, per_cu * cus));
    hipLaunchKernelGGL(enc13::encode13_i16, dim3(blocks), dim3(enc13::THREADS), enc13::LDS_BYTES, c->stream, w, cols,
                       rows, static_cast<const uint64_t*>(t->grid), out);
    VMX_HIP(c, hipGetLastError());
    return 0;
}

}  // namespace vmx
