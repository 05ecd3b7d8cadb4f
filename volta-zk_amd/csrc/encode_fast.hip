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
//   phase B (thread = row j1 x parity h, h = wave >> 1): the 64-point DFT over
//     i2 (w64 = 2^39) as its first radix-2 DIF stage followed by one 32-point
//     DFT per parity; X[2k + h] goes to out[j1 + 128 (2k + h)], so each store
//     instruction writes 64 consecutive u64.
// One workgroup (4 waves) per row; Y lives in LDS with a padded pitch.
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

// Phase A for coset S and column i2 of one row: writes Y[4 t1 + S][i2].
template <int S>
__host__ __device__ __forceinline__ void phase_a(const int16_t* wr, size_t cols, int i2, const uint64_t* grid,
                                                 uint64_t* Y) {
    int32_t x[K];
    // Branchless bounds: clamp the address, zero the value past cols.
#pragma unroll
    for (int i1 = 0; i1 < K; ++i1) {
        const size_t idx = static_cast<size_t>(i1) * N2 + i2;
        const int32_t raw = static_cast<int32_t>(wr[idx < cols ? idx : cols - 1]);
        x[i1] = idx < cols ? raw : 0;
    }
    uint64_t v[K];
    gl::static_for<0, K>([&](auto ii) {
        constexpr int i1 = decltype(ii)::value;
        v[gl::bitrev_c(i1, 5)] = gl::i16_mul_w128<S * i1>(x[i1]);
    });
    gl::dit_pow2<5, gl::E_W32>(v);
#pragma unroll
    for (int t1 = 0; t1 < K; ++t1) {
        const int j1 = 4 * t1 + S;
        Y[j1 * PITCH + i2] = gl::mul32x4(v[t1], grid[j1 * N2 + i2]);
    }
}

// Phase B for row j1 and output parity H: returns X[2k + H] in v[k].
template <int H>
__host__ __device__ __forceinline__ void phase_b(const uint64_t* Y, int j1, uint64_t* v) {
    const uint64_t* y = Y + j1 * PITCH;
    gl::static_for<0, 32>([&](auto qq) {
        constexpr int q = decltype(qq)::value;
        const uint64_t a = y[q], b = y[q + 32];
        if constexpr (H == 0) v[gl::bitrev_c(q, 5)] = gl::add(a, b);
        else v[gl::bitrev_c(q, 5)] = gl::mul_pow2<gl::E_W64 * q>(gl::sub(a, b));
    });
    gl::dit_pow2<5, gl::E_W32>(v);
}

__global__ __launch_bounds__(THREADS, 2) void encode13_i16(const int16_t* __restrict__ w, size_t cols,
                                                          const uint64_t* __restrict__ grid,
                                                          uint64_t* __restrict__ out) {
    extern __shared__ uint64_t Y[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const size_t row = blockIdx.x;
    const int16_t* wr = w + row * cols;
    switch (wave) {
        case 0: phase_a<0>(wr, cols, lane, grid, Y); break;
        case 1: phase_a<1>(wr, cols, lane, grid, Y); break;
        case 2: phase_a<2>(wr, cols, lane, grid, Y); break;
        default: phase_a<3>(wr, cols, lane, grid, Y); break;
    }
    __syncthreads();
    const int j1 = (wave & 1) * 64 + lane;
    uint64_t* o = out + row * N + j1;
    uint64_t v[32];
    if (wave < 2) {
        phase_b<0>(Y, j1, v);
#pragma unroll
        for (int k = 0; k < 32; ++k) __builtin_nontemporal_store(v[k], o + N1 * (2 * k));
    } else {
        phase_b<1>(Y, j1, v);
#pragma unroll
        for (int k = 0; k < 32; ++k) __builtin_nontemporal_store(v[k], o + N1 * (2 * k + 1));
    }
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
    if (ensure_grid_twiddles(c, t, size_t{enc13::N1} * enc13::N2 * sizeof(uint64_t), enc13::build_grid)) return -1;
    static bool lds_ok = false;  // the attribute is per-process, per-kernel
    if (!lds_ok) {
        VMX_HIP(c, hipFuncSetAttribute(reinterpret_cast<const void*>(enc13::encode13_i16),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       static_cast<int>(enc13::LDS_BYTES)));
        lds_ok = true;
    }
    for (size_t r0 = 0; r0 < rows; r0 += 0x7FFFFFFF) {
        const size_t cnt = std::min<size_t>(rows - r0, 0x7FFFFFFF);
        hipLaunchKernelGGL(enc13::encode13_i16, dim3(static_cast<unsigned>(cnt)), dim3(enc13::THREADS),
                           enc13::LDS_BYTES, c->stream, w + r0 * cols, cols, static_cast<const uint64_t*>(t->grid),
                           out + r0 * enc13::N);
        VMX_HIP(c, hipGetLastError());
    }
    return 0;
}

}  // namespace vmx
