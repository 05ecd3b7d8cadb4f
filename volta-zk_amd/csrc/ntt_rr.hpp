// ntt_rr.hpp -- the phases of the one-pass forward NTT of u64 rows of
// n = 32 x 32 x N1 points (N1 = 2^B: 2^13 for B = 3, 2^14 for B = 4) whose
// elements may all be nonzero, as host/device functions of one thread, so
// that a host build can run them thread by thread between the kernel's
// barriers (host_check.cpp).
//
// Semantics: NttPlan::forward (rust/volta-pcs/src/ntt.rs:34-61) of rows of n
// canonical elements, X[k] = sum_j x_j w^(jk), zero from element 32 N1 NZ on.
//
// j = j1 + N1 j2 + 32 N1 j3 (j1 < N1; j2, j3 < 32), k = k3 + 32 k2 + 1024 k1
// (k3, k2 < 32; k1 < N1), so that
// jk = 32 N1 j3 k3 + k3 (j1 + N1 j2) + 32 N1 j2 k2 + 32 j1 k2 + 1024 j1 k1 (mod n):
//   stage A (thread m = j1 + N1 j2): A[k3] = sum_j3 x[m + 32 N1 j3] w_32^(j3 k3),
//     then A[k3] *= w^(k3 m)                  (T1[k3][m], global)
//   stage B (thread (j1, k3)): B[k2] = sum_j2 A_(j1 + N1 j2)[k3] w_32^(j2 k2),
//     then B[k2] *= w^(32 j1 k2)              (T2[k2][j1], LDS)
//   stage C (thread (k3, x), P = 32 / N1 pairs k2 = p + P x): the N1-point
//     DFTs over j1, X[k3 + 32 k2 + 1024 k1].
// A workgroup of 32 N1 threads holds one row, 32 values per thread; for 2^13
// four workgroups share a CU and run independently, so one's loads overlap the
// others' arithmetic.  The exchanges move half a row per round, with the
// register-slot argument of ntt15.hpp: the first pairs k3h with j2b0 (wave
// bit 0 of both roles), the second k2h with j1b0 (wave bit 1 of both roles);
// stage C keeps j1 of pair p in slot p + P bitrev_B(j1), so j1b0 is slot bit 4.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "gl64.hpp"
#include "gl64_shift.hpp"

namespace vmx {
namespace rr {

template <int B>
struct Shape {
    static_assert(B == 3 || B == 4, "n = 2^13 or 2^14");
    static constexpr int N1 = 1 << B;
    static constexpr int LOG_N = 10 + B;
    static constexpr int N = 1 << LOG_N;
    static constexpr int THREADS = 32 * N1;
    // Workgroups per CU: four 4-wave workgroups at 128 VGPRs for 2^13; one
    // 8-wave workgroup for 2^14, whose stage C (two 16-point DFTs per thread)
    // takes 174 VGPRs (at 128 it spilled 61-80).
    static constexpr int PER_CU = B == 3 ? 4 : 1;
    static constexpr int WAVES_PER_SIMD = PER_CU * THREADS / 256;
    static constexpr int P = 32 / N1;  // stage-C pairs per thread
    static constexpr int M = 32 * N1;  // stage-A rows m = j1 + N1 j2
    // First exchange: word (k3l, j2, j1) at k3l X1_PITCH + 16 N1 (j2 & 1) + N1 (j2 >> 1) + j1.
    // A write instruction covers 64 consecutive words; a read, 16 k3l (odd pitch) per 16 lanes.
    static constexpr int X1_PITCH = 32 * N1 + 1;
    // Second exchange: word (j1, k3, k2l) at (16 j1 + k2l) 32 + k3; both sides read or
    // write 32 consecutive k3 per instruction.
    static constexpr int XBUF_WORDS = 16 * X1_PITCH;
    static_assert(XBUF_WORDS >= 512 * N1, "the second exchange fits the buffer");
    static constexpr int T2_OFF = XBUF_WORDS;  // T2[k2 N1 + j1] = w^(32 j1 k2)
    static constexpr int T2_WORDS = 32 * N1;
    static constexpr int LDS_WORDS = T2_OFF + T2_WORDS;
    static constexpr size_t LDS_BYTES = size_t{LDS_WORDS} * sizeof(uint64_t);
    // Device table: T1[k3 M + m] = w^(k3 m), then T2.
    static constexpr int T1_WORDS = 32 * M;
    static constexpr int TABLE_WORDS = T1_WORDS + T2_WORDS;
    static constexpr int E_WN1 = B == 3 ? 120 : 156;  // w_8 = 2^120, w_16 = 2^156
};

// Word idx of the device table from the reference's half table
// fwd = w^0 .. w^(n/2 - 1) (w^e = -w^(e - n/2)).
template <int B>
__host__ __device__ inline uint64_t table_word(const uint64_t* fwd, int idx) {
    using S = Shape<B>;
    const int e = idx < S::T1_WORDS ? (idx / S::M) * (idx % S::M)
                                    : 32 * ((idx - S::T1_WORDS) / S::N1) * ((idx - S::T1_WORDS) % S::N1);
    return e < S::N / 2 ? fwd[e] : gl::neg(fwd[e - S::N / 2]);
}

// The three roles of thread t (wave w = t >> 6: w0 = w & 1, w1 = bit 1 of w,
// wr = w >> 2, zero for B = 3).
struct Role {
    int m;         // stage A: j1 + N1 j2
    int j1b, k3b;  // stage B
    int k3c, xc;   // stage C: k3, and k2 = p + P x for p < P
};

template <int B>
__host__ __device__ inline Role role(int t) {
    const int w = t >> 6, lane = t & 63;
    const int w0 = w & 1, w1 = (w >> 1) & 1, wr = w >> 2;
    constexpr int N1 = 1 << B;
    Role r;
    r.m = (lane & (N1 - 1)) + N1 * (w0 + 2 * (lane >> B) + (1 << (7 - B)) * (w >> 1));
    r.j1b = w1 + 2 * (lane >> 4) + 8 * wr;
    r.k3b = (lane & 15) + 16 * w0;
    r.k3c = lane & 31;
    r.xc = B == 3 ? (lane >> 5) + 2 * w0 + 4 * w1 : (lane >> 5) + 2 * w0 + 4 * wr + 8 * w1;
    return r;
}

constexpr uint64_t prefix_mask(int nz) {
    uint64_t m = 0;
    for (int j = 0; j < nz; ++j) m |= uint64_t{1} << gl::bitrev_c(j, 5);
    return m;
}

#if defined(__HIP_DEVICE_COMPILE__)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, size_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), static_cast<short>(0), static_cast<int>(bytes),
                                             0x00020000);
}
__device__ __forceinline__ uint64_t ld64(const __amdgpu_buffer_rsrc_t& r, uint32_t voff, uint32_t soff) {
    const auto t = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
    return static_cast<uint64_t>(t[0]) | (static_cast<uint64_t>(t[1]) << 32);
}
#endif

// T1 of the device table.
template <int B>
struct Table1 {
#if defined(__HIP_DEVICE_COMPILE__)
    __amdgpu_buffer_rsrc_t r;
    __device__ explicit Table1(const uint64_t* tab) : r(rsrc(tab, size_t{Shape<B>::TABLE_WORDS} * 8)) {}
    __device__ uint64_t at(int k3, int m) const {
        return ld64(r, static_cast<uint32_t>(m) * 8u, static_cast<uint32_t>(k3) * (Shape<B>::M * 8u));
    }
#else
    const uint64_t* p;
    explicit Table1(const uint64_t* tab) : p(tab) {}
    uint64_t at(int k3, int m) const { return p[k3 * Shape<B>::M + m]; }
#endif
};

// Row `row` of x (stride elements apart, len u64 then zeros): element
// m + 32 N1 j3 for j3 < NZ into slot bitrev5(j3), the rest zero.
template <int B, int NZ>
__host__ __device__ __forceinline__ void load_row(uint64_t* v, const uint64_t* x, size_t stride, size_t len,
                                                  size_t row, int m) {
    constexpr int M = Shape<B>::M;
    gl::static_for<0, 32>([&](auto i_) { v[decltype(i_)::value] = 0; });
#if defined(__HIP_DEVICE_COMPILE__)
    const auto r = rsrc(x + row * stride, len * 8);
#endif
    gl::static_for<0, NZ>([&](auto j_) {
        constexpr int j3 = decltype(j_)::value;
#if defined(__HIP_DEVICE_COMPILE__)
        v[gl::bitrev_c(j3, 5)] = ld64(r, static_cast<uint32_t>(m) * 8u, j3 * (M * 8u));
#else
        const size_t idx = static_cast<size_t>(m) + size_t{M} * j3;
        v[gl::bitrev_c(j3, 5)] = idx < len ? x[row * stride + idx] : 0;
#endif
    });
}

// A distinct empty asm statement at both ends of each half's code: the two
// halves of an exchange differ only in which register slots they use, and
// without these the compiler merges them into one path that selects the
// slot at run time, which moves the whole register array into scratch memory.
template <int TAG>
__host__ __device__ __forceinline__ void fence_half() {
#if defined(__HIP_DEVICE_COMPILE__)
    if constexpr (TAG == 0) asm volatile("; ntt_rr half 0");
    else if constexpr (TAG == 1) asm volatile("; ntt_rr half 1");
    else if constexpr (TAG == 2) asm volatile("; ntt_rr half 2");
    else if constexpr (TAG == 3) asm volatile("; ntt_rr half 3");
    else if constexpr (TAG == 4) asm volatile("; ntt_rr half 4");
    else if constexpr (TAG == 5) asm volatile("; ntt_rr half 5");
    else if constexpr (TAG == 6) asm volatile("; ntt_rr half 6");
    else asm volatile("; ntt_rr half 7");
#endif
}

// The first-exchange twiddles w^(k3 m), k3 = 16 h + L0 + l (l < 8), of a
// wave-uniform half h.
template <int B, int L0>
__host__ __device__ __forceinline__ void load_tw1(uint64_t* tw, const Table1<B>& t1, int h, int m) {
    gl::static_for<0, 8>([&](auto l_) {
        constexpr int l = decltype(l_)::value;
        tw[l] = t1.at(16 * h + L0 + l, m);
    });
}

// First exchange, half H of a thread in role m = j1 + N1 j2: A[16 H + l]
// times w^(k3 m) to word (l, j2, j1).  tw holds the twiddles of l < 8 on
// entry; the other eight load while the first eight are written.
template <int B, int H>
__host__ __device__ __forceinline__ void x1_write(uint64_t* lds, const uint64_t* v, uint64_t* tw,
                                                  const Table1<B>& t1, int m) {
    using S = Shape<B>;
    fence_half<H>();
    const int j1 = m & (S::N1 - 1), j2 = m >> B;
    uint64_t* p = lds + 16 * S::N1 * (j2 & 1) + S::N1 * (j2 >> 1) + j1;
    gl::static_for<0, 16>([&](auto l_) {
        constexpr int l = decltype(l_)::value, k3 = 16 * H + l;
        if constexpr (l == 8) {
#if defined(__HIP_DEVICE_COMPILE__)
            __builtin_amdgcn_sched_barrier(0);
#endif
            load_tw1<B, 8>(tw, t1, H, m);
        }
        p[l * S::X1_PITCH] = k3 ? gl::mul32x4(v[k3], tw[l & 7]) : v[k3];
    });
    fence_half<H>();
}

// j2 = H + 2 i (i < 16) of a thread in role (j1, k3) into slot 16 H + bitrev4(i).
template <int B, int H>
__host__ __device__ __forceinline__ void x1_read(const uint64_t* lds, uint64_t* v, int j1, int k3) {
    using S = Shape<B>;
    fence_half<2 + H>();
    const uint64_t* p = lds + (k3 & 15) * S::X1_PITCH + 16 * S::N1 * H + j1;
    gl::static_for<0, 16>([&](auto i_) {
        constexpr int i = decltype(i_)::value;
        v[16 * H + gl::bitrev_c(i, 4)] = p[S::N1 * i];
    });
    fence_half<2 + H>();
}

// Second exchange, half G of a thread in role (j1, k3): B[16 G + i] times
// w^(32 j1 k2) to word (j1, k3, i).
template <int B, int G>
__host__ __device__ __forceinline__ void x2_write(uint64_t* lds, const uint64_t* v, int j1, int k3) {
    using S = Shape<B>;
    fence_half<4 + G>();
    uint64_t* p = lds + 16 * 32 * j1 + k3;
    const uint64_t* t2 = lds + S::T2_OFF + j1;
    gl::static_for<0, 16>([&](auto i_) {
        constexpr int i = decltype(i_)::value, k2 = 16 * G + i;
        p[32 * i] = k2 ? gl::mul32x4(v[k2], t2[S::N1 * k2]) : v[k2];
    });
    fence_half<4 + G>();
}

// j1 = G + 2 q (q < N1 / 2) for the P pairs k2 = p + P x of a thread in role
// (k3, x) into slot 16 G + p + P bitrev_(B-1)(q) (= p + P bitrev_B(j1)).
template <int B, int G>
__host__ __device__ __forceinline__ void x2_read(const uint64_t* lds, uint64_t* v, int k3, int x) {
    using S = Shape<B>;
    fence_half<6 + G>();
    const uint64_t* base = lds + 32 * ((S::P * x) & 15) + k3;
    gl::static_for<0, S::N1 / 2>([&](auto q_) {
        constexpr int q = decltype(q_)::value, j1 = G + 2 * q;
        gl::static_for<0, S::P>([&](auto p_) {
            constexpr int p = decltype(p_)::value;
            v[16 * G + p + S::P * gl::bitrev_c(q, B - 1)] = base[32 * (16 * j1 + p)];
        });
    });
    fence_half<6 + G>();
}

// Stage C: the N1-point DFT of each pair p over slots p + P s (j1 bit-reversed
// in, k1 natural out).
template <int B>
__host__ __device__ __forceinline__ void stage_c(uint64_t* v) {
    using S = Shape<B>;
    gl::static_for<0, S::P>([&](auto p_) {
        constexpr int p = decltype(p_)::value;
        uint64_t u[S::N1];
        gl::static_for<0, S::N1>([&](auto s_) { u[decltype(s_)::value] = v[p + S::P * decltype(s_)::value]; });
        gl::dit_pow2<B, S::E_WN1>(u);
        gl::static_for<0, S::N1>([&](auto s_) { v[p + S::P * decltype(s_)::value] = u[decltype(s_)::value]; });
    });
}

}  // namespace rr
}  // namespace vmx
