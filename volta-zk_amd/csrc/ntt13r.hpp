// ntt13r.hpp -- the phases of the one-pass forward NTT of 2^13-point u64 rows
// whose elements may all be nonzero (rows a caller wrote), as host/device
// functions of one thread, so that a host build can run them thread by thread
// between the kernel's barriers (host_check.cpp).
//
// Semantics: NttPlan::forward (rust/volta-pcs/src/ntt.rs:34-61) of rows of
// 2^13 canonical elements, X[k] = sum_j x_j w^(jk), zero from element 256 NZ on.
//
// Split n = 32 x 32 x 8: j = j1 + 8 j2 + 256 j3 (j1 < 8, j2, j3 < 32),
// k = k3 + 32 k2 + 1024 k1 (k3, k2 < 32, k1 < 8),
// jk = 256 j3 k3 + k3 (j1 + 8 j2) + 256 j2 k2 + 32 j1 k2 + 1024 j1 k1 (mod n):
//   stage A (thread m = j1 + 8 j2): A[k3] = sum_j3 x[m + 256 j3] w_32^(j3 k3),
//     then A[k3] *= w^(k3 m)                  (T1[k3][m], global)
//   stage B (thread (j1, k3)): B[k2] = sum_j2 A_(j1 + 8 j2)[k3] w_32^(j2 k2),
//     then B[k2] *= w_256^(j1 k2)             (T2[k2][j1], LDS)
//   stage C (thread (k3, x), four pairs k2 = p + 4 x): the 8-point DFTs over j1,
//     X[k3 + 32 k2 + 1024 k1].
// A workgroup of 256 threads holds one row, 32 values per thread; four
// workgroups share a CU and run independently, so one's loads overlap the
// others' arithmetic.  The exchanges move half a row per round, with the
// register-slot argument of ntt15.hpp: the first pairs k3h with j2b0 (wave
// bit 0 of both roles), the second k2h with j1b0 (wave bit 1 of both roles);
// stage C keeps j1 in slot p + 4 bitrev3(j1), so j1b0 is slot bit 4.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "gl64.hpp"
#include "gl64_shift.hpp"

namespace vmx {
namespace n13r {

constexpr int LOG_N = 13;
constexpr int N = 1 << LOG_N;
constexpr int THREADS = 256;
// First exchange: word (k3l, j2, j1) at k3l X1_PITCH + 128 (j2 & 1) + 8 (j2 >> 1) + j1.
// A write instruction covers 64 consecutive words; a read, 16 k3l (odd pitch) per 16 lanes.
constexpr int X1_PITCH = 257;
// Second exchange: word (j1, k3, k2l) at (16 j1 + k2l) 32 + k3; both sides read or
// write 32 consecutive k3 per instruction.
constexpr int XBUF_WORDS = 16 * X1_PITCH;
static_assert(XBUF_WORDS >= 4096, "the second exchange fits the buffer");
constexpr int T2_OFF = XBUF_WORDS;  // T2[k2 * 8 + j1] = w_256^(j1 k2), 256 words
constexpr int LDS_WORDS = T2_OFF + 256;
constexpr size_t LDS_BYTES = size_t{LDS_WORDS} * sizeof(uint64_t);
// Device table: T1[k3 * 256 + m] = w^(k3 m), then T2.
constexpr int T1_WORDS = 32 * 256;
constexpr int TABLE_WORDS = T1_WORDS + 256;

// Word idx of the device table from the reference's half table
// fwd = w^0 .. w^(n/2 - 1) (w^e = -w^(e - n/2)).
__host__ __device__ inline uint64_t table_word(const uint64_t* fwd, int idx) {
    const int e = idx < T1_WORDS ? (idx >> 8) * (idx & 255) : 32 * ((idx - T1_WORDS) >> 3) * ((idx - T1_WORDS) & 7);
    return e < N / 2 ? fwd[e] : gl::neg(fwd[e - N / 2]);
}

// The three roles of thread t (wave w = t >> 6: w0 = w & 1, w1 = w >> 1).
struct Role {
    int m;         // stage A: j1 + 8 j2
    int j1b, k3b;  // stage B
    int k3c, xc;   // stage C: k3, and k2 = p + 4 x for p < 4
};

__host__ __device__ inline Role role(int t) {
    const int w = t >> 6, lane = t & 63;
    const int w0 = w & 1, w1 = w >> 1;
    Role r;
    r.m = (lane & 7) + 8 * (w0 + 2 * ((lane >> 3) & 7) + 16 * w1);
    r.j1b = w1 + 2 * (lane >> 4);
    r.k3b = (lane & 15) + 16 * w0;
    r.k3c = lane & 31;
    r.xc = (lane >> 5) + 2 * w0 + 4 * w1;
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
struct Table1 {
#if defined(__HIP_DEVICE_COMPILE__)
    __amdgpu_buffer_rsrc_t r;
    __device__ explicit Table1(const uint64_t* tab) : r(rsrc(tab, size_t{TABLE_WORDS} * 8)) {}
    __device__ uint64_t at(int k3, int m) const {
        return ld64(r, static_cast<uint32_t>(m) * 8u, static_cast<uint32_t>(k3) * 2048u);
    }
#else
    const uint64_t* p;
    explicit Table1(const uint64_t* tab) : p(tab) {}
    uint64_t at(int k3, int m) const { return p[k3 * 256 + m]; }
#endif
};

// Row `row` of x (stride elements apart, len u64 then zeros): element m + 256 j3
// for j3 < NZ into slot bitrev5(j3), the rest zero.
template <int NZ>
__host__ __device__ __forceinline__ void load_row(uint64_t* v, const uint64_t* x, size_t stride, size_t len,
                                                  size_t row, int m) {
    gl::static_for<0, 32>([&](auto i_) { v[decltype(i_)::value] = 0; });
#if defined(__HIP_DEVICE_COMPILE__)
    const auto r = rsrc(x + row * stride, len * 8);
#endif
    gl::static_for<0, NZ>([&](auto j_) {
        constexpr int j3 = decltype(j_)::value;
#if defined(__HIP_DEVICE_COMPILE__)
        v[gl::bitrev_c(j3, 5)] = ld64(r, static_cast<uint32_t>(m) * 8u, j3 * 2048u);
#else
        const size_t idx = static_cast<size_t>(m) + 256 * j3;
        v[gl::bitrev_c(j3, 5)] = idx < len ? x[row * stride + idx] : 0;
#endif
    });
}

template <int TAG>
__host__ __device__ __forceinline__ void fence_half() {
#if defined(__HIP_DEVICE_COMPILE__)
    if constexpr (TAG == 0) asm volatile("; ntt13r half 0");
    else if constexpr (TAG == 1) asm volatile("; ntt13r half 1");
    else if constexpr (TAG == 2) asm volatile("; ntt13r half 2");
    else if constexpr (TAG == 3) asm volatile("; ntt13r half 3");
    else if constexpr (TAG == 4) asm volatile("; ntt13r half 4");
    else if constexpr (TAG == 5) asm volatile("; ntt13r half 5");
    else if constexpr (TAG == 6) asm volatile("; ntt13r half 6");
    else asm volatile("; ntt13r half 7");
#endif
}

// The first-exchange twiddles w^(k3 m), k3 = 16 h + L0 + l (l < 8), of a
// wave-uniform half h.
template <int L0>
__host__ __device__ __forceinline__ void load_tw1(uint64_t* tw, const Table1& t1, int h, int m) {
    gl::static_for<0, 8>([&](auto l_) {
        constexpr int l = decltype(l_)::value;
        tw[l] = t1.at(16 * h + L0 + l, m);
    });
}

// First exchange, half H of a thread in role m = j1 + 8 j2: A[16 H + l] times
// w^(k3 m) to word (l, j2, j1).  tw holds the twiddles of l < 8 on entry.
template <int H>
__host__ __device__ __forceinline__ void x1_write(uint64_t* lds, const uint64_t* v, uint64_t* tw, const Table1& t1,
                                                  int m) {
    fence_half<H>();
    const int j1 = m & 7, j2 = m >> 3;
    uint64_t* p = lds + 128 * (j2 & 1) + 8 * (j2 >> 1) + j1;
    gl::static_for<0, 16>([&](auto l_) {
        constexpr int l = decltype(l_)::value, k3 = 16 * H + l;
        if constexpr (l == 8) {
#if defined(__HIP_DEVICE_COMPILE__)
            __builtin_amdgcn_sched_barrier(0);
#endif
            load_tw1<8>(tw, t1, H, m);
        }
        p[l * X1_PITCH] = k3 ? gl::mul32x4(v[k3], tw[l & 7]) : v[k3];
    });
    fence_half<H>();
}

// j2 = H + 2 i (i < 16) of a thread in role (j1, k3) into slot 16 H + bitrev4(i).
template <int H>
__host__ __device__ __forceinline__ void x1_read(const uint64_t* lds, uint64_t* v, int j1, int k3) {
    fence_half<2 + H>();
    const uint64_t* p = lds + (k3 & 15) * X1_PITCH + 128 * H + j1;
    gl::static_for<0, 16>([&](auto i_) {
        constexpr int i = decltype(i_)::value;
        v[16 * H + gl::bitrev_c(i, 4)] = p[8 * i];
    });
    fence_half<2 + H>();
}

// Second exchange, half G of a thread in role (j1, k3): B[16 G + i] times
// w_256^(j1 k2) to word (j1, k3, i).
template <int G>
__host__ __device__ __forceinline__ void x2_write(uint64_t* lds, const uint64_t* v, int j1, int k3) {
    fence_half<4 + G>();
    uint64_t* p = lds + 16 * 32 * j1 + k3;
    const uint64_t* t2 = lds + T2_OFF + j1;
    gl::static_for<0, 16>([&](auto i_) {
        constexpr int i = decltype(i_)::value, k2 = 16 * G + i;
        p[32 * i] = k2 ? gl::mul32x4(v[k2], t2[8 * k2]) : v[k2];
    });
    fence_half<4 + G>();
}

// j1 = G + 2 q (q < 4) for the four pairs k2 = p + 4 x of a thread in role
// (k3, x) into slot 16 G + p + 4 bitrev2(q) (= p + 4 bitrev3(j1)).
template <int G>
__host__ __device__ __forceinline__ void x2_read(const uint64_t* lds, uint64_t* v, int k3, int x) {
    fence_half<6 + G>();
    const uint64_t* base = lds + 32 * ((4 * x) & 15) + k3;
    gl::static_for<0, 4>([&](auto q_) {
        constexpr int q = decltype(q_)::value, j1 = G + 2 * q;
        gl::static_for<0, 4>([&](auto p_) {
            constexpr int p = decltype(p_)::value;
            v[16 * G + p + 4 * gl::bitrev_c(q, 2)] = base[32 * (16 * j1 + p)];
        });
    });
    fence_half<6 + G>();
}

// Stage C: the 8-point DFT of each pair p over slots p + 4 s (j1 bit-reversed
// in, k1 natural out).
__host__ __device__ __forceinline__ void stage_c(uint64_t* v) {
    gl::static_for<0, 4>([&](auto p_) {
        constexpr int p = decltype(p_)::value;
        uint64_t u[8];
        gl::static_for<0, 8>([&](auto s_) { u[decltype(s_)::value] = v[p + 4 * decltype(s_)::value]; });
        gl::dit_pow2<3, 120>(u);
        gl::static_for<0, 8>([&](auto s_) { v[p + 4 * decltype(s_)::value] = u[decltype(s_)::value]; });
    });
}

}  // namespace n13r
}  // namespace vmx
