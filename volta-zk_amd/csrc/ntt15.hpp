// ntt15.hpp -- the phases of the one-pass forward NTT of 2^15 points
// (ntt15.hip), as host/device functions of one thread, so that a host build
// can run them thread by thread between the kernel's barriers.
//
// Semantics: NttPlan::forward of a zero-tailed row (rust/volta-pcs/src/ntt.rs:34-70),
// X[k] = sum_j x_j w^(jk), w the reference's primitive 2^15-th root, for rows
// whose inputs are zero from index 1024 NZ on.
//
// Split n = 32 x 32 x 32: j = j1 + 32 j2 + 1024 j3, k = k3 + 32 k2 + 1024 k1,
// jk = 1024 j3 k3 + k3 (j1 + 32 j2) + 1024 j2 k2 + 32 j1 k2 + 1024 j1 k1 (mod n):
//   stage A (thread m = j1 + 32 j2): A[k3] = sum_{j3 < NZ} x[m + 1024 j3] w_32^(j3 k3),
//     then A[k3] *= w^(k3 m)                       (table T1[k3][m], global)
//   stage B (thread (j1, k3)): B[k2] = sum_j2 A_(j1 + 32 j2)[k3] w_32^(j2 k2),
//     then B[k2] *= w_1024^(j1 k2)                 (table T2[k2][j1], LDS)
//   stage C (thread (k3, k2)): X[k3 + 32 k2 + 1024 k1] = sum_j1 B_(j1, k3)[k2] w_32^(j1 k1).
// w_32 = 2^78, so the three 32-point DFTs are shift-only; two general
// multiplies per element.
//
// A workgroup of 1024 threads holds one row, 32 values per thread.  The two
// exchanges between the stages go through LDS in two rounds of half a row
// each (128 KiB; a whole row is 256 KiB).  Round r of the first exchange
// moves the pairs with k3h = j2b0 ^ r (k3h: bit 4 of k3, j2b0: bit 0 of j2);
// every thread writes 16 values and reads 16, into the register slots it
// has just written, because
//   - stage A's DFT leaves A[k3] in slot k3, so the 16 written are slots
//     [16 h, 16 h + 16) with h = j2b0 ^ r;
//   - stage B's DFT takes j2 in slot bitrev5(j2), so j2 with bit 0 = h fill
//     the same slots;
//   - bit 0 of the thread's stage-A j2 and bit 4 of its stage-B k3 are the
//     same bit of its wave index (role()).
// The second exchange does the same with k2b0 = j1h ^ r (k2 in natural slots,
// j1 in bit-reversed ones).  Every choice above depends on the wave only, so
// each wave takes one branch.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "gl64.hpp"
#include "gl64_shift.hpp"

namespace vmx {
namespace n15 {

constexpr int LOG_N = 15;
constexpr int N = 1 << LOG_N;
constexpr int THREADS = 1024;
// First exchange: word (k3l, j2, j1) at k3l X1_PITCH + 32 j2 + j1.  The pad
// puts the four k3l runs that one read instruction takes on different banks.
constexpr int X1_PITCH = 32 * 32 + 16;
// Second exchange: word (k2 >> 1, j1, k3) at (k2 >> 1) X2_BLOCK + X2_P j1 + k3.
// The odd pitch keeps the writes, 16 lanes of j1 per run, conflict-free.
constexpr int X2_P = 33;
constexpr int X2_BLOCK = 32 * X2_P;
constexpr int XBUF_WORDS = 16 * X2_BLOCK;
static_assert(16 * X1_PITCH <= XBUF_WORDS, "both exchanges share one buffer");
constexpr int T2_OFF = XBUF_WORDS;  // T2[k2 * 32 + j1] = w_1024^(j1 k2), 1024 words
constexpr int LDS_WORDS = T2_OFF + 1024;
constexpr size_t LDS_BYTES = size_t{LDS_WORDS} * sizeof(uint64_t);
// Device table: T1[k3 * 1024 + m] = w^(k3 m), then T2.
constexpr int T1_WORDS = 32 * 1024;
constexpr size_t TABLE_BYTES = size_t{T1_WORDS + 1024} * sizeof(uint64_t);

// Word idx of the device table from the reference's half table
// fwd = w^0 .. w^(n/2 - 1) (w^e = -w^(e - n/2)).
__host__ __device__ inline uint64_t table_word(const uint64_t* fwd, int idx) {
    const int e = idx < T1_WORDS ? (idx >> 10) * (idx & 1023) : 32 * ((idx - T1_WORDS) >> 5) * ((idx - T1_WORDS) & 31);
    return e < N / 2 ? fwd[e] : gl::neg(fwd[e - N / 2]);
}

// The three roles of thread t (wave w = t >> 6, lane = t & 63).
struct Role {
    int m;         // stage A: j1 + 32 j2, j1 = lane & 31, j2 = w + 16 (lane >> 5)
    int j1b, k3b;  // stage B
    int k3c, k2c;  // stage C
};

__host__ __device__ inline Role role(int t) {
    const int w = t >> 6, lane = t & 63;
    const int w0 = w & 1, w1 = (w >> 1) & 1, w23 = w >> 2;
    Role r;
    r.m = (lane & 31) + 32 * (w + 16 * (lane >> 5));
    r.j1b = (lane & 15) | (w1 << 4);
    r.k3b = (lane >> 4) | (w23 << 2) | (w0 << 4);
    r.k3c = lane & 31;
    r.k2c = w1 | ((lane >> 5) << 1) | (w0 << 2) | (w23 << 3);
    return r;
}

// Positions of a bit-reversed 32-slot array that hold j3 < NZ.
constexpr uint64_t prefix_mask(int nz) {
    uint64_t m = 0;
    for (int j = 0; j < nz; ++j) m |= uint64_t{1} << gl::bitrev_c(j, 5);
    return m;
}

// Device memory access.  The kernel reads through buffer resources: one
// 32-bit lane offset per access plus a scalar offset, so no 64-bit address
// stays live across the row loop, and a read past the resource's end returns
// 0 without touching memory (the zero tail costs no masking).  The host build
// reads through plain pointers with the same results.
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

// T1 of the device table (first-exchange twiddles).
struct Table1 {
#if defined(__HIP_DEVICE_COMPILE__)
    __amdgpu_buffer_rsrc_t r;
    __device__ explicit Table1(const uint64_t* tab) : r(rsrc(tab, TABLE_BYTES)) {}
    __device__ uint64_t at(int k3, int m) const {
        return ld64(r, static_cast<uint32_t>(m) * 8u, static_cast<uint32_t>(k3) * 8192u);
    }
#else
    const uint64_t* p;
    explicit Table1(const uint64_t* tab) : p(tab) {}
    uint64_t at(int k3, int m) const { return p[k3 * 1024 + m]; }
#endif
};

// Sources of stage A's inputs: element m + 1024 j3 of row `row`.  fetch()
// issues the load; value() turns what arrived into the field element, so a
// row's loads can be issued a row ahead.
// SrcU64: x + row stride, len u64 then zeros.
struct SrcU64 {
    const uint64_t* x;
    size_t stride, len;
    struct Raw {
        uint64_t v;
    };
    template <int J3>
    __host__ __device__ Raw fetch(size_t row, int m) const {
#if defined(__HIP_DEVICE_COMPILE__)
        return Raw{ld64(rsrc(x + row * stride, len * 8), static_cast<uint32_t>(m) * 8u, J3 * 8192u)};
#else
        const size_t idx = static_cast<size_t>(m) + 1024 * J3;
        return Raw{idx < len ? x[row * stride + idx] : 0};
#endif
    }
    template <int J3>
    __host__ __device__ uint64_t value(Raw r) const {
        return r.v;
    }
};

// SrcMsg: lift(w) || pads || 0 with cols = 1024 WB (reference
// pcs_messages_kernel, cuda/volta_cuda_backend.cu:2950-2958): blocks
// j3 < WB are i16 weights, block j3 >= WB starts at pad index
// 1024 (j3 - WB).  pads must point at a readable word even when pad = 0.
template <int WB>
struct SrcMsg {
    const int16_t* w;
    const uint64_t* pads;
    size_t cols, pad;
    struct Raw {
        uint64_t v;  // the i16 (j3 < WB) or the pad
    };
    template <int J3>
    __host__ __device__ Raw fetch(size_t row, int m) const {
#if defined(__HIP_DEVICE_COMPILE__)
        if constexpr (J3 < WB) {
            const uint32_t h = __builtin_amdgcn_raw_buffer_load_b16(rsrc(w + row * cols, cols * 2),
                                                                     static_cast<uint32_t>(m) * 2u, J3 * 2048u, 0);
            return Raw{h};
        } else {
            return Raw{ld64(rsrc(pads + row * pad, pad * 8), static_cast<uint32_t>(m) * 8u, (J3 - WB) * 8192u)};
        }
#else
        if constexpr (J3 < WB) {
            return Raw{static_cast<uint16_t>(w[row * cols + static_cast<size_t>(m) + 1024 * J3])};
        } else {
            const size_t pi = static_cast<size_t>(m) + 1024 * (J3 - WB);
            return Raw{pi < pad ? pads[row * pad + pi] : 0};
        }
#endif
    }
    template <int J3>
    __host__ __device__ uint64_t value(Raw r) const {
        if constexpr (J3 < WB) return gl::from_i16(static_cast<int16_t>(static_cast<uint16_t>(r.v)));
        else return r.v;
    }
};

template <int NZ, class Src>
__host__ __device__ __forceinline__ void fetch_row(const Src& s, size_t row, int m, typename Src::Raw* raw) {
    gl::static_for<0, NZ>([&](auto j_) {
        constexpr int j3 = decltype(j_)::value;
        raw[j3] = s.template fetch<j3>(row, m);
    });
}

// Stage A: the sparse 32-point DFT over j3; A[k3] in slot k3.
template <int NZ, class Src>
__host__ __device__ __forceinline__ void stage_a(uint64_t* v, const Src& s, const typename Src::Raw* raw) {
    gl::static_for<0, 32>([&](auto i_) { v[decltype(i_)::value] = 0; });
    gl::static_for<0, NZ>([&](auto j_) {
        constexpr int j3 = decltype(j_)::value;
        v[gl::bitrev_c(j3, 5)] = s.template value<j3>(raw[j3]);
    });
    gl::dit_pow2_sparse<5, gl::E_W32, prefix_mask(NZ)>(v);
}

// A distinct empty asm statement at both ends of each half's code: the two
// halves of an exchange differ only in which register slots they use, and
// without these the compiler merges them into one path that selects the
// slot at run time, which moves the whole register array into scratch memory.
template <int TAG>
__host__ __device__ __forceinline__ void fence_half() {
#if defined(__HIP_DEVICE_COMPILE__)
    if constexpr (TAG == 0) asm volatile("; ntt15 half 0");
    else if constexpr (TAG == 1) asm volatile("; ntt15 half 1");
    else if constexpr (TAG == 2) asm volatile("; ntt15 half 2");
    else if constexpr (TAG == 3) asm volatile("; ntt15 half 3");
    else if constexpr (TAG == 4) asm volatile("; ntt15 half 4");
    else if constexpr (TAG == 5) asm volatile("; ntt15 half 5");
    else if constexpr (TAG == 6) asm volatile("; ntt15 half 6");
    else asm volatile("; ntt15 half 7");
#endif
}

// The first-exchange twiddles w^(k3 m), k3 = 16 h + l for l in [L0, L0 + 8),
// of half h, a wave-uniform value, so one code path serves both halves.
template <int L0>
__host__ __device__ __forceinline__ void load_tw1(uint64_t* tw, const Table1& t1, int h, int m) {
    gl::static_for<0, 8>([&](auto l_) {
        constexpr int l = decltype(l_)::value;
        tw[l] = t1.at(16 * h + L0 + l, m);
    });
}

// First exchange, half H = j2b0 ^ r of a thread in role m: A[16 H + l] times
// w^(k3 m) to word (l, j2, j1).  tw holds the twiddles of l < 8 on entry; the
// other eight load while the first eight are written, so at most eight are
// held at a time beside the 32 values.
template <int H>
__host__ __device__ __forceinline__ void x1_write(uint64_t* lds, const uint64_t* v, uint64_t* tw, const Table1& t1,
                                                  int m) {
    fence_half<H>();
    gl::static_for<0, 16>([&](auto l_) {
        constexpr int l = decltype(l_)::value, k3 = 16 * H + l;
        if constexpr (l == 8) {
#if defined(__HIP_DEVICE_COMPILE__)
            __builtin_amdgcn_sched_barrier(0);
#endif
            load_tw1<8>(tw, t1, H, m);
        }
        lds[l * X1_PITCH + m] = k3 ? gl::mul32x4(v[k3], tw[l & 7]) : v[k3];
    });
    fence_half<H>();
}

// j2 = H + 2 i (i < 16) of a thread in role (j1, k3) into slot bitrev5(j2) = 16 H + bitrev4(i).
template <int H>
__host__ __device__ __forceinline__ void x1_read(const uint64_t* lds, uint64_t* v, int j1, int k3) {
    fence_half<2 + H>();
    const uint64_t* p = lds + (k3 & 15) * X1_PITCH + j1;
    gl::static_for<0, 16>([&](auto i_) {
        constexpr int i = decltype(i_)::value;
        v[16 * H + gl::bitrev_c(i, 4)] = p[32 * (H + 2 * i)];
    });
    fence_half<2 + H>();
}

// Second exchange, half G = j1h ^ r of a thread in role (j1, k3): B[k2]
// for k2 = G + 2 i times w_1024^(j1 k2) to word (i, j1, k3).
template <int G>
__host__ __device__ __forceinline__ void x2_write(uint64_t* lds, const uint64_t* v, int j1, int k3) {
    fence_half<4 + G>();
    uint64_t* p = lds + j1 * X2_P + k3;
    const uint64_t* t2 = lds + T2_OFF + j1;
    gl::static_for<0, 16>([&](auto i_) {
        constexpr int i = decltype(i_)::value, k2 = G + 2 * i;
        p[i * X2_BLOCK] = k2 ? gl::mul32x4(v[k2], t2[k2 * 32]) : v[k2];
    });
    fence_half<4 + G>();
}

// j1 = jl + 16 G (jl < 16) of a thread in role (k3, k2) into slot
// bitrev5(j1) = 2 bitrev4(jl) + G.
template <int G>
__host__ __device__ __forceinline__ void x2_read(const uint64_t* lds, uint64_t* v, int k3, int k2) {
    fence_half<6 + G>();
    const uint64_t* p = lds + (k2 >> 1) * X2_BLOCK + k3 + 16 * G * X2_P;
    gl::static_for<0, 16>([&](auto jl_) {
        constexpr int jl = decltype(jl_)::value;
        v[2 * gl::bitrev_c(jl, 4) + G] = p[jl * X2_P];
    });
    fence_half<6 + G>();
}

}  // namespace n15
}  // namespace vmx
