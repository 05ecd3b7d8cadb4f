// enc13_phase_b.hpp -- phase B of the n = 2^13 i16 encode (encode_fast.hip):
// the 64-point DFT over i2 of one row j1 of Y = X * w_n^(i2 j1), split by
// output parity H into its first radix-2 stage and one 32-point DFT.
//
// With S[q] = Y[q] + Y[q + 32] and D[q] = Y[q] - Y[q + 32] (q < 32; phase A
// stores them in place of Y), X[2k + H] = sum_q T_H[q] w32^(q k) with
// T_0[q] = S[q] and T_1[q] = D[q] w64^q, w64 = 2^39 and w32 = 2^78: every
// twiddle is a power of two.  The 32-point DFT is dit_pow2 on T in
// bit-reversed order.
#pragma once

#include <stdint.h>

#include "gl64.hpp"
#include "gl64_shift.hpp"

namespace enc13m {

// Parity H's 32 inputs T_H from the row's 32 words sd (S for H = 0, D for
// H = 1), in bit-reversed order.
template <int H>
__host__ __device__ __forceinline__ void phase_b_load(const uint64_t* sd, uint64_t* v) {
    gl::static_for<0, 32>([&](auto qq) {
        constexpr int q = decltype(qq)::value;
        if constexpr (H == 0) v[gl::bitrev_c(q, 5)] = sd[q];
        else v[gl::bitrev_c(q, 5)] = gl::mul_pow2<gl::E_W64 * q>(sd[q]);
    });
}

// Parity 1's pre-twiddle applied in place, to S-or-D words loaded as for
// parity 0: v[bitrev q] = D[q] -> D[q] w64^q.
__host__ __device__ __forceinline__ void phase_b_twiddle(uint64_t* v) {
    gl::static_for<1, 32>([&](auto qq) {
        constexpr int q = decltype(qq)::value;
        v[gl::bitrev_c(q, 5)] = gl::mul_pow2<gl::E_W64 * q>(v[gl::bitrev_c(q, 5)]);
    });
}

// The 32-point DFT: v[k] = X[2k + H].
__host__ __device__ __forceinline__ void phase_b_dft(uint64_t* v) { gl::dit_pow2<5, gl::E_W32>(v); }

}  // namespace enc13m
