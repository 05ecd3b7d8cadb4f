// enc13_mfma.hpp -- phase A of the n = 2^13 i16 encode (encode_fast.hip) as an
// exact int8 matrix product on the matrix cores (v_mfma_i32_16x16x64_i8).
//
// Phase A computes, for each column i2 < 64 and output j1 < 128,
//   X[j1][i2] = sum_{i1 < 32} x[64 i1 + i2] W(i1, j1),  W(i1, j1) = w128^(i1 j1),
// where x is a signed 16-bit message entry.
//
// Operands.  Each x splits into two signed bytes, x = 256 d1 + d0 + 128 with
// d0 = (x & 255) - 128 and d1 = x >> 8: the 16-bit pattern x ^ 0x80 holds them
// as little-endian bytes.  Each field element c has a balanced base-256 form
// sum_{pos < 8} e_pos 256^pos with every e_pos in [-128, 127]: c itself when
// c <= 0x7F7F7F7F7F7F7F7F (= 127 (256^8 - 1) / 255), else c - p.  Then with
//   A[(j1, pos)][(i1, d)] = e_pos(W(i1, j1) 256^d mod p)     (K = 32 x 2 = 64)
//   B[(i1, d)][i2] = d_d(x[64 i1 + i2])
// the products a_pos = init[j1][pos] + sum_k A B satisfy
//   sum_pos a_pos 256^pos = sum_i1 (x - 128) W + sum_pos init 256^pos (mod p).
// The init words restore 128 sum_{i1 < 32} W(i1, j1) (zero-tail entries read as
// x = 0 and are covered by the same sum) and add a fixed vector whose value is a
// multiple of p and whose entries lie in [2^20, 2^20 + 256), so every a_pos is
// in [0, 2^21 + 2^9): |sum_k A B| <= 64 x 128 x 128 = 2^20.  `recombine` folds
// the eight sums to a field element.
//
// Layouts (lane l of a wave; m = l & 15, grp = l >> 4), as the instruction
// places them (lane l holds A[l & 15][16 grp + j] and B[16 grp + j][l & 15], j
// < 16; register r of D holds C[4 grp + r][l & 15]):
//   A fragment of pair q = 0..31, half h: row m = 4 g + r is (j1 = 4 q + g,
//     pos = 4 h + r); K slot 16 grp + j is (i1 = 8 grp + j / 2, d = j & 1);
//   B fragment of column tile t: column m is i2 = 16 t + m;
//   D register r of half h, lane l: position 4 h + r of output
//     (j1 = 4 q + grp, i2 = 16 t + m), so one lane holds all 8 positions.
#pragma once

#include <stdint.h>

#include "gl64.hpp"

namespace enc13m {

constexpr int WAVES = 4, PAIRS = 8;                                  // pairs (of 4 outputs j1) per wave
constexpr size_t FRAG_BYTES = size_t{WAVES} * PAIRS * 2 * 64 * 16;  // A fragments of all 32 pairs
constexpr size_t INIT_WORDS = 128 * 8;                             // init[j1][pos], int32
constexpr uint64_t BAL_MAX = 0x7F7F7F7F7F7F7F7Full;                 // 127 (256^8 - 1) / 255

// Digit pos of the balanced base-256 form of the canonical field element c.
__host__ __device__ inline int balanced_digit(uint64_t c, int pos) {
    __int128 s = c <= BAL_MAX ? static_cast<__int128>(c) : static_cast<__int128>(c) - static_cast<__int128>(gl::P);
    int d = 0;
    for (int i = 0; i <= pos; ++i) {
        d = static_cast<int>(static_cast<int64_t>((s + 128) & 255)) - 128;
        s = (s - d) >> 8;  // exact: s - d is a multiple of 256
    }
    return d;
}

// bias[pos] = 2^20 + byte pos of (-X0 mod p), X0 = sum_pos 2^20 256^pos =
// 2^20 (256^8 - 1) / 255: the vector's value X0 + (-X0 mod p) is a multiple of p.
__host__ __device__ inline int bias_digit(int pos) {
    const uint64_t r = gl::mul(0x0101010101010101ull, uint64_t{1} << 20);  // X0 mod p
    const uint64_t dlt = r ? gl::P - r : 0;                                 // -X0 mod p
    return (1 << 20) + static_cast<int>((dlt >> (8 * pos)) & 255);
}

// W(i1, j1) = w^e, e = 64 i1 j1 mod 2^13, from the half table w^0 .. w^4095
// (w^e = -w^(e - 4096)).
__host__ __device__ inline uint64_t w_of(const uint64_t* tw_half, int i1, int j1) {
    const int e = (64 * i1 * j1) & 8191;
    return e < 4096 ? tw_half[e] : gl::neg(tw_half[e - 4096]);
}

// The 16 bytes of A fragment idx = (q 2 + h) 64 + l.
__host__ __device__ inline void a_fragment(const uint64_t* tw_half, int idx, int8_t* out16) {
    const int l = idx & 63, h = (idx >> 6) & 1, q = idx >> 7;
    const int m = l & 15, grp = l >> 4;
    const int j1 = 4 * q + (m >> 2), pos = 4 * h + (m & 3);
    for (int j = 0; j < 16; ++j) {
        const int i1 = 8 * grp + (j >> 1), d = j & 1;
        uint64_t v = w_of(tw_half, i1, j1);
        if (d) v = gl::mul(v, 256);
        out16[j] = static_cast<int8_t>(balanced_digit(v, pos));
    }
}

// init[j1][pos]: the balanced digits of 128 sum_{i1 < 32} W(i1, j1), plus the bias.
__host__ __device__ inline int init_word(const uint64_t* tw_half, int j1, int pos) {
    uint64_t s = 0;
    for (int i1 = 0; i1 < 32; ++i1) s = gl::add(s, w_of(tw_half, i1, j1));
    return balanced_digit(gl::mul(s, 128), pos) + bias_digit(pos);
}

// sum_pos a_pos 256^pos (mod p) for a_pos in [0, 2^21 + 2^9): a u64
// representative, not necessarily below p (gl::mul32x4 takes any u64).
// Adjacent positions pair into 32-bit sums b < 2^30, so V = L + H 2^32 with
// L = b0 + b1 2^16 and H = b2 + b3 2^16 below 2^47; then V = lo + hi 2^64 with
// hi < 2^16, and 2^64 = 2^32 - 1 (mod p).  14 VALU instructions on gfx950.
// k16 = 2^16 and keps = 2^32 - 1 come in as run-time values (kernel
// arguments): as constants the compiler turns the products into 64-bit shifts
// and adds, 8 more instructions per fold than the multiply-adds.
__host__ __device__ __forceinline__ uint64_t recombine(const int* a /* pos 0..3 */, const int* b /* pos 4..7 */,
                                                       uint32_t k16 = 65536u, uint32_t keps = 0xFFFFFFFFu) {
    const uint32_t b0 = static_cast<uint32_t>(a[0]) + (static_cast<uint32_t>(a[1]) << 8);
    const uint32_t b1 = static_cast<uint32_t>(a[2]) + (static_cast<uint32_t>(a[3]) << 8);
    const uint32_t b2 = static_cast<uint32_t>(b[0]) + (static_cast<uint32_t>(b[1]) << 8);
    const uint32_t b3 = static_cast<uint32_t>(b[2]) + (static_cast<uint32_t>(b[3]) << 8);
    const uint64_t L = static_cast<uint64_t>(b1) * k16 + b0;  // one 32 x 32 + 64 multiply-add each
    const uint64_t H = static_cast<uint64_t>(b3) * k16 + b2;
    // lo = L + (H mod 2^32) 2^32, hi = (H >> 32) + its carry: V = lo + hi 2^64
    unsigned c;
    const uint32_t lo_hi = __builtin_addc(static_cast<uint32_t>(L >> 32), static_cast<uint32_t>(H), 0u, &c);
    const uint32_t hi = static_cast<uint32_t>(H >> 32) + c;
    const uint64_t lo = (static_cast<uint64_t>(lo_hi) << 32) | static_cast<uint32_t>(L);
    const uint64_t r = static_cast<uint64_t>(hi) * keps + lo;  // 2^64 = eps
    return r < lo ? static_cast<uint64_t>(1u) * keps + r : r;  // a carry out of 2^64 is worth eps, once
}

}  // namespace enc13m
