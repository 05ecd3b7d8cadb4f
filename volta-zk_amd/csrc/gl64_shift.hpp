// gl64_shift.hpp -- Goldilocks multiply-by-power-of-two and the small DFTs
// built on it.
//
// 2 has multiplicative order 192 mod p (2^96 = -1), and the reference's roots
// of unity of order <= 64 are all powers of 2:
//     w_64 = 7^((p-1)/64) = 2^39,  w_32 = 2^78,  w_16 = 2^156,  w_8 = 2^120,
//     w_4 = 2^48,  w_2 = 2^96 = -1,  and  w_128 = 2^43 - 2^91.
// (checked by tests/test_fast_constants.py against 7^((p-1)/2^k)).
// So every twiddle inside a DFT of length <= 64 is a shift followed by a
// fold of the 128-bit result; no 64x64 product is needed.  All exponents are
// template parameters, so after unrolling each butterfly is straight-line
// code with immediate shift counts.
#pragma once

#include <type_traits>

#include "gl64.hpp"

namespace gl {

constexpr int E_W64 = 39;  // w_64 = 2^39
constexpr int E_W32 = 78;  // w_32 = 2^78

// x * 2^S mod p for 0 <= S < 96, x canonical; canonical result.
template <int S>
__host__ __device__ __forceinline__ uint64_t shl_mod(uint64_t x) {
    static_assert(S >= 0 && S < 96, "shift out of range");
    if constexpr (S == 0) {
        return x;
    } else if constexpr (S < 64) {
        return fold128(x << S, x >> (64 - S));
    } else if constexpr (S == 64) {
        return fold128(0, x);
    } else {
        // x*2^S = y*2^64 with y = x*2^(S-64) = yhi*2^64 + ylo, yhi < 2^32;
        // y*2^64 = ylo*2^64 + yhi*2^128 = ylo*eps - yhi*2^32 (2^128 = -2^32).
        const uint64_t ylo = x << (S - 64);
        const uint64_t yhi = x >> (128 - S);
        return sub(fold128(0, ylo), yhi << 32);  // yhi << 32 <= 2^64 - 2^32 < p
    }
}

// x * 2^E mod p for any E >= 0 (reduced mod 192; E mod 192 >= 96 negates).
template <int E>
__host__ __device__ __forceinline__ uint64_t mul_pow2(uint64_t x) {
    constexpr int e = E % 192;
    if constexpr (e >= 96) return neg(shl_mod<e - 96>(x));
    else return shl_mod<e>(x);
}

// DIT butterfly (u, v) <- (u + w v, u - w v) with w = 2^E.
template <int E>
__host__ __device__ __forceinline__ void bfly_pow2(uint64_t& u, uint64_t& v) {
    constexpr int e = E % 192;
    if constexpr (e == 0) {
        const uint64_t a = add(u, v), b = sub(u, v);
        u = a;
        v = b;
    } else if constexpr (e == 96) {
        const uint64_t a = sub(u, v), b = add(u, v);
        u = a;
        v = b;
    } else if constexpr (e < 96) {
        const uint64_t t = shl_mod<e>(v);
        const uint64_t a = add(u, t), b = sub(u, t);
        u = a;
        v = b;
    } else {
        // w = -2^(e-96): swap the roles of sum and difference
        const uint64_t t = shl_mod<e - 96>(v);
        const uint64_t a = sub(u, t), b = add(u, t);
        u = a;
        v = b;
    }
}

// Field element of a * 2^S for |a| <= 2^15 (a signed), 0 <= S < 96.
template <int S>
__host__ __device__ __forceinline__ uint64_t small_shl_abs(uint32_t ax) {
    if constexpr (S + 16 <= 63) {
        return static_cast<uint64_t>(ax) << S;  // < 2^63 < p
    } else if constexpr (S < 64) {
        return fold128(static_cast<uint64_t>(ax) << S, static_cast<uint64_t>(ax) >> (64 - S));
    } else {
        return shl_mod<S>(static_cast<uint64_t>(ax));
    }
}

// Field element of x * 2^E for a signed 16-bit x (any E >= 0).
template <int E>
__host__ __device__ __forceinline__ uint64_t i16_mul_pow2(int32_t x) {
    constexpr int e = E % 192;
    constexpr bool flip = e >= 96;
    const uint32_t ax = static_cast<uint32_t>(x < 0 ? -x : x);
    const uint64_t m = small_shl_abs<flip ? e - 96 : e>(ax);
    const bool negate = (x < 0) != flip;
    return negate ? neg(m) : m;
}

// Field element of x * w_128^k for a signed 16-bit x: w_128^k = 2^(39 k/2)
// for even k; 2^(43+c) - 2^(91+c) with c = 39 (k-1)/2 for odd k.
template <int K>
__host__ __device__ __forceinline__ uint64_t i16_mul_w128(int32_t x) {
    if constexpr (K % 2 == 0) {
        return i16_mul_pow2<E_W64 * (K / 2)>(x);
    } else {
        constexpr int c = E_W64 * ((K - 1) / 2);
        return sub(i16_mul_pow2<43 + c>(x), i16_mul_pow2<91 + c>(x));
    }
}

// ---- unrolled small DFTs on register arrays -------------------------------

template <int I>
using ic = std::integral_constant<int, I>;

// Compile-time loop: f(ic<B>), f(ic<B+1>), ..., f(ic<E-1>).
template <int B, int E, class F>
__host__ __device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(ic<B>{});
        static_for<B + 1, E>(f);
    }
}

// In-place radix-2 DIT DFT of length N = 2^LOG with root 2^EW on v[], which
// holds the input in bit-reversed order; output in natural order.
template <int LOG, int EW, int LEN = 2>
__host__ __device__ __forceinline__ void dit_pow2(uint64_t* v) {
    if constexpr (LEN <= (1 << LOG)) {
        constexpr int N = 1 << LOG;
        constexpr int HALF = LEN / 2;
        static_for<0, N / LEN>([&](auto g) {
            constexpr int start = decltype(g)::value * LEN;
            static_for<0, HALF>([&](auto kk) {
                constexpr int k = decltype(kk)::value;
                // w_LEN^k = w_N^(k N/LEN) = 2^(EW k N/LEN)
                bfly_pow2<EW * k * (N / LEN)>(v[start + k], v[start + k + HALF]);
            });
        });
        dit_pow2<LOG, EW, LEN * 2>(v);
    }
}

// Bit reversal of I over LOG bits, at compile time.
constexpr int bitrev_c(int i, int log) {
    int r = 0;
    for (int b = 0; b < log; ++b) r |= ((i >> b) & 1) << (log - 1 - b);
    return r;
}

}  // namespace gl
