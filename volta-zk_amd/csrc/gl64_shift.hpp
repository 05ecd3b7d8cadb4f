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

// x * 2^-M mod p for 1 <= M <= 32, x canonical; canonical result.
// With x = q 2^M + r (r < 2^M): x 2^-M = q + r 2^-M and 2^-M = -2^(96-M), so
// x 2^-M = q - r 2^(32-M) 2^64 = q - r' eps with r' = r 2^(32-M) < 2^32; both
// q < 2^(64-M) and r' eps <= (2^32-1)^2 are canonical.
template <int M>
__host__ __device__ __forceinline__ uint64_t shr_mod(uint64_t x) {
    static_assert(M >= 1 && M <= 32, "shift out of range");
    const uint64_t q = x >> M;
    const uint32_t rp = static_cast<uint32_t>(x) << (32 - M);
    return sub(q, static_cast<uint64_t>(rp) * EPS);
}

// x * 2^(32+SM) mod p for 0 <= SM < 32, x canonical; canonical result.
// In 32-bit words x 2^SM = W1 + W2 2^32 + W3 2^64, so x 2^(32+SM) =
// W1 2^32 + W2 2^64 + W3 2^96 = (W1 + W2) 2^32 - (W2 + W3)  (2^64 = 2^32 - 1,
// 2^96 = -1): two 32-bit sums and one borrow-corrected 64-bit difference.
template <int SM>
__host__ __device__ __forceinline__ uint64_t shl_mod_hi(uint64_t x) {
    static_assert(SM >= 0 && SM < 32, "shift out of range");
    const uint32_t x0 = static_cast<uint32_t>(x), x1 = static_cast<uint32_t>(x >> 32);
    uint32_t w1, w2, w3;
    if constexpr (SM == 0) {
        w1 = x0;
        w2 = x1;
        w3 = 0;
    } else {
        w1 = x0 << SM;
        w2 = (x1 << SM) | (x0 >> (32 - SM));
        w3 = x1 >> (32 - SM);
    }
    unsigned ca, cb, c2, b0, b1;
    const uint32_t a = __builtin_addc(w1, w2, 0u, &ca);  // A = a + ca 2^32
    const uint32_t b = __builtin_addc(w2, w3, 0u, &cb);  // B = b + cb 2^32 < 2^32 + 2^31
    const uint32_t h = a + ca;                           // A 2^32 = (a + ca) 2^32 - ca
    const uint32_t clo = __builtin_addc(b, 0u, ca, &c2); // C = B + ca = clo + chi 2^32
    const uint32_t chi = cb | c2;
    const uint32_t r0 = __builtin_subc(0u, clo, 0u, &b0);  // r = h 2^32 - C
    const uint32_t r1 = __builtin_subc(h, chi, b0, &b1);
    const uint64_t r = pack64(r0, r1);
    return b1 ? r - EPS : r;  // negative: + p = - eps mod 2^64
}

// x * 2^S mod p for 0 <= S < 96, x canonical; canonical result.
template <int S>
__host__ __device__ __forceinline__ uint64_t shl_mod(uint64_t x) {
    static_assert(S >= 0 && S < 96, "shift out of range");
    if constexpr (S == 0) {
        return x;
    } else if constexpr (S < 32) {
        return fold96(x << S, static_cast<uint32_t>(x >> (64 - S)));
    } else if constexpr (S < 64) {
        return shl_mod_hi<S - 32>(x);
    } else {
        // 2^S = -2^-(96-S): one division by a power of two <= 2^32.
        return neg(shr_mod<96 - S>(x));
    }
}

// -(x * 2^S) mod p for 64 <= S < 96 without the final negation.
template <int S>
__host__ __device__ __forceinline__ uint64_t shl_mod_neg(uint64_t x) {
    static_assert(S >= 64 && S < 96, "only the division form has a cheap negative");
    return shr_mod<96 - S>(x);
}

// x * 2^E up to sign, in its cheapest form: with S = (E mod 192) mod 96,
// 2^E = +-2^S, and for S >= 64 the division form yields -(x 2^S) directly.
// pow2_neg(E) tells whether the result holds -(x 2^E) rather than x 2^E.
constexpr bool pow2_neg(int E) {
    const int e = E % 192;
    return (e >= 96) != (e % 96 >= 64);
}

template <int E>
__host__ __device__ __forceinline__ uint64_t mul_pow2_signed(uint64_t x) {
    constexpr int S = (E % 192) % 96;
    if constexpr (S >= 64) return shr_mod<96 - S>(x);
    else return shl_mod<S>(x);
}

// x * 2^E mod p for any E >= 0.
template <int E>
__host__ __device__ __forceinline__ uint64_t mul_pow2(uint64_t x) {
    const uint64_t t = mul_pow2_signed<E>(x);
    if constexpr (pow2_neg(E)) return neg(t);
    else return t;
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
    } else {
        // w = +-2^S with S = e mod 96; for S >= 64 the division form yields
        // -(v 2^S) directly, which flips the sign once more.
        constexpr int S = e % 96;
        constexpr bool neg_w = e >= 96;
        uint64_t t;
        bool neg_t;
        if constexpr (S >= 64) {
            t = shl_mod_neg<S>(v);
            neg_t = !neg_w;
        } else {
            t = shl_mod<S>(v);
            neg_t = neg_w;
        }
        if (neg_t) {
            const uint64_t a = sub(u, t), b = add(u, t);
            u = a;
            v = b;
        } else {
            const uint64_t a = add(u, t), b = sub(u, t);
            u = a;
            v = b;
        }
    }
}

// Field element of a signed 64-bit integer y with |y| < 2^63: y, or y + p
// for y < 0.  In two's complement y + p = (2^64 + y) - eps, and the sign word
// y >> 63 read as an unsigned 32-bit value is eps exactly when y < 0.
__host__ __device__ __forceinline__ uint64_t from_i64(uint64_t y) {
    const uint32_t m = static_cast<uint32_t>(static_cast<int32_t>(static_cast<uint32_t>(y >> 32)) >> 31);
    return y - m;
}

// Field element of a * 2^S for |a| <= 2^15 (a signed), 0 <= S < 96.
template <int S>
__host__ __device__ __forceinline__ uint64_t small_shl_abs(uint32_t ax) {
    if constexpr (S + 16 <= 63) {
        return static_cast<uint64_t>(ax) << S;  // < 2^63 < p
    } else if constexpr (S < 64) {
        return fold96(static_cast<uint64_t>(ax) << S, static_cast<uint32_t>(static_cast<uint64_t>(ax) >> (64 - S)));
    } else {
        return shl_mod<S>(static_cast<uint64_t>(ax));
    }
}

// Field element of x * 2^E for a signed 16-bit x (any E >= 0).  Up to a
// shift of 47 the product +-x 2^s is an exact signed 64-bit integer
// (|x| <= 2^15), so one sign fix-up replaces the modular reduction.
template <int E>
__host__ __device__ __forceinline__ uint64_t i16_mul_pow2(int32_t x) {
    constexpr int e = E % 192;
    constexpr bool flip = e >= 96;
    constexpr int s = flip ? e - 96 : e;
    if constexpr (s <= 47) {
        const uint64_t v = static_cast<uint64_t>(static_cast<int64_t>(flip ? -x : x));
        return from_i64(v << s);
    } else {
        const uint32_t ax = static_cast<uint32_t>(x < 0 ? -x : x);
        const uint64_t m = small_shl_abs<s>(ax);
        const bool negate = (x < 0) != flip;
        return negate ? neg(m) : m;
    }
}

// Field element of x * w_128^k for a signed 16-bit x: w_128^k = 2^(39 k/2)
// for even k; 2^(43+c) - 2^(91+c) = 2^(43+c) (1 - 2^48) with c = 39 (k-1)/2
// for odd k.  x (1 - 2^48) is an exact signed 64-bit integer (|x| <= 2^15),
// so the odd case is one sign fix-up and one modular shift.
template <int K>
__host__ __device__ __forceinline__ uint64_t i16_mul_w128(int32_t x) {
    if constexpr (K % 2 == 0) {
        return i16_mul_pow2<E_W64 * (K / 2)>(x);
    } else {
        constexpr int c = E_W64 * ((K - 1) / 2);
        const uint64_t v = static_cast<uint64_t>(static_cast<int64_t>(x));
        return mul_pow2<43 + c>(from_i64(v - (v << 48)));
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

// The positions that may be nonzero after a stage of span LEN of dit_pow2
// whose input may be nonzero at the positions in m: both of a pair, if either.
constexpr uint64_t dit_mask_next(uint64_t m, int len, int n) {
    uint64_t r = 0;
    const int half = len / 2;
    for (int s = 0; s < n; s += len)
        for (int k = 0; k < half; ++k)
            if (((m >> (s + k)) | (m >> (s + k + half))) & 1) r |= (uint64_t{1} << (s + k)) | (uint64_t{1} << (s + k + half));
    return r;
}

// dit_pow2 for an input that is known to be zero outside the positions set in
// MASK (bit i: v[i] may be nonzero; the other positions must hold 0).  A
// butterfly whose second input is known zero is the copy (u, u), one whose
// inputs are both known zero is skipped, so a zero tail of the input costs no
// arithmetic in the stages it reaches.  Runs the stages of spans LEN, 2 LEN,
// ... below STOP (all of them by default).
template <int LOG, int EW, uint64_t MASK, int LEN = 2, int STOP = (2 << LOG)>
__host__ __device__ __forceinline__ void dit_pow2_sparse(uint64_t* v) {
    if constexpr (LEN <= (1 << LOG) && LEN < STOP) {
        constexpr int N = 1 << LOG;
        constexpr int HALF = LEN / 2;
        static_for<0, N / LEN>([&](auto g) {
            constexpr int start = decltype(g)::value * LEN;
            static_for<0, HALF>([&](auto kk) {
                constexpr int k = decltype(kk)::value;
                constexpr bool nz_u = (MASK >> (start + k)) & 1, nz_v = (MASK >> (start + k + HALF)) & 1;
                if constexpr (nz_v) {
                    bfly_pow2<EW * k * (N / LEN)>(v[start + k], v[start + k + HALF]);
                } else if constexpr (nz_u) {
                    v[start + k + HALF] = v[start + k];
                }
            });
        });
        dit_pow2_sparse<LOG, EW, dit_mask_next(MASK, LEN, N), LEN * 2, STOP>(v);
    }
}

// Bit reversal of I over LOG bits, at compile time.
constexpr int bitrev_c(int i, int log) {
    int r = 0;
    for (int b = 0; b < log; ++b) r |= ((i >> b) & 1) << (log - 1 - b);
    return r;
}

}  // namespace gl
