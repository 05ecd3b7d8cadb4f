// gl64.hpp -- Goldilocks field arithmetic for gfx950 (device) and the host.
//
// p = 2^64 - 2^32 + 1.  Elements are u64; "canonical" means in [0, p).
// The identities used are 2^64 = 2^32 - 1 = eps (mod p) and 2^96 = -1 (mod p),
// the same ones the reference's field uses (rust/volta-field/src/lib.rs:89-103).
//
// The device multiply forms the 128-bit product from four 32x32->64 partial
// products (v_mad_u64_u32 on gfx950) and folds the high half with the two
// identities above; no MFMA, no 64-bit hardware multiply exists on the VALU.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gl {

constexpr uint64_t P = 0xFFFFFFFF00000001ull;
constexpr uint64_t EPS = 0x00000000FFFFFFFFull;

// A 64-bit value from two 32-bit words, kept as one register pair on the
// device: written as (hi << 32) | lo, the compiler reads the OR as an add of
// disjoint halves and splits a later 64-bit add into two adds of zero-extended
// halves (an extra add and a register copy each time).
__host__ __device__ __forceinline__ uint64_t pack64(uint32_t lo, uint32_t hi) {
    uint64_t r = (static_cast<uint64_t>(hi) << 32) | lo;
#if defined(__HIP_DEVICE_COMPILE__)
    asm("" : "+v"(r));
#endif
    return r;
}

// ---- host/device scalar ops (canonical in, canonical out) ---------------

__host__ __device__ __forceinline__ uint64_t canon(uint64_t x) { return x >= P ? x - P : x; }

// t = a + b and s = t + eps (mod 2^64).  s wraps past 2^64 exactly when
// a + b >= p (b + eps < 2^64 for b < p), and then s = a + b - p < a; otherwise
// s >= a and the sum is t.  Two 64-bit adds, one compare, one select.
__host__ __device__ __forceinline__ uint64_t add(uint64_t a, uint64_t b) {
    const uint64_t t = a + b;
    const uint64_t s = t + EPS;
    return s < a ? s : t;
}

// d = a - b; a borrow out of 64 bits is worth -2^64 = -eps, i.e. d - eps,
// which stays >= 0 for canonical inputs.
__host__ __device__ __forceinline__ uint64_t sub(uint64_t a, uint64_t b) {
    unsigned b0, b1, e0;
    const uint32_t d0 = __builtin_subc(static_cast<uint32_t>(a), static_cast<uint32_t>(b), 0u, &b0);
    const uint32_t d1 = __builtin_subc(static_cast<uint32_t>(a >> 32), static_cast<uint32_t>(b >> 32), b0, &b1);
    const uint32_t e = b1 ? 0xFFFFFFFFu : 0u;
    const uint32_t r0 = __builtin_subc(d0, e, 0u, &e0);
    const uint32_t r1 = d1 - e0;
    return pack64(r0, r1);
}

__host__ __device__ __forceinline__ uint64_t neg(uint64_t a) { return a ? P - a : 0; }

// Fold a 128-bit value (hi:lo) to a canonical element:
// hi:lo = lo + hl 2^64 + hh 2^96 = lo + hl eps - hh (mod p).
#if defined(__HIP_DEVICE_COMPILE__)
// gfx950: t = lo - hh (mod p) as a borrow chain; then one v_mad_u64_u32
// forms r = t + hl eps and its carry out of 2^64, which the compiler has no
// way to read (it would recompute the product and compare).  A carry is
// worth eps, and r < 2^64 - 2^33 + 1 when it is set, so r + eps is then
// already canonical; without it r + eps is r - p exactly when r >= p, which
// the carry out of r + eps reports.  Hence the result is r + eps when either
// carry is set, else r: 10 VALU instructions and one SALU or, against 16.
// The s_nop lines are the two wait states gfx950 needs between a VALU write
// of VCC and a VALU read of it (the compiler inserts the same); a SALU read
// of a VALU-written mask and a VALU read of a SALU-written one need none.
__device__ __forceinline__ uint64_t fold128(uint64_t lo, uint64_t hi) {
    const uint32_t hh = static_cast<uint32_t>(hi >> 32), hl = static_cast<uint32_t>(hi);
    // t = lo - hh, and eps less when that borrows (t stays >= 0 then)
    uint32_t t0, t1, e;
    asm("v_sub_co_u32 %0, vcc, %3, %5\n\t"
        "s_nop 1\n\t"
        "v_subbrev_co_u32 %1, vcc, 0, %4, vcc\n\t"
        "s_nop 1\n\t"
        "v_cndmask_b32 %2, 0, -1, vcc\n\t"
        "v_sub_co_u32 %0, vcc, %0, %2\n\t"
        "s_nop 1\n\t"
        "v_subbrev_co_u32 %1, vcc, 0, %1, vcc"
        : "=&v"(t0), "=&v"(t1), "=&v"(e)
        : "v"(static_cast<uint32_t>(lo)), "v"(static_cast<uint32_t>(lo >> 32)), "v"(hh)
        : "vcc");
    const uint64_t t = (static_cast<uint64_t>(t1) << 32) | t0;
    uint64_t r, c;
    asm("v_mad_u64_u32 %0, %1, %2, -1, %3" : "=v"(r), "=s"(c) : "v"(hl), "v"(t));
    const uint32_t r0 = static_cast<uint32_t>(r), r1 = static_cast<uint32_t>(r >> 32);
    uint32_t s0, s1;
    asm("v_add_co_u32 %0, vcc, -1, %2\n\t"
        "s_nop 1\n\t"
        "v_addc_co_u32 %1, vcc, 0, %3, vcc\n\t"
        "s_or_b64 vcc, vcc, %4\n\t"
        "v_cndmask_b32 %0, %2, %0, vcc\n\t"
        "v_cndmask_b32 %1, %3, %1, vcc"
        : "=&v"(s0), "=&v"(s1)
        : "v"(r0), "v"(r1), "s"(c)
        : "vcc", "scc");
    return pack64(s0, s1);
}
#else
__host__ __forceinline__ uint64_t fold128(uint64_t lo, uint64_t hi) {
    const uint64_t hh = hi >> 32;
    const uint64_t hl = hi & EPS;
    uint64_t t = lo - hh;               // lo - hh*2^96
    t -= (lo < hh) ? EPS : 0;           // borrow of 2^64 = eps
    const uint64_t m = (hl << 32) - hl; // hl * eps < 2^64
    uint64_t r = t + m;
    r += (r < m) ? EPS : 0;             // carry of 2^64 = eps
    return r >= P ? r - P : r;
}
#endif

// Fold hi 2^64 + lo for hi < 2^32 (hi 2^64 = hi eps): fold128 without the
// hh 2^96 term, 5 VALU instructions fewer on the device.
#if defined(__HIP_DEVICE_COMPILE__)
__device__ __forceinline__ uint64_t fold96(uint64_t lo, uint32_t hi) {
    uint64_t r, c;
    asm("v_mad_u64_u32 %0, %1, %2, -1, %3" : "=v"(r), "=s"(c) : "v"(hi), "v"(lo));
    const uint32_t r0 = static_cast<uint32_t>(r), r1 = static_cast<uint32_t>(r >> 32);
    uint32_t s0, s1;
    asm("v_add_co_u32 %0, vcc, -1, %2\n\t"
        "s_nop 1\n\t"
        "v_addc_co_u32 %1, vcc, 0, %3, vcc\n\t"
        "s_or_b64 vcc, vcc, %4\n\t"
        "v_cndmask_b32 %0, %2, %0, vcc\n\t"
        "v_cndmask_b32 %1, %3, %1, vcc"
        : "=&v"(s0), "=&v"(s1)
        : "v"(r0), "v"(r1), "s"(c)
        : "vcc", "scc");
    return pack64(s0, s1);
}
#else
__host__ __forceinline__ uint64_t fold96(uint64_t lo, uint32_t hi) { return fold128(lo, hi); }
#endif

#if defined(__HIP_DEVICE_COMPILE__)
__device__ __forceinline__ void mul_wide(uint64_t a, uint64_t b, uint64_t& lo, uint64_t& hi) {
    lo = a * b;
    hi = __umul64hi(a, b);
}
#else
inline void mul_wide(uint64_t a, uint64_t b, uint64_t& lo, uint64_t& hi) {
    const unsigned __int128 p = static_cast<unsigned __int128>(a) * b;
    lo = static_cast<uint64_t>(p);
    hi = static_cast<uint64_t>(p >> 64);
}
#endif

__host__ __device__ __forceinline__ uint64_t mul(uint64_t a, uint64_t b) {
    uint64_t lo, hi;
    mul_wide(a, b, lo, hi);
    return fold128(lo, hi);
}

// The same product from four 32x32->64 partial products, each of which maps
// onto one v_mad_u64_u32 on gfx950 (no carries can overflow: every partial
// sum stays below 2^64).
__host__ __device__ __forceinline__ uint64_t mul32x4(uint64_t a, uint64_t b) {
    const uint32_t a0 = static_cast<uint32_t>(a), a1 = static_cast<uint32_t>(a >> 32);
    const uint32_t b0 = static_cast<uint32_t>(b), b1 = static_cast<uint32_t>(b >> 32);
    const uint64_t p00 = static_cast<uint64_t>(a0) * b0;
    const uint64_t p01 = static_cast<uint64_t>(a0) * b1 + (p00 >> 32);
    const uint64_t p10 = static_cast<uint64_t>(a1) * b0 + static_cast<uint32_t>(p01);
    const uint64_t hi = static_cast<uint64_t>(a1) * b1 + (p01 >> 32) + (p10 >> 32);
    const uint64_t lo = (p10 << 32) | static_cast<uint32_t>(p00);
    return fold128(lo, hi);
}

inline uint64_t pow_host(uint64_t a, uint64_t e) {
    uint64_t acc = 1;
    while (e) {
        if (e & 1) acc = mul(acc, a);
        a = mul(a, a);
        e >>= 1;
    }
    return acc;
}

inline uint64_t inv_host(uint64_t a) { return pow_host(a, P - 2); }

// Primitive 2^bits-th root of unity 7^((p-1) >> bits): the generator and
// 2-adicity of the reference's NTT (rust/volta-pcs/src/ntt.rs:9-12).
inline uint64_t root_of_unity(unsigned bits) { return pow_host(7, (P - 1) >> bits); }

// i16 -> field: non-negative values embed as-is, negatives as p - |x|
// (rust/volta-field/src/lib.rs:32-40).
__host__ __device__ __forceinline__ uint64_t from_i16(int16_t x) {
    return x >= 0 ? static_cast<uint64_t>(x) : P - static_cast<uint64_t>(-static_cast<int32_t>(x));
}

// ---- quadratic extension Fp2 = Fp[phi]/(phi^2 - 7) -----------------------

struct alignas(8) Fp2 {
    uint64_t c0;
    uint64_t c1;
};

__host__ __device__ __forceinline__ Fp2 fp2_add(Fp2 a, Fp2 b) { return Fp2{add(a.c0, b.c0), add(a.c1, b.c1)}; }

__host__ __device__ __forceinline__ Fp2 fp2_mul(Fp2 a, Fp2 b) {
    // (a0 + a1 phi)(b0 + b1 phi) = (a0 b0 + 7 a1 b1) + (a0 b1 + a1 b0) phi
    return Fp2{add(mul(a.c0, b.c0), mul(7, mul(a.c1, b.c1))), add(mul(a.c0, b.c1), mul(a.c1, b.c0))};
}

__host__ __device__ __forceinline__ Fp2 fp2_mul_base(Fp2 a, uint64_t x) { return Fp2{mul(a.c0, x), mul(a.c1, x)}; }

}  // namespace gl
