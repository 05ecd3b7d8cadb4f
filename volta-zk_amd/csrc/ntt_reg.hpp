// ntt_reg.hpp -- device helpers of the register four-step NTT passes
// (ntt_reg.hip), shared with the X4 transforms (x4.hip).
//
// Roots: b_k = 7^((p-1)/2^k) is the base field's root of order 2^k.  The X4
// roots (rust/volta-pcs/src/x4/ntt.rs:28-57) are w(2^k) = b_k for k <= 31,
// w(2^32) = -b_32 and w(2^33) = (0, c1) in Fp2 = Fp[phi]/(phi^2 - 7) with
// w(2^33)^2 = w(2^32).  root_pow gives w(2^nb)^e, which for nb <= 31 is the
// base field's b_nb^e.
#pragma once

#include <hip/hip_runtime.h>

#include "gl64.hpp"
#include "gl64_shift.hpp"

namespace vmx {
namespace nreg {

constexpr int THREADS = 256;
constexpr int GBITS = 12;          // inner table: w_4096^j, j < 2048
constexpr int PASS_BITS = 8;       // largest radix of one pass (2^9: see pass_bits)
constexpr int MIN_BITS = 13;       // smallest transform run as passes (below: one LDS tile)
constexpr int MAX_PASSES = 5;      // 2^33 = five passes of at most 2^8
constexpr bool XCD_SWIZZLE = false;  // consecutive tiles on one XCD (shared L2)
constexpr uint64_t ROOT33_C1 = 0x076de30b51a3f645ull;
static_assert(PASS_BITS <= GBITS, "the inner table covers radices up to 2^GBITS");

// Adjacent columns (rows in the gather) per tile, as a power of two, for
// elements of `planes` u64: runs of 128 bytes (one cache line) up to 2^25
// points and 256 bytes above, where the passes' strides reach megabytes
// (measured best on MI355X).
__host__ __device__ constexpr int run_bits(int nb, int planes) {
    return (nb >= 26 ? 4 : 3) + (planes == 1 ? 1 : 0);
}

// Largest radix of a pass for elements of `planes` u64: 2^9 for one-plane
// rows below 2^26 points, whose radix-2^9 tiles stay at 70 KB of LDS (two per
// CU); that saves a pass at 2^17, 2^18 and 2^25 (measured: 2^17 rows 4.4 ms
// against 5.4 ms in three passes).  2^8 otherwise: a radix-2^9 tile of Fp2 or
// of 32 adjacent rows needs 139 KB, one per CU, and ran 1.8x slower.
__host__ __device__ constexpr int pass_bits(int nb, int planes) { return planes == 1 && nb < 26 ? 9 : PASS_BITS; }

// Tile index of this workgroup.  Workgroups are dispatched round-robin over
// the 8 XCDs (blockIdx.x mod 8); with XCD_SWIZZLE the tiles an XCD runs back to
// back are consecutive, so neighbouring tiles' shared cache lines meet in one L2.
template <bool SWIZZLE = XCD_SWIZZLE>
__device__ __forceinline__ uint64_t tile_id() {
    const uint64_t b = blockIdx.x;
    if constexpr (SWIZZLE) {
        const uint64_t g = gridDim.x;
        if ((g & 7) == 0) return (b & 7) * (g >> 3) + (b >> 3);
    }
    return b;
}

// w^e from a two-level table of w (TwiddleSet::split or reg): lo[e mod 2^h] hi[e >> h].
__device__ __forceinline__ uint64_t tw_split(const uint64_t* t, uint64_t e, int h) {
    const uint64_t lo = t[e & ((uint64_t{1} << h) - 1)];
    const uint64_t hi = t[(uint64_t{1} << h) + (e >> h)];
    return gl::mul32x4(lo, hi);
}

// 7 x = 8 x - x.
__device__ __forceinline__ uint64_t mul7(uint64_t x) { return gl::sub(gl::shl_mod<3>(x), x); }

// Which X4 root a transform of 2^nb points uses: the base root (nb <= 31),
// the negated one (nb = 32) or the imaginary one (nb = 33).  A kernel is
// compiled per mode so the per-element twiddle code has no branches and its
// table loads can all be in flight together.
enum RootMode { ROOT_BASE = 0, ROOT_NEG32 = 1, ROOT_IMAG33 = 2 };
constexpr int root_mode(int nb) { return nb <= 31 ? ROOT_BASE : nb == 32 ? ROOT_NEG32 : ROOT_IMAG33; }

// w(2^nb)^e for e < 2^nb from the two-level table of b_min(nb,32): the real
// value, or (imag set) the c1 coordinate of a purely imaginary power (nb = 33,
// e odd).
template <int MODE>
__device__ __forceinline__ uint64_t root_pow(uint64_t e, const uint64_t* split, int h, bool& imag) {
    imag = false;
    if constexpr (MODE == ROOT_BASE) {
        return tw_split(split, e, h);
    } else if constexpr (MODE == ROOT_NEG32) {
        const uint64_t v = tw_split(split, e, h);
        return (e & 1) ? gl::neg(v) : v;
    } else {
        const uint64_t q = e >> 1;
        uint64_t t = tw_split(split, q, h);
        if (q & 1) t = gl::neg(t);
        imag = (e & 1) != 0;
        const uint64_t ti = gl::mul32x4(ROOT33_C1, t);
        return imag ? ti : t;
    }
}

// The same for a transform size known only at run time (the fold kernel).
__device__ __forceinline__ uint64_t root_pow(uint64_t e, int nb, const uint64_t* split, int h, bool& imag) {
    if (nb <= 31) return root_pow<ROOT_BASE>(e, split, h, imag);
    if (nb == 32) return root_pow<ROOT_NEG32>(e, split, h, imag);
    return root_pow<ROOT_IMAG33>(e, split, h, imag);
}

// Mixed-radix layout of a row index of the gather pass.
struct Digits {
    int r1;       // width of the first digit i_1 (0 for a one-pass transform)
    int count;    // middle digits i_2 .. i_(P-1): P - 2, or 0
    int bits[3];  // their widths, i_2 first
};

// The gather tile of this workgroup: the natural index nat0 of its first
// row's first input, its first row row0, and mid_bits, the width of the
// middle digits (rows of one tile are 2^mid_bits apart).  Tiles run over the
// groups of 2^qb first digits fastest.
template <bool SWIZZLE = XCD_SWIZZLE>
__device__ __forceinline__ void gather_tile(int nb, int rb, int qb, const Digits& d, uint64_t& nat0, uint64_t& row0,
                                            int& mid_bits) {
    mid_bits = nb - rb - d.r1;
    const int gbits = d.r1 - qb;
    const uint64_t blk = tile_id<SWIZZLE>();
    const uint64_t g = blk & ((uint64_t{1} << gbits) - 1);
    const uint64_t rest = blk >> gbits;
    uint64_t natr = 0;
    int shift = mid_bits, scale = 0;
    for (int j = 0; j < d.count; ++j) {
        shift -= d.bits[j];
        natr += ((rest >> shift) & ((uint64_t{1} << d.bits[j]) - 1)) << scale;
        scale += d.bits[j];
    }
    nat0 = (g << qb) + (natr << d.r1);
    row0 = ((g << qb) << mid_bits) + rest;
}

}  // namespace nreg
}  // namespace vmx
