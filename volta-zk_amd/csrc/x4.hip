// x4.hip -- the X4 extension-field transforms on gfx950: the Fp2 NTT with the
// order-2^33 root (rust/volta-pcs/src/x4/ntt.rs:66-122, the device entry
// cuda/volta_cuda_backend.cu:5577-5634), codeword folding (x4/ntt.rs:238-256,
// cuda/volta_x4b.cuh:194-218 and 636-667) and the Moebius inverse
// (.cu:2965-2972, 7114-7130).
//
// The X4 roots of unity are real up to order 2^32.  With b_k = 7^((p-1)/2^k),
// the base field's root of order 2^k:
//   w(2^k)  = b_k          for k <= 31,
//   w(2^32) = -b_32,
//   w(2^33) = (0, c1), c1 = 0x076de30b51a3f645, with w(2^33)^2 = w(2^32).
// Every sub-transform of an n-point transform uses a root w(n)^(n/R) with n/R
// even, which is a base-field root b_R; only the twiddles w(n)^e with e odd
// differ from the base field's, by a sign (n = 2^32) or by being purely
// imaginary (n = 2^33).  So the transform is two base-field transforms, one
// per coordinate plane, with real twiddles, except for the odd-exponent
// twiddles of the last pass.  The reference multiplies a full Fp2 twiddle at
// every butterfly; none is needed.
//
// Layout: Fp2 in HBM as (c0, c1) u64 pairs, 16 bytes, the ABI's layout.  In LDS
// a workgroup's tile is split into a c0 plane and a c1 plane of u64 so the
// radix-2^2 butterflies (lds_dit.hpp) run on plain field elements.
//
// An n = 2^nb point transform, n = R_1 R_2 .. R_P, in P passes over HBM
// (decimation in time by the least significant input digit first):
//   pass 1 ("gather"): row r = (i_1, .., i_(P-1)) (i_1 most significant) gets
//     the R_P-point DFT of x[nat(r) + (n / R_P) j], j < R_P, with
//     nat(r) = i_1 + R_1 (i_2 + R_2 (..)), stored contiguously as row r of
//     the output.  A workgroup takes 8 rows (16 from 2^26 points) whose i_1
//     are adjacent, so the reads are runs of 128 (256) bytes; elements at
//     index >= len (the caller's zero tail) are read as zero and never stored.
//   passes P-1 .. 1 ("columns"): the output is [H][R_p][L]
//     (H = R_1 .. R_(p-1), L = R_(p+1) .. R_P); element (i, l) is multiplied
//     by w_(R_p L)^(i l) = w(n)^(H i l) and column l gets the R_p-point DFT
//     over i, in place.  A workgroup takes 8 (16) adjacent columns.
// Up to 2^12 points one workgroup does the whole transform in LDS; above,
// passes have radix <= 2^8 (2 passes up to 2^16, .., 5 for 2^33).  Each pass
// reads and writes every element once (32 bytes of HBM traffic per element)
// and computes its R-point DFTs as register four-steps of shift-only 16-point
// (or smaller) DFTs with one general twiddle per element.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "context.hpp"
#include "gl64.hpp"
#include "gl64_shift.hpp"
#include "kernels.hpp"
#include "lds_dit.hpp"

namespace vmx {
namespace x4 {

using u64x2 = uint64_t __attribute__((ext_vector_type(2)));

constexpr int THREADS = 256;
constexpr int GBITS = 12;         // inner table: w_4096^j, j < 2048
constexpr int TILE_BITS = 12;     // one-pass transforms and Moebius tiles: 2^12 Fp2 (64 KiB of LDS)
constexpr int PASS_BITS = 8;      // largest radix of a pass of a multi-pass transform
constexpr int MAX_PASSES = 5;     // 2^33 = five passes of at most 2^8
constexpr bool XCD_SWIZZLE = false;  // consecutive tiles on one XCD (shared L2)
constexpr int MOBIUS_RUN_BITS = 3;   // Moebius passes above the first: 8 adjacent columns
static_assert(PASS_BITS <= GBITS, "the inner table covers radices up to 2^GBITS");

// Adjacent columns (rows in the gather) per multi-pass tile, as a power of
// two: runs of 8 elements (128 bytes, one cache line) up to 2^25 points, 16
// above, where the passes' strides reach megabytes (measured best on MI355X).
__host__ __device__ constexpr int run_bits(int nb) { return nb >= 26 ? 4 : 3; }

// Tile index of this workgroup.  Workgroups are dispatched round-robin over
// the 8 XCDs (blockIdx.x mod 8); with XCD_SWIZZLE the tiles an XCD runs back to
// back are consecutive, so neighbouring tiles' shared cache lines meet in one L2.
__device__ __forceinline__ uint64_t tile_id() {
    const uint64_t b = blockIdx.x;
    if constexpr (XCD_SWIZZLE) {
        const uint64_t g = gridDim.x;
        if ((g & 7) == 0) return (b & 7) * (g >> 3) + (b >> 3);
    }
    return b;
}
constexpr uint64_t ROOT33_C1 = 0x076de30b51a3f645ull;
constexpr uint64_t INV2 = 0x7FFFFFFF80000001ull;  // (p + 1) / 2

// w^e from a two-level table of w (TwiddleSet::split), e < the table's size.
__device__ __forceinline__ uint64_t tw_split(const uint64_t* t, uint64_t e, int h) {
    const uint64_t lo = t[e & ((uint64_t{1} << h) - 1)];
    const uint64_t hi = t[(uint64_t{1} << h) + (e >> h)];
    return gl::mul32x4(lo, hi);
}

// 7 x = 8 x - x.
__device__ __forceinline__ uint64_t mul7(uint64_t x) { return gl::sub(gl::shl_mod<3>(x), x); }

// x / 2 for canonical x: x >> 1, plus (p + 1) / 2 when x is odd.
__device__ __forceinline__ uint64_t halve(uint64_t x) { return (x >> 1) + ((x & 1) ? INV2 : 0); }

// Fp2 product (phi^2 = 7), three base products (Karatsuba).
__device__ __forceinline__ u64x2 fp2_mul(u64x2 a, u64x2 b) {
    const uint64_t p0 = gl::mul32x4(a.x, b.x), p1 = gl::mul32x4(a.y, b.y);
    const uint64_t s = gl::mul32x4(gl::add(a.x, a.y), gl::add(b.x, b.y));
    return u64x2{gl::add(p0, mul7(p1)), gl::sub(s, gl::add(p0, p1))};
}

// ---- NTT passes ------------------------------------------------------------------------

// w(2^nb)^e for e < 2^nb, nb <= 33, from the table of b_min(nb,32): the real
// value, or (imag set) the c1 coordinate of a purely imaginary power.
__device__ __forceinline__ uint64_t x4_pow(uint64_t e, int nb, const uint64_t* split, int h, bool& imag) {
    imag = false;
    if (nb <= 31) return tw_split(split, e, h);
    if (nb == 32) {
        const uint64_t v = tw_split(split, e, h);
        return (e & 1) ? gl::neg(v) : v;
    }
    const uint64_t q = e >> 1;
    uint64_t t = tw_split(split, q, h);
    if (q & 1) t = gl::neg(t);
    if (e & 1) {
        imag = true;
        return gl::mul32x4(ROOT33_C1, t);
    }
    return t;
}

// Mixed-radix layout of a row index of the gather pass.
struct Digits {
    int r1;       // width of the first digit i_1 (0 for a one-pass transform)
    int count;    // middle digits i_2 .. i_(P-1): P - 2, or 0
    int bits[3];  // their widths, i_2 first
};

// The gather tile of this workgroup: the natural index nat0 of its first
// row's first input, its first row row0, and mid_bits, the width of the
// middle digits (rows of one tile are 2^mid_bits apart).  Tiles run g fastest.
__device__ __forceinline__ void gather_tile(int nb, int rb, int qb, const Digits& d, uint64_t& nat0, uint64_t& row0,
                                            int& mid_bits) {
    mid_bits = nb - rb - d.r1;
    const int gbits = d.r1 - qb;  // groups of Q first digits
    const uint64_t blk = tile_id();
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

// Gather pass: output row r (R = 2^rb elements) is the DFT of
// x[nat(r) + 2^(nb - rb) j], j < R.  A workgroup takes the Q = 2^qb rows
// r = (g Q + t) S + rest, t < Q (S = 2^mid_bits rows per value of i_1), whose
// nat(r) = g Q + t + R_1 nat'(rest) are adjacent; tiles run g fastest, so
// consecutive tiles read adjacent runs.  Reads at index >= len are zero.  The
// DFT runs in LDS (radix-2^2); used for one-pass transforms (n <= 2^12).
__global__ __launch_bounds__(THREADS) void gather_pass(const u64x2* __restrict__ x, uint64_t len,
                                                       u64x2* __restrict__ y, int nb, int rb, int qb, Digits d,
                                                       const uint64_t* inner) {
    extern __shared__ uint64_t s[];
    const uint32_t R = 1u << rb, Q = 1u << qb;
    const uint32_t QR = Q << rb;
    uint64_t nat0, row0;
    int mid_bits;
    gather_tile(nb, rb, qb, d, nat0, row0, mid_bits);
    for (uint32_t e = threadIdx.x; e < QR; e += THREADS) {
        const uint32_t j = e >> qb, t = e & (Q - 1);
        const uint64_t idx = nat0 + t + (static_cast<uint64_t>(j) << (nb - rb));
        const u64x2 v = idx < len ? x[idx] : u64x2{0, 0};
        const uint32_t pos = (t << rb) + brev(j, rb);
        s[pos] = v.x;
        s[QR + pos] = v.y;
    }
    __syncthreads();
    lds_dit(s, static_cast<int>(2 * Q), rb, GBITS, inner);
    for (uint32_t e = threadIdx.x; e < QR; e += THREADS) {
        const uint32_t t = e >> rb, k = e & (R - 1);
        const uint32_t pos = (t << rb) + k;
        y[((row0 + (static_cast<uint64_t>(t) << mid_bits)) << rb) + k] = u64x2{s[pos], s[QR + pos]};
    }
}

// ---- register-resident passes ----------------------------------------------------------
//
// The multi-pass kernels below run each R = A B point DFT (A = 2^LA, B = 2^LB,
// both <= 32) as a four-step inside the tile: with input index j = ja B + jb
// and output index k = ka + A kb,
//   step 1: one thread takes the A inputs of one (plane, column, jb) straight
//     from HBM into registers, DFTs them over ja with shift-only twiddles
//     (every root of order <= 64 is a power of two), multiplies output ka by
//     w_R^(jb ka) and parks them in LDS;
//   step 2: one thread takes the B values of one (plane, column, ka), DFTs
//     them over jb and stores Y[ka + A kb] straight to HBM.
// One general multiply per element and one LDS round trip replace the LDS
// radix-2^2 loop's three multiplies per four elements per two stages.  LDS
// holds (plane, column) pairs fastest, then jb, then ka with a pitch of
// PW (B + 1) words, so both steps' accesses avoid bank conflicts.

// Exponent of the base root of order 2^L (L <= 6) as a power of two:
// w_64 = 2^39, so w_(2^L) = 2^(39 2^(6-L)), exponents mod 192.
template <int L>
constexpr int ew_log() {
    return (gl::E_W64 << (6 - L)) % 192;
}

// w_4096^e for e < 4096 from the inner table (w_4096^j, j < 2048; w_4096^2048 = -1).
__device__ __forceinline__ uint64_t inner_pow(const uint64_t* inner, uint32_t e) {
    return e < 2048 ? inner[e] : gl::neg(inner[e - 2048]);
}

// The partner lane's value (lane ^ 1): the other coordinate of the same element.
__device__ __forceinline__ uint64_t partner(uint64_t v) {
    const uint32_t lo = static_cast<uint32_t>(__shfl_xor(static_cast<int>(static_cast<uint32_t>(v)), 1));
    const uint32_t hi = static_cast<uint32_t>(__shfl_xor(static_cast<int>(static_cast<uint32_t>(v >> 32)), 1));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

// Step 1's tail and step 2's head, shared by both kernels: v (natural order
// over ka after the A-point DFT) times w_R^(jb ka), parked at (pc, jb, ka).
template <int LA, int LB>
__device__ __forceinline__ void park(uint64_t* s, const uint64_t* v, uint32_t pc, uint32_t jb, uint32_t PW,
                                     uint32_t pitch, const uint64_t* inner) {
    constexpr int A = 1 << LA, RB = LA + LB;
    s[pc + PW * jb] = v[0];
    gl::static_for<1, A>([&](auto ka_) {
        constexpr int ka = decltype(ka_)::value;
        s[pc + PW * jb + ka * pitch] = gl::mul32x4(v[ka], inner_pow(inner, (jb * ka) << (GBITS - RB)));
    });
}

template <int LB>
__device__ __forceinline__ void unpark(const uint64_t* s, uint64_t* v, uint32_t pc, uint32_t ka, uint32_t PW,
                                       uint32_t pitch) {
    constexpr int B = 1 << LB;
    gl::static_for<0, B>([&](auto jb_) {
        constexpr int jb = decltype(jb_)::value;
        v[gl::bitrev_c(jb, LB)] = s[pc + PW * jb + ka * pitch];
    });
    gl::dit_pow2<LB, ew_log<LB>()>(v);
}

// Gather pass of a multi-pass transform: the tiles and output of gather_pass,
// with the register four-step.  x and y are viewed as u64: coordinate p of
// element e at 2 e + p.
template <int LA, int LB>
__global__ __launch_bounds__(THREADS) void gather_reg(const uint64_t* __restrict__ x, uint64_t len,
                                                      uint64_t* __restrict__ y, int nb, int qb, Digits d,
                                                      const uint64_t* inner) {
    constexpr int A = 1 << LA, B = 1 << LB, RB = LA + LB;
    extern __shared__ uint64_t s[];
    const int pwb = qb + 1;  // (plane, row) pairs: 2^pwb
    const uint32_t PW = 1u << pwb;
    const uint32_t pitch = PW * (B + 1);
    uint64_t nat0, row0;
    int mid_bits;
    gather_tile(nb, RB, qb, d, nat0, row0, mid_bits);
    const int sh = nb - RB;
    for (uint32_t job = threadIdx.x; job < (PW << LB); job += THREADS) {
        const uint32_t pc = job & (PW - 1), jb = job >> pwb;
        const uint32_t plane = pc & 1, t = pc >> 1;
        uint64_t v[A];
        gl::static_for<0, A>([&](auto ja_) {
            constexpr int ja = decltype(ja_)::value;
            const uint64_t idx = nat0 + t + ((static_cast<uint64_t>(ja) * B + jb) << sh);
            v[gl::bitrev_c(ja, LA)] = idx < len ? x[2 * idx + plane] : 0;
        });
        gl::dit_pow2<LA, ew_log<LA>()>(v);
        park<LA, LB>(s, v, pc, jb, PW, pitch, inner);
    }
    __syncthreads();
    for (uint32_t job = threadIdx.x; job < (PW << LA); job += THREADS) {
        const uint32_t pc = job & (PW - 1), ka = job >> pwb;
        const uint32_t plane = pc & 1, t = pc >> 1;
        uint64_t v[B];
        unpark<LB>(s, v, pc, ka, PW, pitch);
        const uint64_t out0 = ((row0 + (static_cast<uint64_t>(t) << mid_bits)) << RB) + ka;
        gl::static_for<0, B>([&](auto kb_) {
            constexpr int kb = decltype(kb_)::value;
            y[2 * (out0 + A * kb) + plane] = v[kb];
        });
    }
}

// Column pass, in place.  The array is [H][R][L] (H = 2^hb, R = 2^(LA+LB),
// L = 2^lb, n = H R L = 2^nb); the tile takes the 2^cb adjacent columns
// l0 .. of block h: element (i, l) is multiplied by w(n)^(H i l) as it loads,
// then each column gets the R-point DFT over i (register four-step).  For
// n = 2^33 the last pass (hb = 0) meets imaginary twiddles, which mix the two
// coordinates: each lane then also reads its partner lane's coordinate.
template <int LA, int LB>
__global__ __launch_bounds__(THREADS) void col_reg(uint64_t* a, int nb, int hb, int lb, int cb,
                                                   const uint64_t* inner, const uint64_t* split, int split_h) {
    constexpr int A = 1 << LA, B = 1 << LB, RB = LA + LB;
    extern __shared__ uint64_t s[];
    const int pwb = cb + 1;  // (plane, column) pairs: 2^pwb
    const uint32_t PW = 1u << pwb;
    const uint32_t pitch = PW * (B + 1);
    const uint64_t lblocks = (uint64_t{1} << lb) >> cb;
    const uint64_t blk = tile_id();
    const uint64_t h = blk / lblocks;
    const uint64_t l0 = (blk - h * lblocks) << cb;
    const uint64_t base = ((h << RB) << lb) + l0;
    const bool mixed = nb == 33 && hb == 0;  // uniform
    for (uint32_t job = threadIdx.x; job < (PW << LB); job += THREADS) {
        const uint32_t pc = job & (PW - 1), jb = job >> pwb;
        const uint32_t plane = pc & 1, c = pc >> 1;
        const uint64_t l = l0 + c;
        uint64_t v[A];
        gl::static_for<0, A>([&](auto ja_) {
            constexpr int ja = decltype(ja_)::value;
            const uint64_t i = static_cast<uint64_t>(ja) * B + jb;
            const uint64_t xv = a[2 * (base + (i << lb) + c) + plane];
            bool imag;
            const uint64_t t = x4_pow((i * l) << hb, nb, split, split_h, imag);
            uint64_t r;
            if (mixed) {
                const uint64_t other = partner(xv);
                // (v0 + v1 phi) (t phi) = 7 v1 t + v0 t phi
                r = !imag ? gl::mul32x4(xv, t) : plane == 0 ? mul7(gl::mul32x4(other, t)) : gl::mul32x4(other, t);
            } else {
                r = gl::mul32x4(xv, t);
            }
            v[gl::bitrev_c(ja, LA)] = r;
        });
        gl::dit_pow2<LA, ew_log<LA>()>(v);
        park<LA, LB>(s, v, pc, jb, PW, pitch, inner);
    }
    __syncthreads();
    for (uint32_t job = threadIdx.x; job < (PW << LA); job += THREADS) {
        const uint32_t pc = job & (PW - 1), ka = job >> pwb;
        const uint32_t plane = pc & 1, c = pc >> 1;
        uint64_t v[B];
        unpark<LB>(s, v, pc, ka, PW, pitch);
        gl::static_for<0, B>([&](auto kb_) {
            constexpr int kb = decltype(kb_)::value;
            a[2 * (base + ((static_cast<uint64_t>(ka) + A * kb) << lb) + c) + plane] = v[kb];
        });
    }
}

// ---- codeword fold -----------------------------------------------------------------------

// out[j] = (P_j + N_j)/2 + ch (P_j - N_j)/2 w^-(j0 + j), j < count,
// w = w(2^nb) (direct_fold_symbol, cuda/volta_x4b.cuh:194-201).  Thread t
// takes j = t, t + D, .. with D the grid's thread count; its running
// y = w^-(j0 + j) / 2 advances by step = w^-D (real: D is even), and its
// imaginary flag (nb = 33, odd exponent) never changes along the way.
__global__ __launch_bounds__(THREADS) void direct_fold(const u64x2* __restrict__ pos, const u64x2* __restrict__ neg,
                                                       u64x2* __restrict__ out, uint64_t j0, uint64_t count, u64x2 ch,
                                                       int nb, const uint64_t* split, int h, uint64_t step) {
    const uint64_t D = static_cast<uint64_t>(gridDim.x) * THREADS;
    uint64_t j = static_cast<uint64_t>(blockIdx.x) * THREADS + threadIdx.x;
    if (j >= count) return;
    const uint64_t mask = (uint64_t{1} << nb) - 1;
    bool imag;
    uint64_t y = halve(x4_pow((uint64_t{0} - (j0 + j)) & mask, nb, split, h, imag));
    for (; j < count; j += D) {
        const u64x2 p = pos[j], q = neg[j];
        const u64x2 even{halve(gl::add(p.x, q.x)), halve(gl::add(p.y, q.y))};
        const u64x2 dd{gl::sub(p.x, q.x), gl::sub(p.y, q.y)};
        const u64x2 odd = imag ? u64x2{mul7(gl::mul32x4(dd.y, y)), gl::mul32x4(dd.x, y)}
                               : u64x2{gl::mul32x4(dd.x, y), gl::mul32x4(dd.y, y)};
        const u64x2 co = fp2_mul(ch, odd);
        out[j] = u64x2{gl::add(even.x, co.x), gl::add(even.y, co.y)};
        y = gl::mul32x4(y, step);
    }
}

// ---- Moebius transform -------------------------------------------------------------------

// One pass over the middle index of [H][R][L] (R = 2^rb, L = 2^lb): for every
// bit of i, the element with the bit set gains (inverse) or loses the one
// without.  Workgroup (h, l0) takes C = 2^cb adjacent columns.
__global__ __launch_bounds__(THREADS) void mobius_pass(u64x2* a, int rb, int lb, int cb, int inverse) {
    extern __shared__ uint64_t s[];
    const uint32_t C = 1u << cb;
    const uint32_t CR = C << rb;
    const uint64_t lblocks = (uint64_t{1} << lb) >> cb;
    const uint64_t h = blockIdx.x / lblocks;
    const uint64_t l0 = (blockIdx.x - h * lblocks) << cb;
    const uint64_t base = ((h << rb) << lb) + l0;
    for (uint32_t e = threadIdx.x; e < CR; e += THREADS) {
        const uint32_t i = e >> cb, c = e & (C - 1);
        const u64x2 v = a[base + (static_cast<uint64_t>(i) << lb) + c];
        s[(c << rb) + i] = v.x;
        s[CR + (c << rb) + i] = v.y;
    }
    __syncthreads();
    const uint32_t pairs = CR;  // (2 planes x C x R) / 2
    for (int b = 0; b < rb; ++b) {
        const uint32_t bit = 1u << b;
        for (uint32_t e = threadIdx.x; e < pairs; e += THREADS) {
            // e enumerates (plane-column, i with bit b clear)
            const uint32_t col = e >> (rb - 1), r = e & ((1u << (rb - 1)) - 1);
            const uint32_t lo = ((r >> b) << (b + 1)) | (r & (bit - 1));
            const uint32_t base_s = col << rb;
            const uint64_t x = s[base_s + lo], y = s[base_s + (lo | bit)];
            s[base_s + (lo | bit)] = inverse ? gl::add(y, x) : gl::sub(y, x);
        }
        __syncthreads();
    }
    for (uint32_t e = threadIdx.x; e < CR; e += THREADS) {
        const uint32_t i = e >> cb, c = e & (C - 1);
        a[base + (static_cast<uint64_t>(i) << lb) + c] = u64x2{s[(c << rb) + i], s[CR + (c << rb) + i]};
    }
}

}  // namespace x4

// ---- host side -----------------------------------------------------------------------------

namespace {

int log2_exact(uint64_t n) {
    int b = 0;
    while ((uint64_t{1} << b) < n) ++b;
    return b;
}

// w(2^nb)^e on the host as (value, imaginary), the device's x4_pow.
uint64_t x4_pow_host(uint64_t e, int nb, bool* imag) {
    *imag = false;
    if (nb <= 31) return gl::pow_host(gl::root_of_unity(static_cast<unsigned>(nb)), e);
    const uint64_t b32 = gl::root_of_unity(32);
    if (nb == 32) {
        const uint64_t v = gl::pow_host(b32, e);
        return (e & 1) ? gl::neg(v) : v;
    }
    const uint64_t q = e >> 1;
    uint64_t t = gl::pow_host(b32, q);
    if (q & 1) t = gl::neg(t);
    if (e & 1) {
        *imag = true;
        return gl::mul32x4(x4::ROOT33_C1, t);
    }
    return t;
}

// The root constant w(2^33) = (0, c1) must square to w(2^32) = -b_32:
// (0, c1)^2 = (7 c1^2, 0).
bool root33_consistent() {
    const uint64_t sq = gl::mul32x4(7, gl::mul32x4(x4::ROOT33_C1, x4::ROOT33_C1));
    return sq == gl::neg(gl::root_of_unity(32));
}

// Pass radices for a 2^nb-point transform: one pass up to 2^12, else the
// fewest passes of at most 2^8, as even as possible (the gather, last digit,
// runs first).
int plan(int nb, int* r) {
    if (nb <= std::min(x4::TILE_BITS, x4::GBITS)) {
        r[0] = nb;
        return 1;
    }
    const int passes = (nb + x4::PASS_BITS - 1) / x4::PASS_BITS;
    if (passes > x4::MAX_PASSES) return 0;
    for (int p = 0; p < passes; ++p) r[p] = nb / passes + (p < nb % passes ? 1 : 0);
    return passes;
}

using GatherRegFn = void (*)(const uint64_t*, uint64_t, uint64_t*, int, int, x4::Digits, const uint64_t*);
using ColRegFn = void (*)(uint64_t*, int, int, int, int, const uint64_t*, const uint64_t*, int);

// The register kernels for a pass of radix 2^rb: A = 2^ceil(rb/2), B = 2^floor(rb/2).
bool reg_kernels(int rb, GatherRegFn* g, ColRegFn* col) {
    switch (rb) {
        case 5: *g = x4::gather_reg<3, 2>; *col = x4::col_reg<3, 2>; return true;
        case 6: *g = x4::gather_reg<3, 3>; *col = x4::col_reg<3, 3>; return true;
        case 7: *g = x4::gather_reg<4, 3>; *col = x4::col_reg<4, 3>; return true;
        case 8: *g = x4::gather_reg<4, 4>; *col = x4::col_reg<4, 4>; return true;
        default: return false;
    }
}

// LDS bytes of a register-kernel tile: 2^(wb+1) (plane, column) pairs x A x (B + 1) words.
size_t reg_lds(int rb, int wb) {
    const size_t A = size_t{1} << ((rb + 1) / 2), B = size_t{1} << (rb / 2);
    return (size_t{2} << wb) * A * (B + 1) * sizeof(uint64_t);
}

template <class K>
int set_lds(Context* c, K kernel, size_t lds) {
    if (lds <= 65536) return 0;
    VMX_HIP(c, hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
    return 0;
}

}  // namespace

int x4_tables(Context* c, int nb, uint64_t* h2d, X4Tables* out) {
    if (nb < 1 || nb > 33) return fail_msg(c, "X4 transform size out of range");
    if (!root33_consistent()) return fail_msg(c, "X4 root constant is inconsistent with the base field");
    TwiddleSet* inner = nullptr;
    TwiddleSet* t = nullptr;
    if (ensure_twiddles(c, size_t{1} << x4::GBITS, h2d, &inner)) return -1;
    if (ensure_split_twiddles(c, size_t{1} << std::min(nb, 32), h2d, &t)) return -1;
    out->inner = inner->fwd;
    out->split = t->split;
    out->split_h = t->split_h;
    out->nb = nb;
    return 0;
}

int x4_ntt(Context* c, const X4Tables& tb, const gl::Fp2* in, uint64_t len, gl::Fp2* out) {
    using namespace x4;
    const int nb = tb.nb;
    int r[MAX_PASSES] = {};
    const int passes = plan(nb, r);
    if (passes == 0) return fail_msg(c, "X4 NTT size needs more passes than supported");
    const int wb_max = run_bits(nb);
    if (passes == 1) {  // the whole transform in one tile
        Digits d{};
        const size_t lds = size_t{16} << nb;
        if (set_lds(c, gather_pass, lds)) return -1;
        hipLaunchKernelGGL(gather_pass, dim3(1), dim3(THREADS), lds, c->stream, reinterpret_cast<const u64x2*>(in), len,
                           reinterpret_cast<u64x2*>(out), nb, nb, 0, d, tb.inner);
        VMX_HIP(c, hipGetLastError());
        return 0;
    }
    GatherRegFn greg = nullptr;
    ColRegFn creg = nullptr;
    // gather: the last digit's DFT, rows in (i_1, .., i_(P-1)) order
    {
        const int rb = r[passes - 1];
        const int qb = std::min(wb_max, r[0]);
        Digits d{};
        d.r1 = r[0];
        d.count = passes - 2;
        for (int j = 0; j < d.count; ++j) d.bits[j] = r[1 + j];
        const uint64_t blocks = uint64_t{1} << (nb - rb - qb);
        const size_t lds = reg_lds(rb, qb);
        if (!reg_kernels(rb, &greg, &creg) || blocks > 0x7FFFFFFFull || lds > 160 * 1024)
            return fail_msg(c, "X4 NTT pass exceeds its launch limits");
        if (set_lds(c, greg, lds)) return -1;
        hipLaunchKernelGGL(greg, dim3(static_cast<unsigned>(blocks)), dim3(THREADS), lds, c->stream,
                           reinterpret_cast<const uint64_t*>(in), len, reinterpret_cast<uint64_t*>(out), nb, qb, d,
                           tb.inner);
        VMX_HIP(c, hipGetLastError());
    }
    // columns: digits P-1 .. 1, in place
    int lbits = r[passes - 1];
    for (int p = passes - 2; p >= 0; --p) {
        const int rb = r[p], lb = lbits, hb = nb - rb - lb;
        const int cb = std::min(wb_max, lb);
        const uint64_t blocks = uint64_t{1} << (nb - rb - cb);
        const size_t lds = reg_lds(rb, cb);
        if (!reg_kernels(rb, &greg, &creg) || blocks > 0x7FFFFFFFull || lds > 160 * 1024)
            return fail_msg(c, "X4 NTT pass exceeds its launch limits");
        if (set_lds(c, creg, lds)) return -1;
        hipLaunchKernelGGL(creg, dim3(static_cast<unsigned>(blocks)), dim3(THREADS), lds, c->stream,
                           reinterpret_cast<uint64_t*>(out), nb, hb, lb, cb, tb.inner, tb.split, tb.split_h);
        VMX_HIP(c, hipGetLastError());
        lbits += rb;
    }
    return 0;
}

int x4_fold(Context* c, const X4Tables& tb, const gl::Fp2* pos, const gl::Fp2* neg, gl::Fp2* out, uint64_t j0,
            uint64_t count, gl::Fp2 ch) {
    using x4::u64x2;
    if (count == 0) return 0;
    const uint64_t per_block = x4::THREADS;
    const uint64_t max_blocks = static_cast<uint64_t>(std::max(1, c->cu_count)) * 32;
    const uint64_t blocks = std::min((count + per_block - 1) / per_block, max_blocks);
    const uint64_t D = blocks * per_block;
    const uint64_t n = uint64_t{1} << tb.nb;
    bool imag = false;
    const uint64_t step = x4_pow_host((n - (D & (n - 1))) & (n - 1), tb.nb, &imag);
    if (imag) return fail_msg(c, "X4 fold step must be real");  // D is even
    hipLaunchKernelGGL(x4::direct_fold, dim3(static_cast<unsigned>(blocks)), dim3(x4::THREADS), 0, c->stream,
                       reinterpret_cast<const u64x2*>(pos), reinterpret_cast<const u64x2*>(neg),
                       reinterpret_cast<u64x2*>(out), j0, count, u64x2{ch.c0, ch.c1}, tb.nb, tb.split, tb.split_h,
                       step);
    VMX_HIP(c, hipGetLastError());
    return 0;
}

int fp2_mobius(Context* c, gl::Fp2* values, uint64_t n, bool inverse) {
    using namespace x4;
    const int nb = log2_exact(n);
    auto* a = reinterpret_cast<u64x2*>(values);
    // low bits first: contiguous tiles of up to 2^12; then the bits above in
    // passes of up to 2^10 over 4 adjacent columns
    int done = 0;
    while (done < nb) {
        const int lb = done;
        const int cb = std::min(MOBIUS_RUN_BITS, lb);
        const int rb = std::min(nb - done, TILE_BITS - cb);
        const uint64_t blocks = uint64_t{1} << (nb - rb - cb);
        const size_t lds = size_t{16} << (rb + cb);
        if (blocks > 0x7FFFFFFFull) return fail_msg(c, "Moebius pass exceeds its launch limits");
        if (set_lds(c, mobius_pass, lds)) return -1;
        hipLaunchKernelGGL(mobius_pass, dim3(static_cast<unsigned>(blocks)), dim3(THREADS), lds, c->stream, a, rb,
                           lb, cb, inverse ? 1 : 0);
        VMX_HIP(c, hipGetLastError());
        done += rb;
    }
    return 0;
}

}  // namespace vmx
