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
// Layout: Fp2 in HBM as (c0, c1) u64 pairs, 16 bytes, the ABI's layout.
// Transforms of up to 2^12 points run in one workgroup, the tile split into a
// c0 plane and a c1 plane of u64 in LDS (radix-2^2 butterflies, lds_dit.hpp);
// larger ones run as passes of register four-steps (ntt_reg.hip).
#include <hip/hip_runtime.h>

#include <algorithm>

#include "context.hpp"
#include "gl64.hpp"
#include "gl64_shift.hpp"
#include "kernels.hpp"
#include "lds_dit.hpp"
#include "ntt_reg.hpp"

namespace vmx {
namespace x4 {

using u64x2 = uint64_t __attribute__((ext_vector_type(2)));

using nreg::THREADS;
constexpr int GBITS = nreg::GBITS;  // inner table: w_4096^j, j < 2048
constexpr int TILE_BITS = 12;       // one-pass transforms and Moebius tiles: 2^12 Fp2 (64 KiB of LDS)
constexpr int MOBIUS_RUN_BITS = 3;  // Moebius passes above the first: 8 adjacent columns
constexpr uint64_t INV2 = 0x7FFFFFFF80000001ull;  // (p + 1) / 2
using nreg::ROOT33_C1;
using nreg::Digits;
using nreg::tile_id;
using nreg::gather_tile;
using nreg::mul7;
using nreg::root_pow;

// x / 2 for canonical x: x >> 1, plus (p + 1) / 2 when x is odd.
__device__ __forceinline__ uint64_t halve(uint64_t x) { return (x >> 1) + ((x & 1) ? INV2 : 0); }

// Fp2 product (phi^2 = 7), three base products (Karatsuba).
__device__ __forceinline__ u64x2 fp2_mul(u64x2 a, u64x2 b) {
    const uint64_t p0 = gl::mul32x4(a.x, b.x), p1 = gl::mul32x4(a.y, b.y);
    const uint64_t s = gl::mul32x4(gl::add(a.x, a.y), gl::add(b.x, b.y));
    return u64x2{gl::add(p0, mul7(p1)), gl::sub(s, gl::add(p0, p1))};
}

// ---- NTT passes ------------------------------------------------------------------------

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
    uint64_t y = halve(root_pow((uint64_t{0} - (j0 + j)) & mask, nb, split, h, imag));
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

// LDS word of tile index i: one word of padding per 16 keeps the rounds below
// free of bank conflicts (a round's lanes step by 1, 17 or 272 words).
__device__ __forceinline__ uint32_t mob_slot(uint32_t i) { return i + (i >> 4); }

// One round of the Moebius transform on the tile in LDS: bits [b, b + K) of
// the middle index, all K of them in registers.  Group g takes the 2^K
// elements of one (plane-column, the other bits of i); the bits' updates
// commute, so any grouping of the bits gives the same result.
template <int K>
__device__ __forceinline__ void mobius_round(uint64_t* s, int b, int rb, uint32_t planecols, int inverse) {
    const uint32_t lo_mask = (1u << b) - 1, hi_bits = static_cast<uint32_t>(rb - b - K);
    const uint32_t groups = planecols << (rb - K);
    for (uint32_t g = threadIdx.x; g < groups; g += THREADS) {
        const uint32_t lo = g & lo_mask, hi = (g >> b) & ((1u << hi_bits) - 1), pc = g >> (rb - K);
        const uint32_t i0 = (pc << rb) + lo + (hi << (b + K));
        uint64_t v[1 << K];
        gl::static_for<0, (1 << K)>([&](auto m_) {
            constexpr int m = decltype(m_)::value;
            v[m] = s[mob_slot(i0 + (static_cast<uint32_t>(m) << b))];
        });
        gl::static_for<0, K>([&](auto j_) {
            constexpr int j = decltype(j_)::value;
            gl::static_for<0, (1 << K)>([&](auto m_) {
                constexpr int m = decltype(m_)::value;
                if constexpr ((m >> j) & 1) v[m] = inverse ? gl::add(v[m], v[m ^ (1 << j)]) : gl::sub(v[m], v[m ^ (1 << j)]);
            });
        });
        gl::static_for<0, (1 << K)>([&](auto m_) {
            constexpr int m = decltype(m_)::value;
            s[mob_slot(i0 + (static_cast<uint32_t>(m) << b))] = v[m];
        });
    }
}

// One pass over the middle index of [H][R][L] (R = 2^rb, L = 2^lb): for every
// bit of i, the element with the bit set gains (inverse) or loses the one
// without.  Workgroup (h, l0) takes C = 2^cb adjacent columns; the bits are
// applied up to four at a time in registers, with the tile in LDS in between.
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
        s[mob_slot((c << rb) + i)] = v.x;
        s[mob_slot(CR + (c << rb) + i)] = v.y;
    }
    __syncthreads();
    for (int b = 0; b < rb; b += 4) {
        switch (rb - b >= 4 ? 4 : rb - b) {
            case 4: mobius_round<4>(s, b, rb, 2 * C, inverse); break;
            case 3: mobius_round<3>(s, b, rb, 2 * C, inverse); break;
            case 2: mobius_round<2>(s, b, rb, 2 * C, inverse); break;
            default: mobius_round<1>(s, b, rb, 2 * C, inverse); break;
        }
        __syncthreads();
    }
    for (uint32_t e = threadIdx.x; e < CR; e += THREADS) {
        const uint32_t i = e >> cb, c = e & (C - 1);
        a[base + (static_cast<uint64_t>(i) << lb) + c] = u64x2{s[mob_slot((c << rb) + i)], s[mob_slot(CR + (c << rb) + i)]};
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

// w(2^nb)^e on the host as (value, imaginary), the device's root_pow (ntt_reg.hpp).
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
    if (nb > TILE_BITS) {
        RegTables rt;
        rt.inner = tb.inner;
        rt.split = tb.split;
        rt.split_h = tb.split_h;
        return reg_ntt(c, rt, reinterpret_cast<const uint64_t*>(in), 0, len, reinterpret_cast<uint64_t*>(out), 1, nb,
                       2, false);
    }
    // the whole transform in one workgroup's tile
    const Digits d{};
    const size_t lds = size_t{16} << nb;
    if (set_lds(c, gather_pass, lds)) return -1;
    hipLaunchKernelGGL(gather_pass, dim3(1), dim3(THREADS), lds, c->stream, reinterpret_cast<const u64x2*>(in), len,
                       reinterpret_cast<u64x2*>(out), nb, nb, 0, d, tb.inner);
    VMX_HIP(c, hipGetLastError());
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
        const size_t words = size_t{2} << (rb + cb);  // two planes
        const size_t lds = (words + (words >> 4) + 1) * sizeof(uint64_t);  // + the slots' padding
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
