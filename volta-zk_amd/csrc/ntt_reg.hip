// ntt_reg.hip -- batched NTTs of 2^13 .. 2^33 points as passes over HBM,
// each pass a register four-step; used by the base-field transforms
// (ntt.hip: NttPlan::forward semantics, rust/volta-pcs/src/ntt.rs:34-70) and by
// the X4 Fp2 transform (x4.hip, rust/volta-pcs/src/x4/ntt.rs:66-122).
//
// An n = 2^nb point transform, n = R_1 R_2 .. R_P with every R_p <= 2^8 (2^9 for
// one-plane rows below 2^26, ntt_reg.hpp: pass_bits), runs in
// P passes (decimation in time by the least significant input digit first):
//   pass 1 ("gather"): row r = (i_1, .., i_(P-1)) (i_1 most significant) gets
//     the R_P-point DFT of x[nat(r) + (n / R_P) j], j < R_P, with
//     nat(r) = i_1 + R_1 (i_2 + R_2 (..)), stored contiguously as row r of
//     the output.  A tile takes adjacent rows (adjacent i_1), so its reads are
//     runs of 128 or 256 bytes.  Inputs at index >= len (the caller's zero
//     tail) are read as zero and never stored.
//   passes P-1 .. 1 ("columns"): the output is [H][R_p][L]
//     (H = R_1 .. R_(p-1), L = R_(p+1) .. R_P); element (i, l) is multiplied by
//     w(n)^(H i l) as it loads and column l gets the R_p-point DFT over i, in
//     place.  A tile takes adjacent columns.
// Each pass reads and writes every element once.  The roots are the X4 roots
// (ntt_reg.hpp), which are the base field's for n <= 2^31.
//
// Each R = A B point DFT (A = 2^LA <= 32, B = 2^LB <= 16) is a four-step inside
// the tile, with input index j = ja B + jb and output index k = ka + A kb:
//   step 1: one thread takes the A inputs of one (coordinate, column, jb)
//     straight from HBM into registers, DFTs them over ja with shift-only
//     twiddles (every root of order <= 64 is a power of two), multiplies
//     output ka by w_R^(jb ka) and parks them in LDS;
//   step 2: one thread takes the B values of one (coordinate, column, ka),
//     DFTs them over jb and stores Y[ka + A kb] straight to HBM.
// LDS holds (coordinate, column) pairs fastest, then jb, then ka with a pitch
// of PW (B + 1) words (column passes) or PW B + 32 / A words (the gather,
// whose step 2 takes ka fastest so that its stores cover whole lines), so
// both steps' accesses avoid bank conflicts.
//
// Elements are PL u64 wide (PL = 1: Fp; PL = 2: Fp2, coordinate p of element e
// at 2 e + p); each coordinate is transformed independently, except that the
// imaginary twiddles of an X4 transform of 2^33 points mix them.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "context.hpp"
#include "gl64.hpp"
#include "gl64_shift.hpp"
#include "kernels.hpp"
#include "ntt_reg.hpp"

namespace vmx {
namespace nreg {

// Exponent of the base root of order 2^L (L <= 6) as a power of two:
// w_64 = 2^39, so w_(2^L) = 2^(39 2^(6-L)), exponents mod 192.
template <int L>
constexpr int ew_log() {
    return (gl::E_W64 << (6 - L)) % 192;
}

// w_4096^e for e < 4096 from the inner table (w_4096^j, j < 2048; w_4096^2048 = -1).
// The load is unconditional and the sign a select, so no branch splits a
// tile's loads.
__device__ __forceinline__ uint64_t inner_pow(const uint64_t* inner, uint32_t e) {
    const uint64_t v = inner[e & 2047];
    return (e & 2048) ? gl::neg(v) : v;
}

// The partner lane's value (lane ^ 1): the other coordinate of the same element.
__device__ __forceinline__ uint64_t partner(uint64_t v) {
    const uint32_t lo = static_cast<uint32_t>(__shfl_xor(static_cast<int>(static_cast<uint32_t>(v)), 1));
    const uint32_t hi = static_cast<uint32_t>(__shfl_xor(static_cast<int>(static_cast<uint32_t>(v >> 32)), 1));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

// The R = A B inner twiddles w_R^(jb ka) of a tile, at ptw[jb A + ka] in LDS:
// filled once per workgroup (R <= 512 words, two per thread at most) so that
// step 1 reads each with one LDS load instead of an index, a table load and a
// sign select.  The caller synchronises before the first park().
template <int LA, int LB>
__device__ __forceinline__ void fill_park_twiddles(uint64_t* ptw, const uint64_t* inner) {
    constexpr int A = 1 << LA, RB = LA + LB;
    for (uint32_t i = threadIdx.x; i < (1u << RB); i += THREADS)
        ptw[i] = inner_pow(inner, ((i >> LA) * (i & (A - 1))) << (GBITS - RB));
}

// Step 1's tail: v (natural order over ka after the A-point DFT) times
// w_R^(jb ka), parked at (pc, jb, ka).
template <int LA, int LB>
__device__ __forceinline__ void park(uint64_t* s, const uint64_t* v, uint32_t pc, uint32_t jb, uint32_t PW,
                                     uint32_t pitch, const uint64_t* ptw) {
    constexpr int A = 1 << LA;
    s[pc + PW * jb] = v[0];
    const uint64_t* row = ptw + jb * A;
    gl::static_for<1, A>([&](auto ka_) {
        constexpr int ka = decltype(ka_)::value;
        s[pc + PW * jb + ka * pitch] = gl::mul32x4(v[ka], row[ka]);
    });
}

// Step 2's head: the B values of (pc, ka), DFT'd over jb (natural order over kb).
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

// Inputs of the gather pass.  Row `row` of a batch, element idx < n,
// coordinate `plane`.  fetch() only loads (from an index clamped into the
// row, so every load is unconditional and in bounds); finish() masks the
// zero tail and applies any scaling, after all of a tile's loads are issued.
// SrcU64: x + row x_stride elements of PL u64, len elements then zeros; with
//   reverse the transform reads index (n - idx) mod n (the inverse transform
//   as a forward one) and every input is multiplied by scale unless it is 1.
//   For len = 0 the host points x at the inner table with stride 0: fetch()
//   reads its word 0, and finish() masks every input to zero.
struct SrcU64 {
    const uint64_t* x;
    uint64_t x_stride, len;
    int reverse;
    uint64_t scale;
    struct Raw {
        uint64_t v;
    };
    // Inputs at index >= extent(n) are zero.
    __host__ __device__ uint64_t extent(uint64_t n) const { return reverse || len > n ? n : len; }
    __device__ __forceinline__ uint64_t index(uint64_t idx, uint64_t nmask) const {
        return reverse ? (uint64_t{0} - idx) & nmask : idx;
    }
    // Offset of the gather's rows against its tiles (see gather_reg).
    __device__ __forceinline__ uint32_t rotation() const { return reverse ? 1u : 0u; }
    // A tile's u64 runs are whole lines: tiles go to the XCDs round-robin.
    static constexpr bool SWIZZLE = false;
    __device__ __forceinline__ Raw fetch(uint64_t row, uint64_t idx, uint32_t plane, int PL) const {
        const uint64_t ci = idx < len ? idx : 0;
        return Raw{x[(row * x_stride + ci) * PL + plane]};
    }
    __device__ __forceinline__ uint64_t finish(uint64_t idx, Raw r) const {
        uint64_t v = idx < len ? r.v : 0;
        if (scale != 1) v = gl::mul32x4(v, scale);
        return v;
    }
};
// SrcMsgI16: the Ligero message row lift(w) || pads || 0 (reference
//   pcs_messages_kernel, cuda/volta_cuda_backend.cu:2950-2958): cols i16
//   weights lifted as signed residues, then pad u64 pads, then zeros.
//   w and pads always point at readable words: for cols = 0 or pad = 0 the
//   host points them at the inner table, whose words are then masked out.
struct SrcMsgI16 {
    const int16_t* w;
    const uint64_t* pads;
    uint64_t cols, pad;
    struct Raw {
        int16_t w;
        uint64_t p;
    };
    __host__ __device__ uint64_t extent(uint64_t n) const { return cols + pad > n ? n : cols + pad; }
    __device__ __forceinline__ uint64_t index(uint64_t idx, uint64_t) const { return idx; }
    __device__ __forceinline__ uint32_t rotation() const { return 0u; }
    // A tile's i16 runs are 32 bytes, a quarter of a line: consecutive tiles
    // run on one XCD so that the line is fetched into its L2 once.
    static constexpr bool SWIZZLE = true;
    __device__ __forceinline__ Raw fetch(uint64_t row, uint64_t idx, uint32_t, int) const {
        const uint64_t wi = idx < cols ? idx : 0;
        const uint64_t pi = idx >= cols && idx - cols < pad ? idx - cols : 0;
        return Raw{w[row * cols + wi], pads[row * pad + pi]};
    }
    __device__ __forceinline__ uint64_t finish(uint64_t idx, Raw r) const {
        return idx < cols ? gl::from_i16(r.w) : idx - cols < pad ? r.p : 0;
    }
};

// Positions of step 1's bit-reversed register array that hold ja < NZ.
constexpr uint64_t prefix_mask(int nz, int la) {
    uint64_t m = 0;
    for (int ja = 0; ja < nz; ++ja) m |= uint64_t{1} << gl::bitrev_c(ja, la);
    return m;
}

// Output row of the gather row whose inputs sit at x[L + (n / R) j]
// (L < n / R, R = 2^rb): i_1 = the low r1 bits of L, most significant in the
// row index, then the middle digits of L in reverse order (gather_tile's map).
__device__ __forceinline__ uint64_t gather_row(uint64_t L, const Digits& d, int mid_bits) {
    const uint64_t i1 = L & ((uint64_t{1} << d.r1) - 1), m = L >> d.r1;
    uint64_t rest = 0;
    int shift = mid_bits, scale = 0;
    for (int j = 0; j < d.count; ++j) {
        shift -= d.bits[j];
        rest += ((m >> scale) & ((uint64_t{1} << d.bits[j]) - 1)) << shift;
        scale += d.bits[j];
    }
    return (i1 << mid_bits) + rest;
}

// Gather pass of row blockIdx.y of a batch: tile of 2^qb rows, inputs from
// src, output rows n elements apart.  Step 1 reads only ja < NZ: the host
// picks NZ so that every input with ja >= NZ lies in the zero tail
// (ja B + jb >= NZ B puts the index at >= NZ n / A >= the source's extent),
// and the A-point DFT skips the butterflies that only meet those zeros.
// A source read at (n - idx) mod n (the inverse transform) has rotation 1:
// lane t of a tile takes row L = nat0 + t + 1 (mod n / R) instead of
// nat0 + t, so that its reads n - L - (n / R) j of one (ja, jb) cover the
// aligned run [n / R - nat0 - 2^qb, n / R - nat0) + (n / R)(R - 1 - j): one
// 128-byte line per run instead of two (only the wrap to L = 0 in the last
// tile straddles).  The rows still cover 0 .. n / R - 1 once.
template <int LA, int LB, int PL, int NZ, class Src>
__global__ __launch_bounds__(THREADS) void gather_reg(Src src, uint64_t* __restrict__ y, int nb, int qb, Digits d,
                                                      const uint64_t* inner) {
    constexpr int A = 1 << LA, B = 1 << LB, RB = LA + LB;
    static_assert(NZ >= 1 && NZ <= A, "step 1 reads between 1 and A inputs");
    extern __shared__ uint64_t s[];
    const uint64_t row = blockIdx.y;
    y += (row << nb) * PL;
    const int pwb = qb + (PL - 1);  // (coordinate, row) pairs: 2^pwb
    const uint32_t PW = 1u << pwb;
    // Step 2 runs ka fastest, so each store writes A adjacent outputs of a row
    // (whole 128-byte lines for A = 16).  Its LDS reads, (pc, ka) at
    // pc + ka pitch, then meet distinct banks in every 32-lane group when
    // pitch = 32 / A (mod 32) words; step 1's writes are contiguous per ka.
    const uint32_t pitch = PW * B + 32 / A;
    uint64_t* ptw = s + A * pitch;  // the inner twiddles follow the tile
    fill_park_twiddles<LA, LB>(ptw, inner);
    __syncthreads();
    uint64_t nat0, row0;
    int mid_bits;
    gather_tile<Src::SWIZZLE>(nb, RB, qb, d, nat0, row0, mid_bits);
    const int sh = nb - RB;
    const uint64_t nmask = (uint64_t{1} << nb) - 1, lmask = (uint64_t{1} << sh) - 1;
    const uint32_t rot = sh > 0 ? src.rotation() : 0u;
    // Step 1 (loads, A-point DFTs) issues at a higher wave priority than step 2
    // (B-point DFTs, stores), so co-resident workgroups interleave their
    // phases (measured: C4 +6%, p15 +3%, X4 2^24 +3%, C5 and p17 within 2%).
    __builtin_amdgcn_s_setprio(1);
    for (uint32_t job = threadIdx.x; job < (PW << LB); job += THREADS) {
        const uint32_t pc = job & (PW - 1), jb = job >> pwb;
        const uint32_t plane = PL == 2 ? (pc & 1) : 0, t = PL == 2 ? (pc >> 1) : pc;
        const uint64_t L = (nat0 + t + rot) & lmask;
        typename Src::Raw raw[NZ];
        gl::static_for<0, NZ>([&](auto ja_) {
            constexpr int ja = decltype(ja_)::value;
            const uint64_t idx = src.index(L + ((static_cast<uint64_t>(ja) * B + jb) << sh), nmask);
            raw[ja] = src.fetch(row, idx, plane, PL);
        });
        uint64_t v[A];
        gl::static_for<0, A>([&](auto i_) { v[decltype(i_)::value] = 0; });
        gl::static_for<0, NZ>([&](auto ja_) {
            constexpr int ja = decltype(ja_)::value;
            const uint64_t idx = src.index(L + ((static_cast<uint64_t>(ja) * B + jb) << sh), nmask);
            v[gl::bitrev_c(ja, LA)] = src.finish(idx, raw[ja]);
        });
        gl::dit_pow2_sparse<LA, ew_log<LA>(), prefix_mask(NZ, LA)>(v);
        park<LA, LB>(s, v, pc, jb, PW, pitch, ptw);
    }
    __syncthreads();
    __builtin_amdgcn_s_setprio(0);
    for (uint32_t job = threadIdx.x; job < (PW << LA); job += THREADS) {
        const uint32_t ka = job & (A - 1), pc = job >> LA;
        const uint32_t plane = PL == 2 ? (pc & 1) : 0, t = PL == 2 ? (pc >> 1) : pc;
        uint64_t v[B];
        unpark<LB>(s, v, pc, ka, PW, pitch);
        const uint64_t orow =
            rot ? gather_row((nat0 + t + rot) & lmask, d, mid_bits) : row0 + (static_cast<uint64_t>(t) << mid_bits);
        const uint64_t out0 = (orow << RB) + ka;
        gl::static_for<0, B>([&](auto kb_) {
            constexpr int kb = decltype(kb_)::value;
            y[PL * (out0 + A * kb) + plane] = v[kb];
        });
    }
}

// Column pass of row blockIdx.y of a batch, in place (rows n elements
// apart).  The array is [H][R][L] (H = 2^hb, R = 2^(LA+LB), L = 2^lb,
// n = 2^nb); the tile takes the 2^cb adjacent columns l0 .. of block h:
// element (i, l) is multiplied by w(n)^(H i l) as it loads, then each column
// gets the R-point DFT over i.  For an X4 transform of 2^33 points the last
// pass (hb = 0) meets imaginary twiddles, which mix the two coordinates: each
// lane then also reads its partner lane's coordinate.
// With TBL the pre-twiddles come from ctab[(i << lb) + l] = w(n)^(H i l), a
// table of R L words (the host builds it on first use); without, from the
// two-level table split, and then every output is also multiplied by scale
// (one product per job, on t0): the inverse transform's n^-1 when this is its
// last pass.  With rows_inner the dispatch order runs every row's copy of a
// tile back to back (workgroup d of the grid takes tile d / rows, row
// d mod rows), so a large table's slice for that tile is read from HBM about
// once per XCD (workgroups go round-robin over the 8 XCDs) instead of once per
// row.  Keeping all rows of a tile on one XCD, so that the slice is read once,
// measured 2.7% slower on C5.
template <int LA, int LB, int PL, int MODE, bool TBL>
__global__ __launch_bounds__(THREADS) void col_reg(uint64_t* a, int nb, int hb, int lb, int cb, const uint64_t* inner,
                                                   const uint64_t* split, int split_h, const uint64_t* ctab,
                                                   uint64_t scale, int rows_inner) {
    static_assert(PL == 2 || MODE == ROOT_BASE, "one-plane transforms stop at 2^31 points");
    static_assert(!TBL || MODE == ROOT_BASE, "column tables hold real roots");
    constexpr int A = 1 << LA, B = 1 << LB, RB = LA + LB;
    extern __shared__ uint64_t s[];
    uint64_t row = blockIdx.y, blk = tile_id();
    if (rows_inner) {
        const uint64_t d = blockIdx.x + static_cast<uint64_t>(gridDim.x) * blockIdx.y;
        blk = d / gridDim.y;
        row = d - blk * gridDim.y;
    }
    a += (row << nb) * PL;
    const int pwb = cb + (PL - 1);
    const uint32_t PW = 1u << pwb;
    const uint32_t pitch = PW * (B + 1);
    uint64_t* ptw = s + A * pitch;  // the inner twiddles follow the tile
    fill_park_twiddles<LA, LB>(ptw, inner);
    __syncthreads();
    const uint64_t lblocks = (uint64_t{1} << lb) >> cb;
    const uint64_t h = blk / lblocks;
    const uint64_t l0 = (blk - h * lblocks) << cb;
    const uint64_t base = ((h << RB) << lb) + l0;
    const bool mixed = MODE == ROOT_IMAG33 && hb == 0;  // uniform
    // Step 1 (loads, A-point DFTs) issues at a higher wave priority than step 2
    // (B-point DFTs, stores), so co-resident workgroups interleave their
    // phases (measured: C4 +6%, p15 +3%, X4 2^24 +3%, C5 and p17 within 2%).
    __builtin_amdgcn_s_setprio(1);
    for (uint32_t job = threadIdx.x; job < (PW << LB); job += THREADS) {
        const uint32_t pc = job & (PW - 1), jb = job >> pwb;
        const uint32_t plane = PL == 2 ? (pc & 1) : 0, c = PL == 2 ? (pc >> 1) : pc;
        const uint64_t l = l0 + c;
        uint64_t v[A];
        if constexpr (TBL) {
            // the job's A inputs and A table words, all in flight, then A products
            uint64_t xv[A], tv[A];
            gl::static_for<0, A>([&](auto ja_) {
                constexpr int ja = decltype(ja_)::value;
                const uint64_t i = static_cast<uint64_t>(ja) * B + jb;
                xv[ja] = a[PL * (base + (i << lb) + c) + plane];
                tv[ja] = ctab[(i << lb) + l];
            });
            __builtin_amdgcn_sched_barrier(0);
            gl::static_for<0, A>([&](auto ja_) {
                constexpr int ja = decltype(ja_)::value;
                v[gl::bitrev_c(ja, LA)] = gl::mul32x4(xv[ja], tv[ja]);
            });
        } else if constexpr (MODE != ROOT_IMAG33) {
            // real roots: the pre-twiddles w^(H l (ja B + jb)) are t0 s^ja with
            // t0 = w^(H l jb) and s = w^(H l B); the job loads its A inputs and
            // four table words, then multiplies along the progression
            uint64_t xv[A];
            gl::static_for<0, A>([&](auto ja_) {
                constexpr int ja = decltype(ja_)::value;
                const uint64_t i = static_cast<uint64_t>(ja) * B + jb;
                xv[ja] = a[PL * (base + (i << lb) + c) + plane];
            });
            const uint64_t e0 = (static_cast<uint64_t>(jb) * l) << hb, es = (static_cast<uint64_t>(B) * l) << hb;
            const uint64_t hmask = (uint64_t{1} << split_h) - 1;
            const uint64_t p0 = split[e0 & hmask], q0 = split[hmask + 1 + (e0 >> split_h)];
            const uint64_t p1 = split[es & hmask], q1 = split[hmask + 1 + (es >> split_h)];
            __builtin_amdgcn_sched_barrier(0);  // every load of the job is in flight before the arithmetic
            uint64_t t = gl::mul32x4(p0, q0);
            uint64_t st = gl::mul32x4(p1, q1);
            if (scale != 1) t = gl::mul32x4(t, scale);
            if constexpr (MODE == ROOT_NEG32) {  // w(2^32)^e = (-1)^e b_32^e
                if (e0 & 1) t = gl::neg(t);
                if (es & 1) st = gl::neg(st);
            }
            gl::static_for<0, A>([&](auto ja_) {
                constexpr int ja = decltype(ja_)::value;
                v[gl::bitrev_c(ja, LA)] = gl::mul32x4(xv[ja], t);
                if constexpr (ja + 1 < A) t = gl::mul32x4(t, st);
            });
        } else {
            // all of this job's loads first (data and both twiddle-table words),
            // then the arithmetic: the loads are in flight together
            uint64_t xv[A], tlo[A], thi[A];
            const uint64_t hmask = (uint64_t{1} << split_h) - 1;
            gl::static_for<0, A>([&](auto ja_) {
                constexpr int ja = decltype(ja_)::value;
                const uint64_t i = static_cast<uint64_t>(ja) * B + jb;
                xv[ja] = a[PL * (base + (i << lb) + c) + plane];
                const uint64_t e = (i * l) << hb;
                const uint64_t q = MODE == ROOT_IMAG33 ? e >> 1 : e;
                tlo[ja] = split[q & hmask];
                thi[ja] = split[hmask + 1 + (q >> split_h)];
            });
            __builtin_amdgcn_sched_barrier(0);
            gl::static_for<0, A>([&](auto ja_) {
                constexpr int ja = decltype(ja_)::value;
                const uint64_t i = static_cast<uint64_t>(ja) * B + jb;
                const uint64_t e = (i * l) << hb;
                uint64_t t = gl::mul32x4(tlo[ja], thi[ja]);
                bool imag = false;
                if constexpr (MODE == ROOT_NEG32) {
                    t = (e & 1) ? gl::neg(t) : t;
                } else if constexpr (MODE == ROOT_IMAG33) {
                    if ((e >> 1) & 1) t = gl::neg(t);
                    imag = (e & 1) != 0;
                    const uint64_t ti = gl::mul32x4(ROOT33_C1, t);
                    t = imag ? ti : t;
                }
                const uint64_t xvv = xv[ja];
                uint64_t r;
                if constexpr (MODE == ROOT_IMAG33) {
                    if (mixed) {
                        const uint64_t other = partner(xvv);
                        r = !imag ? gl::mul32x4(xvv, t)
                                  : plane == 0 ? mul7(gl::mul32x4(other, t)) : gl::mul32x4(other, t);
                    } else {
                        r = gl::mul32x4(xvv, t);
                    }
                } else {
                    r = gl::mul32x4(xvv, t);
                }
                v[gl::bitrev_c(ja, LA)] = r;
            });
        }
        gl::dit_pow2<LA, ew_log<LA>()>(v);
        park<LA, LB>(s, v, pc, jb, PW, pitch, ptw);
    }
    __syncthreads();
    __builtin_amdgcn_s_setprio(0);
    for (uint32_t job = threadIdx.x; job < (PW << LA); job += THREADS) {
        const uint32_t pc = job & (PW - 1), ka = job >> pwb;
        const uint32_t plane = PL == 2 ? (pc & 1) : 0, c = PL == 2 ? (pc >> 1) : pc;
        uint64_t v[B];
        unpark<LB>(s, v, pc, ka, PW, pitch);
        gl::static_for<0, B>([&](auto kb_) {
            constexpr int kb = decltype(kb_)::value;
            a[PL * (base + ((static_cast<uint64_t>(ka) + A * kb) << lb) + c) + plane] = v[kb];
        });
    }
}

// Column-pass table of an m = R L point column span, R = 2^rb, L = 2^lb, from
// the two-level table of w = w(n), n = m 2^hb: out[(i << lb) + l] = w^((i l) << hb)
// = w(m)^(i l), whatever n it is built from, times scale.
__global__ void col_table(const uint64_t* split, int split_h, int hb, int rb, int lb, uint64_t scale,
                          uint64_t* out) {
    const uint64_t total = uint64_t{1} << (rb + lb), lmask = (uint64_t{1} << lb) - 1;
    for (uint64_t j = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; j < total;
         j += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        const uint64_t t = tw_split(split, ((j >> lb) * (j & lmask)) << hb, split_h);
        out[j] = scale == 1 ? t : gl::mul32x4(t, scale);
    }
}

// Tables for the passes from the reference's table fwd = w^0 .. w^(n/2 - 1),
// n = 2^nb >= 2^13: out = [w_4096^j, j < 2048][w^j, j < 2^h][w^(j 2^h), j < 2^(nb-h)].
__global__ void derive_tables(const uint64_t* fwd, int nb, int h, uint64_t* out) {
    const uint64_t half = uint64_t{1} << (nb - 1);
    const uint64_t lo = uint64_t{1} << h, hi = uint64_t{1} << (nb - h);
    const uint64_t total = 2048 + lo + hi;
    for (uint64_t j = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; j < total;
         j += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        uint64_t e;
        if (j < 2048) e = j << (nb - GBITS);
        else if (j < 2048 + lo) e = j - 2048;
        else e = (j - 2048 - lo) << h;
        out[j] = e < half ? fwd[e] : gl::neg(fwd[e - half]);
    }
}

}  // namespace nreg

namespace {

template <class Src>
using GatherFn = void (*)(Src, uint64_t*, int, int, nreg::Digits, const uint64_t*);
using ColFn = void (*)(uint64_t*, int, int, int, int, const uint64_t*, const uint64_t*, int, const uint64_t*,
                      uint64_t, int);

// Column passes whose span R L is at most 2^COL_TABLE_BITS points read their
// pre-twiddles from a table of R L words (2 MiB at most, L2-resident); larger
// spans build them from the two-level table, except the last pass of a batch
// of at least BIG_TABLE_ROWS transforms of at most 2^BIG_TABLE_BITS points,
// which reads a table of n words (128 MiB at 2^24; times n^-1 for an inverse)
// with every row's copy of a tile dispatched back to back.
constexpr int COL_TABLE_BITS = 18;
constexpr int BIG_TABLE_BITS = 24;
constexpr uint64_t BIG_TABLE_ROWS = 16;

template <int LA, int LB, int PL>
ColFn col_for(int mode, bool tbl) {
    if constexpr (PL == 2) {
        if (mode == nreg::ROOT_NEG32) return nreg::col_reg<LA, LB, PL, nreg::ROOT_NEG32, false>;
        if (mode == nreg::ROOT_IMAG33) return nreg::col_reg<LA, LB, PL, nreg::ROOT_IMAG33, false>;
    }
    if (mode != nreg::ROOT_BASE) return nullptr;
    return tbl ? nreg::col_reg<LA, LB, PL, nreg::ROOT_BASE, true> : nreg::col_reg<LA, LB, PL, nreg::ROOT_BASE, false>;
}

// The gather kernel whose step 1 reads the fewest inputs covering nza: NZ is
// compiled for the powers of two and for A / 4 + 1, which covers a message of
// just over a quarter of the row (cols + 512 pads at rate 1/4).
template <int LA, int LB, int PL, class Src>
GatherFn<Src> gather_for(uint64_t nza) {
    constexpr int A = 1 << LA;
    if (nza <= 1) return nreg::gather_reg<LA, LB, PL, 1, Src>;
    if (nza <= 2) return nreg::gather_reg<LA, LB, PL, 2, Src>;
    if constexpr (A == 8) {
        if (nza <= 3) return nreg::gather_reg<LA, LB, PL, 3, Src>;
        if (nza <= 4) return nreg::gather_reg<LA, LB, PL, 4, Src>;
    } else {
        if (nza <= 4) return nreg::gather_reg<LA, LB, PL, 4, Src>;
        if (nza <= A / 4 + 1) return nreg::gather_reg<LA, LB, PL, A / 4 + 1, Src>;
        if (nza <= 8) return nreg::gather_reg<LA, LB, PL, 8, Src>;
        if constexpr (A == 32) {
            if (nza <= 16) return nreg::gather_reg<LA, LB, PL, 16, Src>;
        }
    }
    return nreg::gather_reg<LA, LB, PL, A, Src>;
}

// Kernels of a pass of radix 2^rb; nza = how many of step 1's A inputs per
// job can be nonzero (the gather's), tbl = the column pass reads a column
// table.
template <int PL, class Src>
bool kernels_for(int rb, int mode, uint64_t nza, bool tbl, GatherFn<Src>* g, ColFn* col) {
    switch (rb) {
        case 5: *g = gather_for<3, 2, PL, Src>(nza); *col = col_for<3, 2, PL>(mode, tbl); break;
        case 6: *g = gather_for<3, 3, PL, Src>(nza); *col = col_for<3, 3, PL>(mode, tbl); break;
        case 7: *g = gather_for<4, 3, PL, Src>(nza); *col = col_for<4, 3, PL>(mode, tbl); break;
        case 8: *g = gather_for<4, 4, PL, Src>(nza); *col = col_for<4, 4, PL>(mode, tbl); break;
        case 9:
            if constexpr (PL == 1) {
                *g = gather_for<5, 4, PL, Src>(nza);
                *col = col_for<5, 4, PL>(mode, tbl);
                break;
            }
            return false;
        default: return false;
    }
    return *col != nullptr;
}

// Pass radices: the fewest passes of at most 2^pass_bits, as even as possible.
int plan(int nb, int planes, int* r) {
    const int pb = nreg::pass_bits(nb, planes);
    const int passes = (nb + pb - 1) / pb;
    if (nb < nreg::MIN_BITS || passes > nreg::MAX_PASSES) return 0;
    for (int p = 0; p < passes; ++p) r[p] = nb / passes + (p < nb % passes ? 1 : 0);
    return passes;
}

// LDS bytes of a column tile: 2^pwb (coordinate, column) pairs x A x (B + 1)
// words, then the R = A B inner twiddles.
size_t tile_lds(int rb, int pwb) {
    const size_t A = size_t{1} << ((rb + 1) / 2), B = size_t{1} << (rb / 2);
    return ((size_t{1} << pwb) * A * (B + 1) + A * B) * sizeof(uint64_t);
}

// LDS bytes of a gather tile: A rows of 2^pwb B words, each padded by 32 / A,
// then the R = A B inner twiddles.
size_t gather_lds(int rb, int pwb) {
    const size_t A = size_t{1} << ((rb + 1) / 2), B = size_t{1} << (rb / 2);
    return (((size_t{1} << pwb) * B) * A + 32 + A * B) * sizeof(uint64_t);
}

template <class K>
int allow_lds(Context* c, K kernel, size_t lds) {
    if (lds <= 65536) return 0;
    VMX_HIP(c, hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
    return 0;
}

}  // namespace

bool reg_ntt_covers(uint64_t n) {
    int r[nreg::MAX_PASSES];
    int nb = 0;
    while ((uint64_t{1} << nb) < n) ++nb;
    return (uint64_t{1} << nb) == n && plan(nb, 1, r) > 0;
}

int derive_reg_tables(Context* c, TwiddleSet* t) {
    if (t->reg) return 0;
    int nb = 0;
    while ((size_t{1} << nb) < t->n) ++nb;
    if (nb < nreg::MIN_BITS || nb > 31 || !t->fwd) return fail_msg(c, "pass tables need a size in [2^13, 2^31]");
    const int h = (nb + 1) / 2;
    const size_t words = 2048 + (size_t{1} << h) + (size_t{1} << (nb - h));
    void* p = nullptr;
    VMX_HIP(c, hipMalloc(&p, words * sizeof(uint64_t)));
    ++c->stats.allocation_calls;
    c->stats.live_device_bytes += words * sizeof(uint64_t);
    c->stats.peak_device_bytes = std::max(c->stats.peak_device_bytes, c->stats.live_device_bytes);
    t->reg = static_cast<uint64_t*>(p);
    t->reg_bytes = words * sizeof(uint64_t);
    t->reg_h = h;
    hipLaunchKernelGGL(nreg::derive_tables, dim3(static_cast<unsigned>((words + 255) / 256)), dim3(256), 0, c->stream,
                       static_cast<const uint64_t*>(t->fwd), nb, h, t->reg);
    VMX_HIP(c, hipGetLastError());
    return 0;
}

// The column table of a pass spanning 2^(rb + lb) points, built from this
// transform's two-level table on first use and kept with the other tables of
// that size.  Inside a coarse timing scope, where tables may not grow, a
// missing table leaves *out null and the pass builds its pre-twiddles itself.
static int col_table_for(Context* c, const RegTables& tb, int hb, int rb, int lb, const uint64_t** out,
                         uint64_t scale = 1) {
    TwiddleSet& t = c->twiddles[size_t{1} << (rb + lb)];
    t.n = size_t{1} << (rb + lb);
    uint64_t*& slot = scale == 1 ? t.col[rb] : t.col_scaled[rb];
    if (!slot) {
        if (c->coarse_active) return 0;
        const size_t bytes = (size_t{1} << (rb + lb)) * sizeof(uint64_t);
        void* p = nullptr;
        VMX_HIP(c, hipMalloc(&p, bytes));
        ++c->stats.allocation_calls;
        c->stats.live_device_bytes += bytes;
        c->stats.peak_device_bytes = std::max(c->stats.peak_device_bytes, c->stats.live_device_bytes);
        slot = static_cast<uint64_t*>(p);
        t.col_bytes += bytes;
        const unsigned blocks = static_cast<unsigned>(std::min<size_t>((size_t{1} << (rb + lb)) / 256, 4096));
        hipLaunchKernelGGL(nreg::col_table, dim3(std::max(blocks, 1u)), dim3(256), 0, c->stream, tb.split,
                           tb.split_h, hb, rb, lb, scale, slot);
        VMX_HIP(c, hipGetLastError());
    }
    *out = slot;
    return 0;
}

// The passes of rows transforms with inputs from src; shift(src, r0) moves
// src to row r0 for each launch slice of at most 65535 rows.
template <int PL, class Src, class Shift>
int run_passes(Context* c, const RegTables& tb, Src src, Shift shift, uint64_t* out, uint64_t rows, int nb) {
    int r[nreg::MAX_PASSES] = {};
    const int passes = plan(nb, PL, r);
    if (passes == 0) return fail_msg(c, "NTT size outside the pass engine's range");
    // A scaled source (the inverse transform's n^-1) hands its scale to the
    // last column pass when that pass builds its pre-twiddles as a progression
    // (span n > 2^COL_TABLE_BITS, real roots): one product per job instead of
    // one per input.
    // Column passes whose columns span at most 2^COL_TABLE_BITS points (real
    // roots only) read a column table; the last pass spans all n points.  The
    // same predicate decides the hand-off below and the table lookup of each
    // pass, and the last pass refuses a table while it holds the scale.
    auto table_span = [&](int span_bits) {
        return nreg::root_mode(nb) == nreg::ROOT_BASE && span_bits <= COL_TABLE_BITS;
    };
    // A batch of many transforms of up to 2^BIG_TABLE_BITS points: the last
    // pass reads an n-word table (scaled by the source's n^-1 for an inverse,
    // which then leaves the source) and runs every row's copy of a tile back
    // to back.
    const bool big_last = passes >= 2 && nreg::root_mode(nb) == nreg::ROOT_BASE && !table_span(nb) &&
                          nb <= BIG_TABLE_BITS && rows >= BIG_TABLE_ROWS && !c->coarse_active;
    uint64_t last_scale = 1, big_scale = 1;
    if constexpr (std::is_same<Src, nreg::SrcU64>::value) {
        if (src.scale != 1 && passes >= 2 && nreg::root_mode(nb) == nreg::ROOT_BASE && !table_span(nb)) {
            (big_last ? big_scale : last_scale) = src.scale;
            src.scale = 1;
        }
    }
    const int wb = nreg::run_bits(nb, PL);
    GatherFn<Src> g = nullptr;
    ColFn col = nullptr;
    for (uint64_t r0 = 0; r0 < rows; r0 += 65535) {
        const unsigned cnt = static_cast<unsigned>(std::min<uint64_t>(rows - r0, 65535));
        const Src s0 = shift(src, r0);
        uint64_t* y = out + (r0 << nb) * PL;
        {  // gather: the last digit's DFT, rows in (i_1, .., i_(P-1)) order
            const int rb = r[passes - 1];
            const int qb = std::min(wb, r[0]);
            nreg::Digits d{};
            d.r1 = r[0];
            d.count = passes - 2;
            for (int j = 0; j < d.count; ++j) d.bits[j] = r[1 + j];
            const uint64_t blocks = uint64_t{1} << (nb - rb - qb);
            const size_t lds = gather_lds(rb, qb + PL - 1);
            // step 1's input ja sits at index >= ja n / A: ja >= ceil(extent A / n) reads only zeros
            const int la = (rb + 1) / 2;
            const uint64_t nza = (s0.extent(uint64_t{1} << nb) + (uint64_t{1} << (nb - la)) - 1) >> (nb - la);
            if (!kernels_for<PL, Src>(rb, nreg::root_mode(nb), nza, false, &g, &col) || blocks > 0x7FFFFFFFull ||
                lds > 160 * 1024)
                return fail_msg(c, "NTT pass exceeds its launch limits");
            if (allow_lds(c, g, lds)) return -1;
            hipLaunchKernelGGL(g, dim3(static_cast<unsigned>(blocks), cnt), dim3(nreg::THREADS), lds, c->stream, s0, y,
                               nb, qb, d, tb.inner);
            VMX_HIP(c, hipGetLastError());
        }
        int lbits = r[passes - 1];
        for (int p = passes - 2; p >= 0; --p) {  // columns: digits P-1 .. 1, in place
            const int rb = r[p], lb = lbits, hb = nb - rb - lb;
            const int cb = std::min(wb, lb);
            const uint64_t blocks = uint64_t{1} << (nb - rb - cb);
            const size_t lds = tile_lds(rb, cb + PL - 1);
            const uint64_t* ctab = nullptr;
            const bool big = p == 0 && big_last;
            if (table_span(rb + lb) && col_table_for(c, tb, hb, rb, lb, &ctab)) return -1;
            if (big && col_table_for(c, tb, hb, rb, lb, &ctab, big_scale)) return -1;
            if (big && ctab == nullptr) return fail_msg(c, "NTT pass without its column table");
            if (p == 0 && last_scale != 1 && ctab != nullptr)
                return fail_msg(c, "inverse NTT scale handed to a column pass that reads a table");
            if (!kernels_for<PL, Src>(rb, nreg::root_mode(nb), 0, ctab != nullptr, &g, &col) ||
                blocks > 0x7FFFFFFFull || lds > 160 * 1024)
                return fail_msg(c, "NTT pass exceeds its launch limits");
            if (allow_lds(c, col, lds)) return -1;
            const uint64_t pass_scale = p == 0 && ctab == nullptr ? last_scale : uint64_t{1};
            hipLaunchKernelGGL(col, dim3(static_cast<unsigned>(blocks), cnt), dim3(nreg::THREADS), lds, c->stream, y,
                               nb, hb, lb, cb, tb.inner, tb.split, tb.split_h, ctab, pass_scale, big ? 1 : 0);
            VMX_HIP(c, hipGetLastError());
            lbits += rb;
        }
    }
    return 0;
}

int reg_ntt(Context* c, const RegTables& tb, const uint64_t* in, uint64_t in_stride, uint64_t len, uint64_t* out,
            uint64_t rows, int nb, int planes, bool inverse) {
    if (inverse && nb > 31) return fail_msg(c, "inverse transforms are defined up to 2^31 points");
    // a zero-length input reads one in-bounds word of the inner table, masked to zero
    const nreg::SrcU64 src{len ? in : tb.inner, len ? in_stride : 0, len, inverse ? 1 : 0,
                           inverse ? gl::inv_host(gl::canon(uint64_t{1} << nb)) : uint64_t{1}};
    auto shift1 = [](nreg::SrcU64 s, uint64_t r0) {  // to the launch slice's first row
        s.x += r0 * s.x_stride;
        return s;
    };
    auto shift2 = [](nreg::SrcU64 s, uint64_t r0) {
        s.x += r0 * s.x_stride * 2;
        return s;
    };
    if (planes == 1) return run_passes<1>(c, tb, src, shift1, out, rows, nb);
    if (planes == 2) return run_passes<2>(c, tb, src, shift2, out, rows, nb);
    return fail_msg(c, "NTT elements are one or two u64");
}

int reg_ntt_msg_i16(Context* c, const RegTables& tb, const int16_t* w, const uint64_t* pads, uint64_t cols,
                    uint64_t pad, uint64_t* out, uint64_t rows, int nb) {
    const nreg::SrcMsgI16 src{cols ? w : reinterpret_cast<const int16_t*>(tb.inner), pad ? pads : tb.inner, cols,
                              pad};
    auto shift = [](nreg::SrcMsgI16 s, uint64_t r0) {
        s.w += r0 * s.cols;
        if (s.pad) s.pads += r0 * s.pad;
        return s;
    };
    return run_passes<1>(c, tb, src, shift, out, rows, nb);
}

}  // namespace vmx
