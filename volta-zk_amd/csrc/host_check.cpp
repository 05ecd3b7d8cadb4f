// host_check.cpp -- host build of the device arithmetic headers, exported so
// CPU tests can check every compile-time shift form against big integers.
// Not part of the product library.
#include <stdint.h>

#include <algorithm>
#include <array>
#include <utility>
#include <vector>

#include "enc13_mfma.hpp"
#include "enc13_phase_b.hpp"
#include "gl64.hpp"
#include "gl64_shift.hpp"
#include "ntt_rr.hpp"
#include "ntt15.hpp"

namespace {
using Fn = uint64_t (*)(uint64_t);
using FnI = uint64_t (*)(int32_t);

template <int... E>
constexpr auto pow2_table(std::integer_sequence<int, E...>) {
    return std::array<Fn, sizeof...(E)>{+[](uint64_t x) { return gl::mul_pow2<E>(x); }...};
}
template <int... K>
constexpr auto w128_table(std::integer_sequence<int, K...>) {
    return std::array<FnI, sizeof...(K)>{+[](int32_t x) { return gl::i16_mul_w128<K>(x); }...};
}
template <int... E>
constexpr auto i16_table(std::integer_sequence<int, E...>) {
    return std::array<FnI, sizeof...(E)>{+[](int32_t x) { return gl::i16_mul_pow2<E>(x); }...};
}
const auto kPow2 = pow2_table(std::make_integer_sequence<int, 192>{});
const auto kW128 = w128_table(std::make_integer_sequence<int, 128>{});
const auto kI16 = i16_table(std::make_integer_sequence<int, 192>{});

// butterfly with twiddle 2^E: returns u + w v in *a and u - w v in *b
template <int... E>
constexpr auto bfly_table(std::integer_sequence<int, E...>) {
    using B = void (*)(uint64_t*, uint64_t*);
    return std::array<B, sizeof...(E)>{+[](uint64_t* u, uint64_t* v) { gl::bfly_pow2<E>(*u, *v); }...};
}
const auto kBfly = bfly_table(std::make_integer_sequence<int, 192>{});
}  // namespace

extern "C" __attribute__((visibility("default"))) uint64_t glc_mul_pow2(uint64_t x, int e) { return kPow2[e](x); }
extern "C" __attribute__((visibility("default"))) uint64_t glc_i16_mul_w128(int32_t x, int k) { return kW128[k](x); }
extern "C" __attribute__((visibility("default"))) uint64_t glc_i16_mul_pow2(int32_t x, int e) { return kI16[e](x); }
extern "C" __attribute__((visibility("default"))) void glc_bfly(uint64_t* u, uint64_t* v, int e) { kBfly[e](u, v); }
extern "C" __attribute__((visibility("default"))) uint64_t glc_mul32x4(uint64_t a, uint64_t b) { return gl::mul32x4(a, b); }
extern "C" __attribute__((visibility("default"))) uint64_t glc_add(uint64_t a, uint64_t b) { return gl::add(a, b); }
extern "C" __attribute__((visibility("default"))) uint64_t glc_sub(uint64_t a, uint64_t b) { return gl::sub(a, b); }

// Phase A of the n = 2^13 i16 encode as encode_fast.hip runs it on the matrix
// cores (enc13_mfma.hpp), emulated lane by lane with the instruction's operand
// layout: Y[j1 * 64 + i2] = (sum_{i1 < 32} x[64 i1 + i2] w^(64 i1 j1)) w^(i2 j1).
extern "C" __attribute__((visibility("default"))) int glc_balanced_digit(uint64_t c, int pos) {
    return enc13m::balanced_digit(c, pos);
}
extern "C" __attribute__((visibility("default"))) int glc_bias_digit(int pos) { return enc13m::bias_digit(pos); }
extern "C" __attribute__((visibility("default"))) uint64_t glc_recombine(const int* a8) {
    return enc13m::recombine(a8, a8 + 4);
}
extern "C" __attribute__((visibility("default"))) void glc_enc13_phase_a(const uint64_t* tw_half, const int16_t* x,
                                                                         size_t cols, uint64_t* Y) {
    static int8_t frags[enc13m::FRAG_BYTES];
    static int init[enc13m::INIT_WORDS];
    for (int idx = 0; idx < static_cast<int>(enc13m::FRAG_BYTES / 16); ++idx)
        enc13m::a_fragment(tw_half, idx, frags + 16 * idx);
    for (int i = 0; i < static_cast<int>(enc13m::INIT_WORDS); ++i) init[i] = enc13m::init_word(tw_half, i >> 3, i & 7);
    // B fragments: lane l of column tile t holds the digit pairs x ^ 0x80 of
    // x[64 i1 + 16 t + (l & 15)], i1 = 8 (l >> 4) .. + 7 (zero past cols).
    int8_t bfrag[4][64][16];
    for (int t = 0; t < 4; ++t)
        for (int l = 0; l < 64; ++l)
            for (int k = 0; k < 8; ++k) {
                const size_t e = size_t{64} * (8 * (l >> 4) + k) + 16 * t + (l & 15);
                const uint16_t pat = static_cast<uint16_t>(e < cols ? x[e] : 0) ^ 0x80u;
                bfrag[t][l][2 * k] = static_cast<int8_t>(pat & 255);
                bfrag[t][l][2 * k + 1] = static_cast<int8_t>(pat >> 8);
            }
    for (int q = 0; q < 32; ++q)
        for (int t = 0; t < 4; ++t)
            for (int l = 0; l < 64; ++l) {
                int acc[8];
                for (int h = 0; h < 2; ++h)
                    for (int r = 0; r < 4; ++r) {
                        // D register r of lane l: C[4 (l >> 4) + r][l & 15], accumulated
                        // over K = 64 from the lanes that hold that A row and B column.
                        const int row = 4 * (l >> 4) + r, col = l & 15;
                        const int j1 = 4 * q + (row >> 2), pos = 4 * h + (row & 3);
                        long s = init[j1 * 8 + pos];
                        for (int k = 0; k < 64; ++k) {
                            const int8_t av = frags[((q * 2 + h) * 64 + 16 * (k >> 4) + row) * 16 + (k & 15)];
                            const int8_t bv = bfrag[t][16 * (k >> 4) + col][k & 15];
                            s += static_cast<long>(av) * bv;
                        }
                        acc[4 * h + r] = static_cast<int>(s);
                    }
                const int j1 = 4 * q + (l >> 4), i2 = 16 * t + (l & 15);
                const int e = (i2 * j1) & 8191;
                const uint64_t g = e < 4096 ? tw_half[e] : gl::neg(tw_half[e - 4096]);
                Y[j1 * 64 + i2] = gl::mul32x4(enc13m::recombine(acc, acc + 4), g);
            }
}

// Phase B of one row as the encode kernel runs it: y holds the row's 64 values
// Y[i2] (canonical), out receives X[2k + H] for k < 32.  The sums and
// differences are phase A's stores.
extern "C" __attribute__((visibility("default"))) void glc_enc13_phase_b(const uint64_t* y, int H, uint64_t* out) {
    uint64_t sd[32], v[32];
    for (int q = 0; q < 32; ++q) sd[q] = H == 0 ? gl::add(y[q], y[q + 32]) : gl::sub(y[q], y[q + 32]);
    if (H == 0) enc13m::phase_b_load<0>(sd, v);
    else enc13m::phase_b_load<1>(sd, v);
    enc13m::phase_b_dft(v);
    for (int k = 0; k < 32; ++k) out[k] = v[k];
}

// ---- the one-pass 2^15 transform (ntt15.hip), emulated on the host ----------
// Each workgroup's 1024 threads run the kernel's phases one after the other,
// thread by thread, between the kernel's barriers; the exchange buffer is
// poisoned before every write round, so a read of a word the round did not
// write shows up in the result, and guard words around the LDS image and its
// T2 table are checked after every row.  Returns 0, or -1 when a guard or
// T2 changed.
namespace {
template <int NZ, class Src>
int n15_emulate(const uint64_t* fwd, const Src& src, size_t rows, size_t blocks, uint64_t* out) {
    using namespace vmx::n15;
    constexpr int GUARD = 64;
    constexpr uint64_t POISON = 0xA5A5A5A55A5A5A5Aull;
    std::vector<uint64_t> tab(T1_WORDS + 1024);
    for (int i = 0; i < T1_WORDS + 1024; ++i) tab[i] = table_word(fwd, i);
    const Table1 t1(tab.data());
    std::vector<uint64_t> image(LDS_WORDS + 2 * GUARD, POISON);
    uint64_t* lds = image.data() + GUARD;
    std::vector<std::array<uint64_t, 32>> v(THREADS);
    std::vector<std::array<typename Src::Raw, NZ>> raw(THREADS);
    auto intact = [&]() {
        for (int i = 0; i < GUARD; ++i)
            if (image[i] != POISON || image[GUARD + LDS_WORDS + i] != POISON) return false;
        for (int t = 0; t < THREADS; ++t)
            if (lds[T2_OFF + t] != tab[T1_WORDS + t]) return false;
        return true;
    };
    auto poison = [&]() { std::fill(lds, lds + XBUF_WORDS, POISON); };
    for (size_t b = 0; b < blocks; ++b) {
        for (int t = 0; t < THREADS; ++t) lds[T2_OFF + t] = tab[T1_WORDS + t];
        size_t row = b;
        if (row < rows)
            for (int t = 0; t < THREADS; ++t) fetch_row<NZ>(src, row, role(t).m, raw[t].data());
        for (; row < rows; row += blocks) {
            for (int t = 0; t < THREADS; ++t) stage_a<NZ>(v[t].data(), src, raw[t].data());
            for (int rd = 0; rd < 2; ++rd) {
                poison();
                for (int t = 0; t < THREADS; ++t) {
                    const Role r = role(t);
                    const int h = ((t >> 6) & 1) ^ rd;
                    uint64_t tw[8];
                    load_tw1<0>(tw, t1, h, r.m);
                    if (h == 0) x1_write<0>(lds, v[t].data(), tw, t1, r.m);
                    else x1_write<1>(lds, v[t].data(), tw, t1, r.m);
                }
                for (int t = 0; t < THREADS; ++t) {
                    const Role r = role(t);
                    if ((((t >> 6) & 1) ^ rd) == 0) x1_read<0>(lds, v[t].data(), r.j1b, r.k3b);
                    else x1_read<1>(lds, v[t].data(), r.j1b, r.k3b);
                }
            }
            for (int t = 0; t < THREADS; ++t) gl::dit_pow2<5, gl::E_W32>(v[t].data());
            for (int rd = 0; rd < 2; ++rd) {
                poison();
                for (int t = 0; t < THREADS; ++t) {
                    const Role r = role(t);
                    if ((((t >> 7) & 1) ^ rd) == 0) x2_write<0>(lds, v[t].data(), r.j1b, r.k3b);
                    else x2_write<1>(lds, v[t].data(), r.j1b, r.k3b);
                }
                for (int t = 0; t < THREADS; ++t) {
                    const Role r = role(t);
                    if ((((t >> 7) & 1) ^ rd) == 0) x2_read<0>(lds, v[t].data(), r.k3c, r.k2c);
                    else x2_read<1>(lds, v[t].data(), r.k3c, r.k2c);
                }
            }
            for (int t = 0; t < THREADS; ++t) {
                if (row + blocks < rows) fetch_row<NZ>(src, row + blocks, role(t).m, raw[t].data());
                gl::dit_pow2<5, gl::E_W32>(v[t].data());
                const Role r = role(t);
                for (int k1 = 0; k1 < 32; ++k1) out[row * N + r.k3c + 32 * r.k2c + 1024 * k1] = v[t][k1];
            }
            if (!intact()) return -1;
        }
    }
    return 0;
}
}  // namespace

// The kernel's choice of NZ for u64 rows (ntt15_u64_rows), then the emulation.
extern "C" __attribute__((visibility("default"))) int glc_ntt15_u64(const uint64_t* fwd, const uint64_t* in,
                                                                    size_t stride, size_t len, size_t rows,
                                                                    size_t blocks, uint64_t* out) {
    const vmx::n15::SrcU64 s{in, stride, len};
    if (len == 0 || stride < len) return 1;
    if (len <= 2048) return n15_emulate<2>(fwd, s, rows, blocks, out);
    if (len <= 4096) return n15_emulate<4>(fwd, s, rows, blocks, out);
    if (len <= 8192) return n15_emulate<8>(fwd, s, rows, blocks, out);
    if (len <= 16384) return n15_emulate<16>(fwd, s, rows, blocks, out);
    if (len <= 32768) return n15_emulate<32>(fwd, s, rows, blocks, out);
    return 1;
}

// The same for message rows lift(w) || pads || 0 (ntt15_msg_rows).
extern "C" __attribute__((visibility("default"))) int glc_ntt15_msg(const uint64_t* fwd, const int16_t* w,
                                                                    const uint64_t* pads, size_t cols, size_t pad,
                                                                    size_t rows, size_t blocks, uint64_t* out) {
    const uint64_t* pp = pad ? pads : fwd;
    if (cols == 8192 && pad <= 1024) {
        const vmx::n15::SrcMsg<8> s{w, pp, cols, pad};
        return pad == 0 ? n15_emulate<8>(fwd, s, rows, blocks, out) : n15_emulate<9>(fwd, s, rows, blocks, out);
    }
    if (cols == 4096 && pad <= 1024) {
        const vmx::n15::SrcMsg<4> s{w, pp, cols, pad};
        return pad == 0 ? n15_emulate<4>(fwd, s, rows, blocks, out) : n15_emulate<5>(fwd, s, rows, blocks, out);
    }
    return 1;
}

// ---- the one-pass 2^13 / 2^14 transforms (ntt_rr.hip), emulated ---------------------
// As for the 2^15 transform: the workgroup's threads run the phases one after
// the other between the kernel's barriers, on a poisoned exchange buffer with
// guard words.  Rows read in full (NZ = 32) take stage A's first two stages
// per wave of 64 threads as the kernel does: copies when the wave's inputs are
// all zero from 8 M on, in full otherwise; the waves of each kind are counted.
namespace {
long g_rr_waves_full = 0, g_rr_waves_copy = 0;
template <int B, int NZ>
int rr_emulate(const uint64_t* fwd, const uint64_t* in, size_t stride, size_t len, size_t rows, size_t blocks,
               uint64_t* out) {
    using namespace vmx::rr;
    using S = Shape<B>;
    constexpr int GUARD = 64;
    constexpr uint64_t POISON = 0xA5A5A5A55A5A5A5Aull;
    std::vector<uint64_t> tab(S::TABLE_WORDS);
    for (int i = 0; i < S::TABLE_WORDS; ++i) tab[i] = table_word<B>(fwd, i);
    const Table1<B> t1(tab.data());
    std::vector<uint64_t> image(S::LDS_WORDS + 2 * GUARD, POISON);
    uint64_t* lds = image.data() + GUARD;
    std::vector<std::array<uint64_t, 32>> v(S::THREADS);
    auto intact = [&]() {
        for (int i = 0; i < GUARD; ++i)
            if (image[i] != POISON || image[GUARD + S::LDS_WORDS + i] != POISON) return false;
        for (int t = 0; t < S::T2_WORDS; ++t)
            if (lds[S::T2_OFF + t] != tab[S::T1_WORDS + t]) return false;
        return true;
    };
    auto poison = [&]() { std::fill(lds, lds + S::XBUF_WORDS, POISON); };
    for (size_t b = 0; b < blocks; ++b) {
        for (int t = 0; t < S::T2_WORDS; ++t) lds[S::T2_OFF + t] = tab[S::T1_WORDS + t];
        for (size_t row = b; row < rows; row += blocks) {
            for (int t = 0; t < S::THREADS; ++t) load_row<B, NZ>(v[t].data(), in, stride, len, row, role<B>(t).m);
            if constexpr (NZ == 32) {
                for (int w0 = 0; w0 < S::THREADS; w0 += 64) {
                    bool tail = false;
                    for (int t = w0; t < w0 + 64; ++t)
                        for (int j3 = 8; j3 < 32; ++j3) tail = tail || v[t][gl::bitrev_c(j3, 5)] != 0;
                    ++(tail ? g_rr_waves_full : g_rr_waves_copy);
                    for (int t = w0; t < w0 + 64; ++t) {
                        if (tail) gl::dit_pow2_sparse<5, gl::E_W32, prefix_mask(32), 2, 8>(v[t].data());
                        else gl::dit_pow2_sparse<5, gl::E_W32, prefix_mask(8), 2, 8>(v[t].data());
                        gl::dit_pow2<5, gl::E_W32, 8>(v[t].data());
                    }
                }
            } else {
                for (int t = 0; t < S::THREADS; ++t) gl::dit_pow2_sparse<5, gl::E_W32, prefix_mask(NZ)>(v[t].data());
            }
            for (int rd = 0; rd < 2; ++rd) {
                poison();
                for (int t = 0; t < S::THREADS; ++t) {
                    const Role r = role<B>(t);
                    const int h = ((t >> 6) & 1) ^ rd;
                    uint64_t tw[8];
                    load_tw1<B, 0>(tw, t1, h, r.m);
                    if (h == 0) x1_write<B, 0>(lds, v[t].data(), tw, t1, r.m);
                    else x1_write<B, 1>(lds, v[t].data(), tw, t1, r.m);
                }
                for (int t = 0; t < S::THREADS; ++t) {
                    const Role r = role<B>(t);
                    if ((((t >> 6) & 1) ^ rd) == 0) x1_read<B, 0>(lds, v[t].data(), r.j1b, r.k3b);
                    else x1_read<B, 1>(lds, v[t].data(), r.j1b, r.k3b);
                }
            }
            for (int t = 0; t < S::THREADS; ++t) gl::dit_pow2<5, gl::E_W32>(v[t].data());
            for (int rd = 0; rd < 2; ++rd) {
                poison();
                for (int t = 0; t < S::THREADS; ++t) {
                    const Role r = role<B>(t);
                    if ((((t >> 7) & 1) ^ rd) == 0) x2_write<B, 0>(lds, v[t].data(), r.j1b, r.k3b);
                    else x2_write<B, 1>(lds, v[t].data(), r.j1b, r.k3b);
                }
                for (int t = 0; t < S::THREADS; ++t) {
                    const Role r = role<B>(t);
                    if ((((t >> 7) & 1) ^ rd) == 0) x2_read<B, 0>(lds, v[t].data(), r.k3c, r.xc);
                    else x2_read<B, 1>(lds, v[t].data(), r.k3c, r.xc);
                }
            }
            for (int t = 0; t < S::THREADS; ++t) {
                stage_c<B>(v[t].data());
                const Role r = role<B>(t);
                for (int s = 0; s < 32; ++s)
                    out[row * S::N + r.k3c + 32 * ((s % S::P) + S::P * r.xc) + 1024 * (s / S::P)] = v[t][s];
            }
            if (!intact()) return -1;
        }
    }
    return 0;
}

template <int B>
int rr_dispatch(const uint64_t* fwd, const uint64_t* in, size_t stride, size_t len, size_t rows, size_t blocks,
                uint64_t* out) {
    using S = vmx::rr::Shape<B>;
    if (len == 0 || len > size_t{S::N} || stride < len) return 1;
    if (len <= size_t{8} * S::M) return rr_emulate<B, 8>(fwd, in, stride, len, rows, blocks, out);
    if (len <= size_t{16} * S::M) return rr_emulate<B, 16>(fwd, in, stride, len, rows, blocks, out);
    return rr_emulate<B, 32>(fwd, in, stride, len, rows, blocks, out);
}
}  // namespace

// Waves of rows read in full that ran stage A's first two stages in full /
// as copies, since the last reset.
extern "C" __attribute__((visibility("default"))) void glc_rr_wave_counts(long* full, long* copy, int reset) {
    *full = g_rr_waves_full;
    *copy = g_rr_waves_copy;
    if (reset) g_rr_waves_full = g_rr_waves_copy = 0;
}

// The kernels' choice of NZ (ntt_rr.hip), then the emulation: n = 2^13 or 2^14.
extern "C" __attribute__((visibility("default"))) int glc_ntt13r_u64(const uint64_t* fwd, const uint64_t* in,
                                                                     size_t stride, size_t len, size_t rows,
                                                                     size_t blocks, uint64_t* out) {
    return rr_dispatch<3>(fwd, in, stride, len, rows, blocks, out);
}
extern "C" __attribute__((visibility("default"))) int glc_ntt14r_u64(const uint64_t* fwd, const uint64_t* in,
                                                                     size_t stride, size_t len, size_t rows,
                                                                     size_t blocks, uint64_t* out) {
    return rr_dispatch<4>(fwd, in, stride, len, rows, blocks, out);
}
