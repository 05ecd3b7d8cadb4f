// host_check.cpp -- host build of the device arithmetic headers, exported so
// CPU tests can check every compile-time shift form against big integers.
// Not part of the product library.
#include <stdint.h>

#include <array>
#include <utility>

#include "enc13_mfma.hpp"
#include "gl64.hpp"
#include "gl64_shift.hpp"

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
