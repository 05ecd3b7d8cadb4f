// host_check.cpp -- host build of the device arithmetic headers, exported so
// CPU tests can check every compile-time shift form against big integers.
// Not part of the product library.
#include <stdint.h>

#include <array>
#include <utility>

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
