// chacha8.hpp -- device/host ChaCha8 keystream and the FpStream sampler.
//
// FpStream (rust/volta-field/src/lib.rs:224-258) is rand_chacha 0.3.1's
// ChaCha8Rng: Bernstein's ChaCha with 8 rounds, a 64-bit block counter in
// state words 12-13 and the 64-bit stream id in words 14-15, the 32-byte seed
// as the key in little-endian words.  next_u64 joins two consecutive block
// words, low word first; next_fp rejects draws >= p; next_fp2 is two accepted
// draws (c0 then c1).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace chacha8 {

constexpr uint64_t P = 0xFFFFFFFF00000001ull;

struct Key {
    uint32_t k[8];
};

inline Key key_from_seed(const uint8_t seed[32]) {
    Key key{};
    for (int i = 0; i < 8; ++i)
        key.k[i] = static_cast<uint32_t>(seed[4 * i]) | (static_cast<uint32_t>(seed[4 * i + 1]) << 8) |
                   (static_cast<uint32_t>(seed[4 * i + 2]) << 16) | (static_cast<uint32_t>(seed[4 * i + 3]) << 24);
    return key;
}

__host__ __device__ __forceinline__ uint32_t rotl(uint32_t x, int n) { return (x << n) | (x >> (32 - n)); }

__host__ __device__ __forceinline__ void qr(uint32_t& a, uint32_t& b, uint32_t& c, uint32_t& d) {
    a += b;
    d = rotl(d ^ a, 16);
    c += d;
    b = rotl(b ^ c, 12);
    a += b;
    d = rotl(d ^ a, 8);
    c += d;
    b = rotl(b ^ c, 7);
}

__host__ __device__ __forceinline__ void block(const Key& key, uint64_t stream, uint64_t counter, uint32_t out[16]) {
    const uint32_t init[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u,
                               key.k[0],    key.k[1],    key.k[2],    key.k[3],
                               key.k[4],    key.k[5],    key.k[6],    key.k[7],
                               static_cast<uint32_t>(counter), static_cast<uint32_t>(counter >> 32),
                               static_cast<uint32_t>(stream),  static_cast<uint32_t>(stream >> 32)};
    uint32_t x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = init[i];
#pragma unroll
    for (int r = 0; r < 4; ++r) {  // 4 double rounds = 8 rounds
        qr(x[0], x[4], x[8], x[12]);
        qr(x[1], x[5], x[9], x[13]);
        qr(x[2], x[6], x[10], x[14]);
        qr(x[3], x[7], x[11], x[15]);
        qr(x[0], x[5], x[10], x[15]);
        qr(x[1], x[6], x[11], x[12]);
        qr(x[2], x[7], x[8], x[13]);
        qr(x[3], x[4], x[9], x[14]);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) out[i] = x[i] + init[i];
}

class FpStream {
  public:
    __host__ __device__ FpStream(const Key& key, uint64_t stream) : key_(key), stream_(stream) {}

    __host__ __device__ uint64_t next_u64() {
        if (idx_ >= 8) {
            block(key_, stream_, ctr_, w_);
            ++ctr_;
            idx_ = 0;
        }
        const uint64_t v = static_cast<uint64_t>(w_[2 * idx_]) | (static_cast<uint64_t>(w_[2 * idx_ + 1]) << 32);
        ++idx_;
        return v;
    }

    __host__ __device__ uint64_t next_fp() {
        for (;;) {
            const uint64_t v = next_u64();
            if (v < P) return v;
        }
    }

  private:
    Key key_;
    uint64_t stream_;
    uint64_t ctr_ = 0;
    uint32_t idx_ = 8;
    uint32_t w_[16] = {};
};

}  // namespace chacha8
