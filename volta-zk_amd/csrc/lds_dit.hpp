// lds_dit.hpp -- radix-2^2 DIT transforms of power-of-two length held in LDS,
// shared by the base-field NTT (ntt.hip) and the X4 Fp2 NTT (x4.hip).
#pragma once

#include <hip/hip_runtime.h>

#include "gl64.hpp"

namespace vmx {

__device__ __forceinline__ uint32_t brev(uint32_t x, int bits) { return __brev(x) >> (32 - bits); }

// `count` independent DIT transforms of size 2^fbits stored back to back in s,
// each already in bit-reversed order.  Twiddle for stage length L = 2^l,
// position k: tw[k << (gbits - l)] where 2^gbits is the size the table was
// built for (the sub-transform root is a power of the table root).
__device__ inline void lds_dit(uint64_t* s, int count, int fbits, int gbits, const uint64_t* tw) {
    const int T = blockDim.x;
    const int tid = threadIdx.x;
    const size_t m = size_t{1} << fbits;
    const size_t total = m * count;
    int l = 1;
    if (fbits & 1) {
        for (size_t b = tid; b < total / 2; b += T) {
            const size_t i0 = 2 * b;
            const uint64_t u = s[i0], v = s[i0 + 1];
            s[i0] = gl::add(u, v);
            s[i0 + 1] = gl::sub(u, v);
        }
        __syncthreads();
        l = 2;
    }
    for (; l < fbits; l += 2) {
        const size_t half = size_t{1} << (l - 1);
        const size_t len = size_t{1} << l;
        const int sh1 = gbits - l;
        const int sh2 = gbits - l - 1;
        const size_t quads_per = m >> 2;
        for (size_t qq = tid; qq < total / 4; qq += T) {
            const size_t c = qq / quads_per;
            const size_t q = qq - c * quads_per;
            const size_t group = q >> (l - 1);
            const size_t k = q & (half - 1);
            uint64_t* base = s + c * m + group * 2 * len + k;
            const uint64_t a0 = base[0], a1 = base[half], a2 = base[len], a3 = base[len + half];
            const uint64_t w1 = tw[k << sh1];
            uint64_t t = gl::mul(a1, w1);
            const uint64_t b0 = gl::add(a0, t), b1 = gl::sub(a0, t);
            t = gl::mul(a3, w1);
            const uint64_t b2 = gl::add(a2, t), b3 = gl::sub(a2, t);
            const uint64_t w2 = tw[k << sh2];
            const uint64_t w3 = tw[(k + half) << sh2];
            t = gl::mul(b2, w2);
            base[0] = gl::add(b0, t);
            base[len] = gl::sub(b0, t);
            t = gl::mul(b3, w3);
            base[half] = gl::add(b1, t);
            base[len + half] = gl::sub(b1, t);
        }
        __syncthreads();
    }
}

}  // namespace vmx
