// ntt15.hip -- one-pass forward NTT of 2^15 points over HBM, for rows whose
// inputs are zero from index 1024 NZ on (the rate-1/8 and rate-1/4 Ligero
// encodes of 2^15-point codewords, and denser rows up to all 2^15 inputs).  The split and the exchanges are in
// ntt15.hpp.
//
// One workgroup of 1024 threads per CU walks the rows (persistent grid); a
// row's 2^15 values stay in registers, 32 per thread, between its input
// loads and its stores, so HBM sees the inputs once and the codewords once
// (the pass engine reads and writes the whole row once more).  The next
// row's inputs are loaded during the current row.  Each store instruction
// writes two runs of 32 consecutive u64 (256 bytes each).
#include <hip/hip_runtime.h>

#include <algorithm>

#include "context.hpp"
#include "kernels.hpp"
#include "ntt15.hpp"

namespace vmx {
namespace n15 {

typedef uint32_t v2u __attribute__((ext_vector_type(2)));

template <int NZ, class Src>
__global__ __launch_bounds__(THREADS) void ntt15_rows(Src src, size_t rows, const uint64_t* __restrict__ tab,
                                                      uint64_t* __restrict__ out) {
#if defined(__HIP_DEVICE_COMPILE__)
    extern __shared__ uint64_t lds[];
    const int t = static_cast<int>(threadIdx.x);
    const Role r = role(t);
    // the wave index as a scalar, so that the half choices below are branches
    // of the whole wave
    const int w = __builtin_amdgcn_readfirstlane(t >> 6);
    const int w0 = w & 1, w1 = (w >> 1) & 1;
    lds[T2_OFF + t] = tab[T1_WORDS + t];
    const Table1 t1(tab);
    // Up to 4 nonzero inputs per thread the next row's load a row ahead, into
    // registers; denser rows load at the top of their own row.  Measured: C4
    // (4 u64) 5.07 -> 5.03 ms with the prefetch, p15 (8 i16 + 1 pad) 3.92 ->
    // 4.27 ms, whose 11 prefetch registers spill beside the 32 values.
    constexpr bool PREFETCH = NZ <= 4;
    typename Src::Raw raw[NZ];
    size_t row = blockIdx.x;
    if (PREFETCH && row < rows) fetch_row<NZ>(src, row, r.m, raw);
    __syncthreads();
    // Wave priority by phase, as in the one-pass 2^13 kernel: between a row's
    // last barrier and the next row's first one the waves run apart, and the
    // ones storing go first (2), then the ones loading and in stage A (1),
    // before any wave in the exchanges (0).  C4 4.85-4.93 -> 4.70-4.76 ms,
    // p15 3.80-3.86 -> 3.72-3.78 ms, alternating on one box.
    __builtin_amdgcn_s_setprio(1);
    for (; row < rows; row += gridDim.x) {
        // The role indices are recomputed from an opaque copy of the thread
        // index where each phase needs them (a few adds), so neither they nor
        // the LDS addresses formed from them are hoisted out of the loop and
        // kept live across it (which spills).
        auto here = [&]() {
            // the lane from mbcnt and the wave from its scalar: no register
            // holds the thread index across the loop
            const int lane = static_cast<int>(__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)));
            int tt = (w << 6) + lane;
            asm volatile("" : "+v"(tt));
            return role(tt);
        };
        uint64_t v[32], tw[8];
        // Per row: the first half's twiddles load after stage A, the second
        // half's while the first half goes through LDS, the next row's inputs
        // during stage C.  The scheduling barriers keep each group of loads
        // where it is (hoisted, they would be live beside all 32 values).
        if constexpr (!PREFETCH) fetch_row<NZ>(src, row, here().m, raw);
        stage_a<NZ>(v, src, raw);
        __builtin_amdgcn_sched_barrier(0);
        {
            const Role q = here();
            load_tw1<0>(tw, t1, w0, q.m);
            if (w0 == 0) x1_write<0>(lds, v, tw, t1, q.m);
            else x1_write<1>(lds, v, tw, t1, q.m);
        }
        __builtin_amdgcn_s_setprio(0);  // the exchanges and stage B
        __builtin_amdgcn_sched_barrier(0);
        load_tw1<0>(tw, t1, w0 ^ 1, here().m);
        __syncthreads();
        {
            const Role q = here();
            if (w0 == 0) x1_read<0>(lds, v, q.j1b, q.k3b);
            else x1_read<1>(lds, v, q.j1b, q.k3b);
        }
        __syncthreads();
        {
            const Role q = here();
            if (w0 == 1) x1_write<0>(lds, v, tw, t1, q.m);
            else x1_write<1>(lds, v, tw, t1, q.m);
        }
        __syncthreads();
        {
            const Role q = here();
            if (w0 == 1) x1_read<0>(lds, v, q.j1b, q.k3b);
            else x1_read<1>(lds, v, q.j1b, q.k3b);
        }
        __syncthreads();
        gl::dit_pow2<5, gl::E_W32>(v);
        gl::static_for<0, 2>([&](auto rr) {
            constexpr int rd = decltype(rr)::value;
            {
                const Role q = here();
                if ((w1 ^ rd) == 0) x2_write<0>(lds, v, q.j1b, q.k3b);
                else x2_write<1>(lds, v, q.j1b, q.k3b);
            }
            __syncthreads();
            {
                const Role q = here();
                if ((w1 ^ rd) == 0) x2_read<0>(lds, v, q.k3c, q.k2c);
                else x2_read<1>(lds, v, q.k3c, q.k2c);
            }
            __syncthreads();
        });
        if (PREFETCH && row + gridDim.x < rows) fetch_row<NZ>(src, row + gridDim.x, here().m, raw);
        __builtin_amdgcn_s_setprio(2);  // stage C and the stores
        __builtin_amdgcn_sched_barrier(0);
        gl::dit_pow2<5, gl::E_W32>(v);
        // X[k3 + 32 k2 + 1024 k1]: scalar offset k1 8 KiB, non-temporal (aux bit 1)
        const auto orow = rsrc(out + row * N, size_t{N} * 8);
        const Role q = here();
        const uint32_t qo = static_cast<uint32_t>(q.k3c + 32 * q.k2c) * 8u;
        gl::static_for<0, 32>([&](auto k_) {
            constexpr int k1 = decltype(k_)::value;
            const v2u d = {static_cast<uint32_t>(v[k1]), static_cast<uint32_t>(v[k1] >> 32)};
            __builtin_amdgcn_raw_buffer_store_b64(d, orow, qo, k1 * 8192u, 2);
        });
        __builtin_amdgcn_s_setprio(1);  // the next row's loads, stage A and first exchange write
    }
#endif
}

// T1[k3 * 1024 + m] = w^(k3 m) and T2[k2 * 32 + j1] = w^(32 j1 k2).
__global__ void build_tables(const uint64_t* __restrict__ fwd, uint64_t* __restrict__ tab) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx < T1_WORDS + 1024) tab[idx] = table_word(fwd, idx);
}

int build(Context* c, TwiddleSet* t) {
    hipLaunchKernelGGL(build_tables, dim3((T1_WORDS + 1024 + 255) / 256), dim3(256), 0, c->stream,
                       static_cast<const uint64_t*>(t->fwd), t->grid);
    VMX_HIP(c, hipGetLastError());
    return 0;
}

template <int NZ, class Src>
int launch(Context* c, const Src& src, size_t rows, uint64_t* out, TwiddleSet* t) {
    if (ensure_grid_twiddles(c, t, TABLE_BYTES, build)) return -1;
    auto k = ntt15_rows<NZ, Src>;
    VMX_HIP(c, hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
                                   static_cast<int>(LDS_BYTES)));
    const size_t cus = c->cu_count > 0 ? static_cast<size_t>(c->cu_count) : 256;
    const unsigned blocks = static_cast<unsigned>(std::min(rows, cus));
    hipLaunchKernelGGL(k, dim3(blocks), dim3(THREADS), LDS_BYTES, c->stream, src, rows,
                       static_cast<const uint64_t*>(t->grid), out);
    VMX_HIP(c, hipGetLastError());
    return 0;
}

}  // namespace n15

int ntt15_u64_rows(Context* c, const uint64_t* in, size_t stride, size_t len, size_t rows, size_t n, uint64_t* out,
                   TwiddleSet* t) {
    if (n != static_cast<size_t>(n15::N) || len == 0 || len > n || stride < len || !t->fwd) return 1;
    if (!t->grid && c->coarse_active) return 1;  // tables may not grow inside a coarse scope
    if (rows == 0) return 0;
    const n15::SrcU64 s{in, stride, len};
    if (len <= 2048) return n15::launch<2>(c, s, rows, out, t);
    if (len <= 4096) return n15::launch<4>(c, s, rows, out, t);
    if (len <= 8192) return n15::launch<8>(c, s, rows, out, t);
    if (len <= 16384) return n15::launch<16>(c, s, rows, out, t);
    return n15::launch<32>(c, s, rows, out, t);
}

int ntt15_msg_rows(Context* c, const int16_t* w, const uint64_t* pads, size_t cols, size_t pad, size_t rows,
                   size_t n, uint64_t* out, TwiddleSet* t) {
    if (n != static_cast<size_t>(n15::N) || !t->fwd || cols == 0) return 1;
    if (!t->grid && c->coarse_active) return 1;
    if (rows == 0) return 0;
    const uint64_t* pp = pad ? pads : t->fwd;  // a readable word when there are no pads
    if (cols == 8192 && pad <= 1024) {
        const n15::SrcMsg<8> s{w, pp, cols, pad};
        if (pad == 0) return n15::launch<8>(c, s, rows, out, t);
        return n15::launch<9>(c, s, rows, out, t);
    }
    if (cols == 4096 && pad <= 1024) {
        const n15::SrcMsg<4> s{w, pp, cols, pad};
        if (pad == 0) return n15::launch<4>(c, s, rows, out, t);
        return n15::launch<5>(c, s, rows, out, t);
    }
    return 1;
}

}  // namespace vmx
