// ntt_rr.hip -- one-pass forward NTT of u64 rows of 2^13 and 2^14 points held
// in registers (the split, the roles and the exchanges are in ntt_rr.hpp).
//
// Persistent workgroups of 32 N1 threads (four per CU for 2^13, one for
// 2^14; Shape::PER_CU), one row each at a time, without prefetch: the other
// workgroups on the CU run while one waits on its row's loads.  Each store
// instruction writes two runs of 32 consecutive u64.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "context.hpp"
#include "kernels.hpp"
#include "ntt_rr.hpp"

namespace vmx {
namespace rr {

typedef uint32_t v2u __attribute__((ext_vector_type(2)));

template <int B, int NZ>
__global__ __launch_bounds__(Shape<B>::THREADS, Shape<B>::WAVES_PER_SIMD) void rows_kernel(
    const uint64_t* __restrict__ in, size_t stride, size_t len, size_t rows, const uint64_t* __restrict__ tab,
    uint64_t* __restrict__ out) {
#if defined(__HIP_DEVICE_COMPILE__)
    using S = Shape<B>;
    extern __shared__ uint64_t lds[];
    const int t = static_cast<int>(threadIdx.x);
    const int w = __builtin_amdgcn_readfirstlane(t >> 6);
    const int w0 = w & 1, w1 = (w >> 1) & 1;
    lds[S::T2_OFF + t] = tab[S::T1_WORDS + t];
    const Table1<B> t1(tab);
    __syncthreads();
    // role indices recomputed per phase from mbcnt (nothing kept live across the loop)
    auto here = [&]() {
        const int lane = static_cast<int>(__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)));
        int tt = (w << 6) + lane;
        asm volatile("" : "+v"(tt));
        return role<B>(tt);
    };
    // Wave priority by phase.  The four workgroups of a CU run the same phases
    // out of step; a wave in stage C and its stores goes first (2), then one
    // loading its next row, running stage A and writing its first exchange
    // (1), and the waves between barriers in the exchanges and stage B fill
    // what is left (0).  The loads of the next row so leave early and overlap
    // the other workgroups' exchanges.  C3-shape rows in full, mostly zero
    // (the written commit chain): 2.50-2.57 -> 2.15 ms; rows read to 2^11:
    // 2.29-2.36 -> 2.08 ms.  One priority for the loads and stage A only gave
    // 2.46-2.49 ms; the same through the whole first exchange 2.22-2.24 ms.
    __builtin_amdgcn_s_setprio(1);
    for (size_t row = blockIdx.x; row < rows; row += gridDim.x) {
        uint64_t v[32], tw[8];
        load_row<B, NZ>(v, in, stride, len, row, here().m);
        if constexpr (NZ == 32) {
            // Rows the length does not bound (a buffer the caller may have
            // written through a device pointer) are often still zero from
            // 8 M on (message rows).  A wave whose inputs are all zero there
            // takes the first two stages as the copies dit_pow2_sparse makes
            // for NZ = 8; any nonzero value in the wave runs them in full.
            // Both give the same values on such rows.
            uint64_t tail = 0;
            gl::static_for<8, 32>([&](auto j_) { tail |= v[gl::bitrev_c(decltype(j_)::value, 5)]; });
            if (__builtin_amdgcn_ballot_w64(tail != 0) != 0)
                gl::dit_pow2_sparse<5, gl::E_W32, prefix_mask(32), 2, 8>(v);
            else
                gl::dit_pow2_sparse<5, gl::E_W32, prefix_mask(8), 2, 8>(v);
            gl::dit_pow2<5, gl::E_W32, 8>(v);
        } else {
            gl::dit_pow2_sparse<5, gl::E_W32, prefix_mask(NZ)>(v);
        }
        __builtin_amdgcn_sched_barrier(0);
        {
            const Role q = here();
            load_tw1<B, 0>(tw, t1, w0, q.m);
            if (w0 == 0) x1_write<B, 0>(lds, v, tw, t1, q.m);
            else x1_write<B, 1>(lds, v, tw, t1, q.m);
        }
        __builtin_amdgcn_s_setprio(0);  // the exchanges and stage B yield to the other workgroups
        __builtin_amdgcn_sched_barrier(0);
        load_tw1<B, 0>(tw, t1, w0 ^ 1, here().m);
        __syncthreads();
        {
            const Role q = here();
            if (w0 == 0) x1_read<B, 0>(lds, v, q.j1b, q.k3b);
            else x1_read<B, 1>(lds, v, q.j1b, q.k3b);
        }
        __syncthreads();
        {
            const Role q = here();
            if (w0 == 1) x1_write<B, 0>(lds, v, tw, t1, q.m);
            else x1_write<B, 1>(lds, v, tw, t1, q.m);
        }
        __syncthreads();
        {
            const Role q = here();
            if (w0 == 1) x1_read<B, 0>(lds, v, q.j1b, q.k3b);
            else x1_read<B, 1>(lds, v, q.j1b, q.k3b);
        }
        __syncthreads();
        gl::dit_pow2<5, gl::E_W32>(v);
        gl::static_for<0, 2>([&](auto rr_) {
            constexpr int rd = decltype(rr_)::value;
            {
                const Role q = here();
                if ((w1 ^ rd) == 0) x2_write<B, 0>(lds, v, q.j1b, q.k3b);
                else x2_write<B, 1>(lds, v, q.j1b, q.k3b);
            }
            __syncthreads();
            {
                const Role q = here();
                if ((w1 ^ rd) == 0) x2_read<B, 0>(lds, v, q.k3c, q.xc);
                else x2_read<B, 1>(lds, v, q.k3c, q.xc);
            }
            __syncthreads();
        });
        __builtin_amdgcn_s_setprio(2);
        stage_c<B>(v);
        // X[k3 + 32 (p + P x) + 1024 k1] from slot p + P k1: lane offset
        // (k3 + 32 P x) 8, scalar offset (32 p + 1024 k1) 8, non-temporal (aux bit 1)
        const auto orow = rsrc(out + row * S::N, size_t{S::N} * 8);
        const Role q = here();
        const uint32_t qo = static_cast<uint32_t>(q.k3c + 32 * S::P * q.xc) * 8u;
        gl::static_for<0, 32>([&](auto s_) {
            constexpr int s = decltype(s_)::value, pp = s % S::P, k1 = s / S::P;
            const v2u d = {static_cast<uint32_t>(v[s]), static_cast<uint32_t>(v[s] >> 32)};
            __builtin_amdgcn_raw_buffer_store_b64(d, orow, qo, (32 * pp + 1024 * k1) * 8u, 2);
        });
        __builtin_amdgcn_s_setprio(1);  // the next row's loads, stage A and first exchange write
    }
#endif
}

template <int B>
__global__ void build_table(const uint64_t* __restrict__ fwd, uint64_t* __restrict__ tab) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx < Shape<B>::TABLE_WORDS) tab[idx] = table_word<B>(fwd, idx);
}

template <int B>
int launch(Context* c, const uint64_t* in, size_t stride, size_t len, size_t rows, const uint64_t* tab,
           uint64_t* out) {
    using S = Shape<B>;
    const size_t cus = c->cu_count > 0 ? static_cast<size_t>(c->cu_count) : 256;
    const unsigned blocks = static_cast<unsigned>(std::min(rows, S::PER_CU * cus));
    auto k = len <= size_t{8} * S::M ? rows_kernel<B, 8> : len <= size_t{16} * S::M ? rows_kernel<B, 16>
                                                                                     : rows_kernel<B, 32>;
    if (S::LDS_BYTES > 65536)
        VMX_HIP(c, hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
                                       static_cast<int>(S::LDS_BYTES)));
    hipLaunchKernelGGL(k, dim3(blocks), dim3(S::THREADS), S::LDS_BYTES, c->stream, in, stride, len, rows, tab, out);
    VMX_HIP(c, hipGetLastError());
    return 0;
}

int build14(Context* c, TwiddleSet* t) {
    hipLaunchKernelGGL(build_table<4>, dim3((Shape<4>::TABLE_WORDS + 255) / 256), dim3(256), 0, c->stream,
                       static_cast<const uint64_t*>(t->fwd), t->grid);
    VMX_HIP(c, hipGetLastError());
    return 0;
}

}  // namespace rr

// n = 2^13: the tables share the encode's device table (encode_fast.hip).
int build_rr13_table(Context* c, const uint64_t* fwd, uint64_t* tab) {
    hipLaunchKernelGGL(rr::build_table<3>, dim3((rr::Shape<3>::TABLE_WORDS + 255) / 256), dim3(256), 0, c->stream,
                       fwd, tab);
    VMX_HIP(c, hipGetLastError());
    return 0;
}

int ntt13r_u64_rows(Context* c, const uint64_t* in, size_t stride, size_t len, size_t rows, size_t n, uint64_t* out,
                    TwiddleSet* t) {
    if (n != static_cast<size_t>(rr::Shape<3>::N) || len == 0 || len > n || stride < len || !t->fwd) return 1;
    if (!t->grid && c->coarse_active) return 1;  // tables may not grow inside a coarse scope
    if (rows == 0) return 0;
    const uint64_t* tab = enc13_rr_table(c, t);
    if (!tab) return -1;
    return rr::launch<3>(c, in, stride, len, rows, tab, out);
}

int ntt14r_u64_rows(Context* c, const uint64_t* in, size_t stride, size_t len, size_t rows, size_t n, uint64_t* out,
                    TwiddleSet* t) {
    if (n != static_cast<size_t>(rr::Shape<4>::N) || len == 0 || len > n || stride < len || !t->fwd) return 1;
    if (!t->grid && c->coarse_active) return 1;
    if (rows == 0) return 0;
    if (ensure_grid_twiddles(c, t, size_t{rr::Shape<4>::TABLE_WORDS} * sizeof(uint64_t), rr::build14)) return -1;
    return rr::launch<4>(c, in, stride, len, rows, t->grid, out);
}

}  // namespace vmx
