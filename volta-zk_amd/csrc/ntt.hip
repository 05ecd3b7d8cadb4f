// ntt.hip -- batched Goldilocks NTT kernels for gfx950.
//
// Semantics are the reference's NttPlan::forward (rust/volta-pcs/src/ntt.rs:36-61):
// out[j] = sum_i a_i w^(ij), w = 7^((p-1)/n), natural-order output.  Field sums
// are exact, so any factorisation of the DFT gives bit-identical results.
//
// Rows of n >= 2^13 (u64, Fp2, and i16 weights + pads message rows) run on the
// pass engine of ntt_reg.hip (register four-steps with shift-only sub-DFTs).
// The generic path below serves smaller rows (any power-of-two n <= 2^14): one
// workgroup per row, the whole row in LDS (<= 128 KiB of the 160 KiB per CU),
// bit-reversed load then radix-2^2 DIT passes (two stages per LDS round trip).
// One HBM read + one HBM write per element.
// Its twiddles come from the reference's table w^0..w^(n/2-1): a stage of
// length L of any sub-transform uses tw[k * n/L], and w^e for e >= n/2 is
// -tw[e - n/2].
#include <hip/hip_runtime.h>

#include <algorithm>

#include "context.hpp"
#include "gl64.hpp"
#include "kernels.hpp"
#include "lds_dit.hpp"

namespace vmx {

// w^e for 0 <= e < n from the half table.
__device__ __forceinline__ uint64_t tw_pow(const uint64_t* tw, size_t e, size_t half) {
    return e < half ? tw[e] : gl::neg(tw[e - half]);
}

// ---- input loaders ------------------------------------------------------------

// Dense u64 rows of `stride` elements; positions >= msg_len read as zero.
struct LoadU64 {
    const uint64_t* src;
    size_t stride;
    size_t msg_len;
    __device__ uint64_t operator()(size_t row, size_t j) const {
        return j < msg_len ? src[row * stride + j] : 0;
    }
};

// Strided u64 lanes of Fp2 rows (component comp of rows of n Fp2).
struct LoadFp2Comp {
    const uint64_t* src;  // Fp2 storage viewed as u64
    size_t n;
    int comp;
    __device__ uint64_t operator()(size_t row, size_t j) const { return src[2 * (row * n + j) + comp]; }
};

// PCS message rows lift(w) || pads || 0 (reference pcs_messages_kernel,
// cuda/volta_cuda_backend.cu:2950-2958), fused into the transform load.
struct LoadMsgI16 {
    const int16_t* w;
    const uint64_t* pads;
    size_t cols, pad;
    __device__ uint64_t operator()(size_t row, size_t j) const {
        if (j < cols) return gl::from_i16(w[row * cols + j]);
        if (j < cols + pad) return pads[row * pad + (j - cols)];
        return 0;
    }
};

struct StoreU64 {
    uint64_t* dst;
    __device__ void operator()(size_t idx, uint64_t v) const { dst[idx] = v; }
};

struct StoreFp2Comp {
    uint64_t* dst;
    int comp;
    __device__ void operator()(size_t idx, uint64_t v) const { dst[2 * idx + comp] = v; }
};

// ---- whole-row kernel (n <= 2^14) ----------------------------------------------

template <class Load, class Store>
__global__ __launch_bounds__(512) void ntt_row_lds(Load ld, Store st, int bits, const uint64_t* tw,
                                                  uint64_t scale) {
    extern __shared__ uint64_t s[];
    const size_t n = size_t{1} << bits;
    const size_t row = blockIdx.x;
    for (size_t j = threadIdx.x; j < n; j += blockDim.x) s[brev(static_cast<uint32_t>(j), bits)] = ld(row, j);
    __syncthreads();
    lds_dit(s, 1, bits, bits, tw);
    if (scale != 1) {
        for (size_t j = threadIdx.x; j < n; j += blockDim.x) st(row * n + j, gl::mul(s[j], scale));
    } else {
        for (size_t j = threadIdx.x; j < n; j += blockDim.x) st(row * n + j, s[j]);
    }
}

// ---- launchers -------------------------------------------------------------------------

// Row-offset adjusters so a launch can start at row r0.
static void shift_rows(LoadU64& l, StoreU64& s, size_t r0, size_t n) {
    l.src += r0 * l.stride;
    s.dst += r0 * n;
}
static void shift_rows(LoadMsgI16& l, StoreU64& s, size_t r0, size_t n) {
    l.w += r0 * l.cols;
    if (l.pad) l.pads += r0 * l.pad;
    s.dst += r0 * n;
}
static void shift_rows(LoadFp2Comp& l, StoreFp2Comp& s, size_t r0, size_t n) {
    l.src += 2 * r0 * l.n;
    s.dst += 2 * r0 * n;
}


static int ilog2(size_t n) {
    int b = 0;
    while ((size_t{1} << b) < n) ++b;
    return b;
}

constexpr int LDS_MAX_BITS = 14;           // 128 KiB of u64 per workgroup

template <class K>
static hipError_t allow_lds(K kernel, size_t bytes) {
    if (bytes <= 65536) return hipSuccess;
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
}

template <class Load, class Store>
static int run_ntt(Context* c, Load ld, Store st, size_t rows, size_t n, const uint64_t* tw, uint64_t scale) {
    const int bits = ilog2(n);
    if (bits <= LDS_MAX_BITS) {
        const size_t lds = n * sizeof(uint64_t);
        const int threads = static_cast<int>(std::min<size_t>(512, std::max<size_t>(64, n / 4)));
        auto k = ntt_row_lds<Load, Store>;
        VMX_HIP(c, allow_lds(k, lds));
        // Rows are independent; launch in slices that fit the 32-bit grid.
        for (size_t r0 = 0; r0 < rows; r0 += 0x7FFFFFFF) {
            const size_t cnt = std::min<size_t>(rows - r0, 0x7FFFFFFF);
            Load l2 = ld;
            Store s2 = st;
            shift_rows(l2, s2, r0, n);
            hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(cnt)), dim3(threads), lds, c->stream, l2, s2, bits,
                               tw, scale);
            VMX_HIP(c, hipGetLastError());
        }
        return 0;
    }
    // Rows above 2^LDS_MAX_BITS points run on the pass engine (ntt_reg.hip), whose
    // tables every size from 2^13 to 2^31 gets with its twiddles.
    return fail_msg(c, "NTT rows above 2^14 points need the pass engine's tables");
}

static RegTables reg_tables(const TwiddleSet* t) {
    RegTables rt;
    rt.inner = t->reg;
    rt.split = t->reg + 2048;
    rt.split_h = t->reg_h;
    return rt;
}

int ntt_fp_rows(Context* c, const uint64_t* in, size_t in_stride, size_t msg_len, size_t rows, size_t n,
                uint64_t* out, TwiddleSet* t, bool inverse) {
    // n = 2^13 forward: one pass over HBM (the pass engine's two otherwise),
    // unless its device-built table is missing inside a coarse timing scope,
    // where tables may not grow.
    if (!inverse && n == 8192 && (t->grid || !c->coarse_active)) {
        const int rc = ntt13r_u64_rows(c, in, in_stride, msg_len, rows, n, out, t);
        if (rc <= 0) return rc;
    }
    if (!inverse && n == 16384) {
        const int rc = ntt14r_u64_rows(c, in, in_stride, msg_len, rows, n, out, t);
        if (rc <= 0) return rc;
    }
    // n = 2^15 forward: one pass as well.
    if (!inverse && n == 32768) {
        const int rc = ntt15_u64_rows(c, in, in_stride, msg_len, rows, n, out, t);
        if (rc <= 0) return rc;
    }
    if (t->reg) return reg_ntt(c, reg_tables(t), in, in_stride, msg_len, out, rows, ilog2(n), 1, inverse);
    const uint64_t scale = inverse ? gl::inv_host(gl::canon(n)) : 1;
    const uint64_t* tw = inverse ? t->inv : t->fwd;
    if (!tw) return fail_msg(c, "NTT twiddle table missing");
    return run_ntt(c, LoadU64{in, in_stride, msg_len}, StoreU64{out}, rows, n, tw, scale);
}

int ntt_fp2_rows(Context* c, const uint64_t* in, size_t rows, size_t n, uint64_t* out, const TwiddleSet* t) {
    if (t->reg) return reg_ntt(c, reg_tables(t), in, n, n, out, rows, ilog2(n), 2, false);
    for (int comp = 0; comp < 2; ++comp)
        if (run_ntt(c, LoadFp2Comp{in, n, comp}, StoreFp2Comp{out, comp}, rows, n, t->fwd, 1)) return -1;
    return 0;
}

int ntt_msg_i16_rows(Context* c, const int16_t* w, const uint64_t* pads, size_t rows, size_t cols, size_t pad,
                     size_t n, uint64_t* out, TwiddleSet* t) {
    if (n == 32768) {
        const int rc = ntt15_msg_rows(c, w, pads, cols, pad, rows, n, out, t);
        if (rc <= 0) return rc;
    }
    if (t->reg) return reg_ntt_msg_i16(c, reg_tables(t), w, pads, cols, pad, out, rows, ilog2(n));
    return run_ntt(c, LoadMsgI16{w, pads, cols, pad}, StoreU64{out}, rows, n, t->fwd, 1);
}

}  // namespace vmx
