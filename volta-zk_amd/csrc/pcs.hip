// pcs.hip -- PCS row kernels for gfx950: message rows, row combinations,
// column gathers, Fp2 powers/adds, ChaCha8 FpStream rows, measurement probes.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <string>
#include <type_traits>

#include "chacha8.hpp"
#include "context.hpp"
#include "gl64.hpp"
#include "kernels.hpp"

namespace vmx {

using gl::Fp2;

static unsigned grid_for(size_t items, size_t per_block, size_t cap = 1u << 20) {
    const size_t g = (items + per_block - 1) / per_block;
    return static_cast<unsigned>(std::max<size_t>(1, std::min(g, cap)));
}

// ---- message rows (reference pcs_messages_kernel, .cu:2950-2958) --------------------
// A row is cut into S spans of MSG_THREADS x MSG_PER consecutive elements.
// Workgroup b walks rows r0, r0 + G, r0 + 2G, ... (G = gridDim.x / S row
// groups, r0 = b / S) and takes span (b + i) mod S of its i-th row, so every
// (row, span) is written once and each workgroup meets every kind of span in
// turn: the weight spans, which wait on loads, are spread over all workgroups
// instead of holding a quarter of them to the end.  The next unit's weights
// load before the current unit's stores.  The span's kind is uniform over the
// workgroup (a scalar branch); there is no division per element.  Each store
// instruction writes 512 contiguous bytes, non-temporal (the rows are larger
// than the caches).  8-byte stores: the output may start at any element
// offset.  C3 (2^16 rows of 2^11 weights into 2^13): 1.09 ms with a fixed span
// per workgroup, 0.91 ms with the rotation, 0.90 ms with the prefetch, 0.845
// ms at 128 workgroups per CU (64: 0.90, 256: 0.89); the same stores without
// any loads take 0.80 ms.
constexpr int MSG_THREADS = 256, MSG_PER = 8;

__global__ __launch_bounds__(MSG_THREADS) void messages_kernel(const int16_t* w, const uint64_t* pads, uint64_t* out,
                                                               size_t rows, size_t cols, size_t pad, size_t code_len,
                                                               unsigned spans_per_row) {
    constexpr size_t SPAN = size_t{MSG_THREADS} * MSG_PER;
    const unsigned row_step = gridDim.x / spans_per_row;
    size_t r = blockIdx.x / spans_per_row;
    unsigned s = blockIdx.x - static_cast<unsigned>(r) * spans_per_row;
    // 0: all zero tail, 1: all weights, 2: mixed
    auto kind = [&](unsigned sp) {
        const size_t j0 = static_cast<size_t>(sp) * SPAN;
        return j0 >= cols + pad ? 0 : (j0 + SPAN <= cols ? 1 : 2);
    };
    auto load_span = [&](size_t row, unsigned sp, int16_t* dst) {
        const int16_t* src = w + row * cols + static_cast<size_t>(sp) * SPAN + threadIdx.x;
#pragma unroll
        for (int k = 0; k < MSG_PER; ++k) dst[k] = src[static_cast<size_t>(k) * MSG_THREADS];
    };
    int16_t nxt[MSG_PER];
    if (r < rows && kind(s) == 1) load_span(r, s, nxt);
    for (; r < rows; r += row_step, s = (s + 1 == spans_per_row) ? 0 : s + 1) {
        const size_t j0 = static_cast<size_t>(s) * SPAN;
        uint64_t* o = out + r * code_len;
        const int kd = kind(s);
        int16_t cur[MSG_PER];
        if (kd == 1) {
#pragma unroll
            for (int k = 0; k < MSG_PER; ++k) cur[k] = nxt[k];
        }
        const size_t rn = r + row_step;
        const unsigned sn = (s + 1 == spans_per_row) ? 0 : s + 1;
        if (rn < rows && kind(sn) == 1) load_span(rn, sn, nxt);
        if (kd == 0) {
#pragma unroll
            for (int k = 0; k < MSG_PER; ++k) {
                const size_t j = j0 + static_cast<size_t>(k) * MSG_THREADS + threadIdx.x;
                if (j < code_len) __builtin_nontemporal_store(uint64_t{0}, o + j);
            }
        } else if (kd == 1) {
#pragma unroll
            for (int k = 0; k < MSG_PER; ++k) {
                const size_t j = j0 + static_cast<size_t>(k) * MSG_THREADS + threadIdx.x;
                __builtin_nontemporal_store(gl::from_i16(cur[k]), o + j);
            }
        } else {
            const int16_t* wr = w + r * cols;
#pragma unroll
            for (int k = 0; k < MSG_PER; ++k) {
                const size_t j = j0 + static_cast<size_t>(k) * MSG_THREADS + threadIdx.x;
                if (j < code_len) {
                    uint64_t x = 0;
                    if (j < cols) x = gl::from_i16(wr[j]);
                    else if (j < cols + pad) x = pads[r * pad + (j - cols)];
                    __builtin_nontemporal_store(x, o + j);
                }
            }
        }
    }
}

int pcs_messages(Context* c, const int16_t* w, const uint64_t* pads, size_t rows, size_t cols, size_t pad,
                 size_t code_len, uint64_t* out) {
    constexpr size_t SPAN = size_t{MSG_THREADS} * MSG_PER;
    const size_t spans = (code_len + SPAN - 1) / SPAN;
    if (spans > (1u << 20)) return fail_msg(c, "message row too long for the message kernel");
    const size_t cus = c->cu_count > 0 ? static_cast<size_t>(c->cu_count) : 256;
    // rows per span column: enough workgroups for about 128 per CU, at most one per row
    const size_t row_groups = std::max<size_t>(1, std::min(rows, std::max<size_t>(1, cus * 128 / spans)));
    const unsigned blocks = static_cast<unsigned>(spans * row_groups);
    hipLaunchKernelGGL(messages_kernel, dim3(blocks), dim3(MSG_THREADS), 0, c->stream, w, pads, out, rows, cols, pad,
                       code_len, static_cast<unsigned>(spans));
    VMX_HIP(c, hipGetLastError());
    return 0;
}

// ---- row combinations ---------------------------------------------------------------------
//
// out[comb][j] = sum_i coeff[comb][i] * msg_i[j] (reference combine_row_range,
// rust/volta-pcs/src/ligero.rs:1114-1135; coefficient layout combinations x
// rows, rust/volta-accel/src/lib.rs:6522-6569).  Unlike the reference kernel,
// which re-reads the matrix once per (combination, column) thread, the matrix
// is read once per pair of combinations: each workgroup owns a chunk of rows x
// a tile of columns, accumulates two combinations lazily, and writes one
// partial per chunk; a second kernel sums partials mod p.  A chunk whose
// coefficients are zero for the pair is not read at all (an opening's block
// claims weight only their own block's rows).
//
// i16 data: with w' = w + 2^15 in [0, 2^16) and a coefficient component
// x = xh*2^32 + xl, sum_i x_i w_i = sum xl_i w'_i + 2^32 sum xh_i w'_i
// - 2^15 sum_i x_i.  Each 32x16-bit product is < 2^48, so u64 accumulators
// absorb up to 2^16 rows exactly; the fold to a field element happens once.

constexpr int COMB_THREADS = 256;
constexpr size_t COMB_CHUNK = 128;  // rows per partial (u64 rows)

// i16 rows: a workgroup's four waves share one tile of 64 x CI_COLS columns
// and split the chunk's rows four ways; the waves' sums meet in LDS, so one
// partial leaves per workgroup.  Four columns per thread keep the
// accumulators at 64 VGPRs (4 waves per SIMD).
constexpr int CI_COLS = 4;          // columns per thread (one 8-byte i16 load)
typedef uint32_t CombWords __attribute__((ext_vector_type(CI_COLS / 2)));
constexpr int CI_WAVES = 4;
constexpr int CI_TILE = 64 * CI_COLS;  // columns per workgroup
constexpr size_t CI_CHUNK = 512;    // rows per partial at most (128 per wave)
constexpr int CI_UNROLL = 8;        // row loads kept in flight per thread

// S[ck][comb][h] = sum over the chunk's rows of component h of coeff[comb][i]
// (mod p): the 2^15 bias correction of the offset-binary trick below.
// nz[ck][comb] = 1 when any coefficient of the chunk is nonzero: the exact
// sums of the 32-bit halves are zero only then (a nonzero chunk can sum to
// 0 mod p, so the field sums cannot tell).  A block claim's equality weights
// cover only the rows of its block, so most (chunk, combination) pairs of an
// opening are zero and skip their share of the matrix.
__global__ __launch_bounds__(256) void coeff_chunk_sums(const Fp2* coeffs, uint64_t* sums, uint32_t* nz,
                                                        size_t rows, size_t chunk) {
    __shared__ uint64_t red[4][256];
    const size_t ck = blockIdx.x, comb = blockIdx.y, combinations = gridDim.y;
    const size_t r0 = ck * chunk, r1 = min(rows, r0 + chunk);
    uint64_t lo0 = 0, hi0 = 0, lo1 = 0, hi1 = 0;  // 32-bit halves summed exactly
    for (size_t i = r0 + threadIdx.x; i < r1; i += blockDim.x) {
        const Fp2 cf = coeffs[comb * rows + i];
        lo0 += static_cast<uint32_t>(cf.c0);
        hi0 += cf.c0 >> 32;
        lo1 += static_cast<uint32_t>(cf.c1);
        hi1 += cf.c1 >> 32;
    }
    red[0][threadIdx.x] = lo0;
    red[1][threadIdx.x] = hi0;
    red[2][threadIdx.x] = lo1;
    red[3][threadIdx.x] = hi1;
    __syncthreads();
    for (int w = blockDim.x / 2; w > 0; w >>= 1) {
        if (static_cast<int>(threadIdx.x) < w)
            for (int q = 0; q < 4; ++q) red[q][threadIdx.x] += red[q][threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const uint64_t two32 = 0x100000000ull;
        // chunk <= 2^16 rows keeps each half-sum below 2^48
        sums[(ck * combinations + comb) * 2 + 0] = gl::add(gl::canon(red[0][0]), gl::mul(gl::canon(red[1][0]), two32));
        sums[(ck * combinations + comb) * 2 + 1] = gl::add(gl::canon(red[2][0]), gl::mul(gl::canon(red[3][0]), two32));
        nz[ck * combinations + comb] = (red[0][0] | red[1][0] | red[2][0] | red[3][0]) != 0;
    }
}

// out[comb][j] = sum_i coeff[comb][i] * msg_i[j] (reference combine_row_range,
// rust/volta-pcs/src/ligero.rs:1114-1135) for KC combinations at once.
// i16 data: with w' = w + 2^15 in [0, 2^16) and a coefficient component
// x = xh*2^32 + xl, sum_i x_i w_i = sum xl_i w'_i + 2^32 sum xh_i w'_i
// - 2^15 sum_i x_i.  Each 32x16-bit product is < 2^48, so u64 accumulators
// absorb up to 2^16 rows exactly; the fold to a field element happens once.
// Combinations comb_base + KC z .. + KC - 1 for z = blockIdx.z.  A chunk whose
// coefficients are all zero for these combinations (nz) reads no matrix row:
// it writes zeros when its partials are the output (one chunk), and nothing
// otherwise (reduce_partials skips it).
template <int KC>
__global__ __launch_bounds__(COMB_THREADS) void combine_i16_partial(const int16_t* w, const Fp2* coeffs,
                                                                   const uint64_t* sums, const uint32_t* nz,
                                                                   Fp2* partials, size_t rows, size_t cols,
                                                                   size_t msg_len, size_t comb_base,
                                                                   size_t combinations, size_t chunk, int vec_ok,
                                                                   int direct) {
    __shared__ Fp2 red[CI_WAVES - 1][KC][CI_COLS][64];
    // the wave index is uniform: row bounds and coefficient addresses stay scalar (SMEM loads)
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const size_t j0 = (static_cast<size_t>(blockIdx.x) * 64 + lane) * CI_COLS;
    const size_t ck = blockIdx.y;
    const size_t comb0 = comb_base + static_cast<size_t>(KC) * blockIdx.z;
    uint32_t any = 0;
#pragma unroll
    for (int k = 0; k < KC; ++k) any |= nz[ck * combinations + comb0 + k];
    if (!any) {  // uniform over the workgroup
        if (!direct || wave > 0) return;
#pragma unroll
        for (int k = 0; k < KC; ++k)
#pragma unroll
            for (int q = 0; q < CI_COLS; ++q)
                if (j0 + q < cols) partials[(ck * combinations + comb0 + k) * msg_len + j0 + q] = Fp2{0, 0};
        return;
    }
    const size_t c0 = ck * chunk, c1 = min(rows, c0 + chunk);
    const size_t per = (c1 - c0 + CI_WAVES - 1) / CI_WAVES;
    const size_t r0 = min(c1, c0 + wave * per), r1 = min(c1, r0 + per);
    uint64_t acc_lo[KC][2][CI_COLS] = {};
    uint64_t acc_hi[KC][2][CI_COLS] = {};
    auto accumulate = [&](size_t i, const uint32_t* wp) {
#pragma unroll
        for (int k = 0; k < KC; ++k) {
            const Fp2 cf = coeffs[(comb0 + k) * rows + i];
            const uint64_t comp[2] = {cf.c0, cf.c1};
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t xl = static_cast<uint32_t>(comp[h]);
                const uint32_t xh = static_cast<uint32_t>(comp[h] >> 32);
#pragma unroll
                for (int q = 0; q < CI_COLS; ++q) {
                    acc_lo[k][h][q] += static_cast<uint64_t>(xl) * wp[q];
                    acc_hi[k][h][q] += static_cast<uint64_t>(xh) * wp[q];
                }
            }
        }
    };
    // The vector/scalar load choice is made once, outside the row loop, so the
    // loop body has no branches and its CI_UNROLL row loads are all in flight
    // together.
    auto rows_loop = [&](auto fast_tag) {
        constexpr bool FAST = decltype(fast_tag)::value;
        auto load = [&](size_t i, uint32_t* wp) {
            if constexpr (FAST) {
                // CI_COLS i16 in one aligned vector load of CI_COLS / 2 words
                const CombWords raw =
                    __builtin_nontemporal_load(reinterpret_cast<const CombWords*>(w + i * cols + j0));
#pragma unroll
                for (int q = 0; q < CI_COLS / 2; ++q) {
                    wp[2 * q] = (raw[q] & 0xFFFFu) ^ 0x8000u;
                    wp[2 * q + 1] = (raw[q] >> 16) ^ 0x8000u;
                }
            } else {
#pragma unroll
                for (int q = 0; q < CI_COLS; ++q) {
                    const size_t j = min(j0 + q, cols - 1);  // in bounds; masked below
                    const uint32_t x = static_cast<uint32_t>(static_cast<uint16_t>(w[i * cols + j])) ^ 0x8000u;
                    wp[q] = j0 + q < cols ? x : 0x8000u;
                }
            }
        };
        size_t i = r0;
        for (; i + CI_UNROLL <= r1; i += CI_UNROLL) {
            uint32_t wp[CI_UNROLL][CI_COLS];
#pragma unroll
            for (int u = 0; u < CI_UNROLL; ++u) load(i + u, wp[u]);
#pragma unroll
            for (int u = 0; u < CI_UNROLL; ++u) accumulate(i + u, wp[u]);
        }
        for (; i < r1; ++i) {
            uint32_t wp[CI_COLS];
            load(i, wp);
            accumulate(i, wp);
        }
    };
    if ((j0 + CI_COLS <= cols) && vec_ok) rows_loop(std::true_type{});
    else rows_loop(std::false_type{});
    // this wave's sums as field elements: sum x w' = sum xl w' + 2^32 sum xh w'
    const uint64_t two32 = 0x100000000ull;
    auto fold = [&](int k, int h, int q) {
        return gl::add(gl::canon(acc_lo[k][h][q]), gl::mul(gl::canon(acc_hi[k][h][q]), two32));
    };
    if (wave > 0) {
#pragma unroll
        for (int k = 0; k < KC; ++k)
#pragma unroll
            for (int q = 0; q < CI_COLS; ++q) red[wave - 1][k][q][lane] = Fp2{fold(k, 0, q), fold(k, 1, q)};
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int k = 0; k < KC; ++k) {
        // the offset-binary bias of the whole chunk: 2^15 sum_i x_i
        uint64_t bias[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) bias[h] = gl::mul(sums[(ck * combinations + comb0 + k) * 2 + h], 0x8000ull);
#pragma unroll
        for (int q = 0; q < CI_COLS; ++q) {
            const size_t j = j0 + q;
            if (j >= cols) break;
            Fp2 t{fold(k, 0, q), fold(k, 1, q)};
#pragma unroll
            for (int o = 0; o < CI_WAVES - 1; ++o) t = gl::fp2_add(t, red[o][k][q][lane]);
            partials[(ck * combinations + comb0 + k) * msg_len + j] = Fp2{gl::sub(t.c0, bias[0]), gl::sub(t.c1, bias[1])};
        }
    }
}

// Pad columns j in [cols, cols+pad): full field products.
constexpr int PAD_UNROLL = 8;  // rows whose loads are in flight together
constexpr int PAD_WAVES = 4;   // the chunk's rows split four ways, summed in LDS

// A workgroup takes 64 pad columns (one per lane) of one (chunk, combination);
// its four waves sum a quarter of the chunk's rows each.  An opening's
// proximity pass has a single combination: one thread per column and chunk
// would leave most CUs idle and serialise the chunk's row loads.
__global__ __launch_bounds__(64 * PAD_WAVES) void combine_pads_partial(const uint64_t* pads, const Fp2* coeffs,
                                                                      const uint32_t* nz, Fp2* partials, size_t rows,
                                                                      size_t cols, size_t pad, size_t msg_len,
                                                                      size_t combinations, size_t chunk, int direct) {
    __shared__ Fp2 red[PAD_WAVES - 1][64];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const size_t p = static_cast<size_t>(blockIdx.x) * 64 + lane;
    const size_t comb = blockIdx.z, ck = blockIdx.y;
    Fp2* dst = partials + (ck * combinations + comb) * msg_len + cols + p;
    if (!nz[ck * combinations + comb]) {  // zero coefficients (uniform): as combine_i16_partial
        if (direct && wave == 0 && p < pad) *dst = Fp2{0, 0};
        return;
    }
    const size_t c0 = ck * chunk, c1 = min(rows, c0 + chunk);
    const size_t per = (c1 - c0 + PAD_WAVES - 1) / PAD_WAVES;
    const size_t r0 = min(c1, c0 + wave * per), r1 = min(c1, r0 + per);
    const size_t pc = p < pad ? p : pad - 1;  // in bounds; the column is masked at the write
    const Fp2* cf = coeffs + comb * rows;
    Fp2 acc{0, 0};
    size_t i = r0;
    for (; i + PAD_UNROLL <= r1; i += PAD_UNROLL) {
        Fp2 cv[PAD_UNROLL];
        uint64_t pv[PAD_UNROLL];
#pragma unroll
        for (int u = 0; u < PAD_UNROLL; ++u) {
            cv[u] = cf[i + u];
            pv[u] = pads[(i + u) * pad + pc];
        }
#pragma unroll
        for (int u = 0; u < PAD_UNROLL; ++u) acc = gl::fp2_add(acc, gl::fp2_mul_base(cv[u], pv[u]));
    }
    for (; i < r1; ++i) acc = gl::fp2_add(acc, gl::fp2_mul_base(cf[i], pads[i * pad + pc]));
    if (wave > 0) red[wave - 1][lane] = acc;
    __syncthreads();
    if (wave == 0 && p < pad) {
#pragma unroll
        for (int o = 0; o < PAD_WAVES - 1; ++o) acc = gl::fp2_add(acc, red[o][lane]);
        *dst = acc;
    }
}

// Dense u64 rows: 128-bit products accumulated in three 64-bit limbs, folded
// once per chunk (2^128 = -2^32 mod p).
__device__ __forceinline__ uint64_t fold192(uint64_t lo, uint64_t hi, uint64_t top) {
    const uint64_t base = gl::fold128(lo, hi);
    // 2^128 = eps^2 = -2^32 (mod p)
    return gl::sub(base, gl::mul(gl::canon(top), 0x100000000ull));
}

constexpr int FP_COLS = 2;

template <int KC>
__global__ __launch_bounds__(COMB_THREADS) void combine_fp_partial(const uint64_t* m, const Fp2* coeffs,
                                                                  Fp2* partials, size_t rows, size_t cols,
                                                                  size_t comb0, size_t combinations,
                                                                  size_t chunk) {
    const size_t j0 = (static_cast<size_t>(blockIdx.x) * COMB_THREADS + threadIdx.x) * FP_COLS;
    const size_t ck = blockIdx.y;
    const size_t r0 = ck * chunk, r1 = min(rows, r0 + chunk);
    uint64_t lo[KC][2][FP_COLS] = {}, hi[KC][2][FP_COLS] = {}, top[KC][2][FP_COLS] = {};
    for (size_t i = r0; i < r1; ++i) {
        uint64_t x[FP_COLS];
#pragma unroll
        for (int q = 0; q < FP_COLS; ++q) x[q] = (j0 + q < cols) ? m[i * cols + j0 + q] : 0;
#pragma unroll
        for (int k = 0; k < KC; ++k) {
            const Fp2 cf = coeffs[(comb0 + k) * rows + i];
            const uint64_t comp[2] = {cf.c0, cf.c1};
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int q = 0; q < FP_COLS; ++q) {
                    uint64_t pl, ph;
                    gl::mul_wide(comp[h], x[q], pl, ph);
                    const uint64_t nl = lo[k][h][q] + pl;
                    const uint64_t c1 = nl < pl;
                    const uint64_t t = ph + c1;  // ph <= 2^64-2, no overflow
                    const uint64_t nh = hi[k][h][q] + t;
                    top[k][h][q] += (nh < t);
                    lo[k][h][q] = nl;
                    hi[k][h][q] = nh;
                }
            }
        }
    }
#pragma unroll
    for (int k = 0; k < KC; ++k) {
        if (comb0 + k >= combinations) break;
#pragma unroll
        for (int q = 0; q < FP_COLS; ++q) {
            const size_t j = j0 + q;
            if (j >= cols) break;
            partials[(ck * combinations + comb0 + k) * cols + j] =
                Fp2{fold192(lo[k][0][q], hi[k][0][q], top[k][0][q]), fold192(lo[k][1][q], hi[k][1][q], top[k][1][q])};
        }
    }
}

// out[z] = sum over chunks of partials[ck][z]: 64 outputs x 16 chunk lanes per
// workgroup, then a tree over the lanes in LDS.
constexpr int RED_Z = 64;
constexpr int RED_LANES = 16;

// With nz (combinations x msg_len outputs per chunk), a chunk whose flag for
// the output's combination is 0 has no partial and is skipped.
__global__ __launch_bounds__(RED_Z * RED_LANES) void reduce_partials(const Fp2* partials, Fp2* out, size_t chunks,
                                                                     size_t per_chunk, const uint32_t* nz,
                                                                     size_t combinations, size_t msg_len) {
    __shared__ Fp2 red[RED_LANES][RED_Z];
    const int tz = threadIdx.x % RED_Z, tl = threadIdx.x / RED_Z;
    const size_t z = static_cast<size_t>(blockIdx.x) * RED_Z + tz;
    Fp2 acc{0, 0};
    if (z < per_chunk) {
        const size_t comb = nz ? z / msg_len : 0;
        for (size_t ck = tl; ck < chunks; ck += RED_LANES)
            if (!nz || nz[ck * combinations + comb]) acc = gl::fp2_add(acc, partials[ck * per_chunk + z]);
    }
    red[tl][tz] = acc;
    __syncthreads();
    for (int w = RED_LANES / 2; w > 0; w >>= 1) {
        if (tl < w) red[tl][tz] = gl::fp2_add(red[tl][tz], red[tl + w][tz]);
        __syncthreads();
    }
    if (tl == 0 && z < per_chunk) out[z] = red[0][tz];
}

template <class F>
static int launch_comb_groups(size_t combinations, F&& f) {
    for (size_t c0 = 0; c0 < combinations;) {
        const size_t left = combinations - c0;
        const int kc = left >= 2 ? 2 : 1;
        if (f(c0, kc)) return -1;
        c0 += kc;
    }
    return 0;
}

// Rows per partial: at most `largest`, or fewer (down to 8) when the column
// blocks times the chunks would not give about 1024 workgroups, so small
// matrices still spread over the GPU's 256 CUs.  The reduce pass sums the chunks.
static size_t comb_chunk(size_t rows, size_t col_blocks, size_t largest = COMB_CHUNK) {
    size_t chunk = largest;
    while (chunk > 8 && col_blocks * ((rows + chunk - 1) / chunk) < 1024) chunk >>= 1;
    return chunk;
}

// The i16 combination's launch plan: rows per partial chunk and the bytes of
// the per-chunk partials (none for one chunk: it writes out directly) and of
// the chunks' coefficient sums followed by their nonzero flags.
struct CombinePlan {
    size_t msg_len, col_blocks, chunk, chunks, per_chunk, part_bytes, sum_bytes;
};

// Rows per chunk at most: each wave's u64 accumulators, and each chunk's
// coefficient half-sums, stay exact up to 2^16 rows.
constexpr size_t CI_CHUNK_MAX = size_t{1} << 16;

// The plan with comb_chunk's rows per chunk, or `chunk` rows when given.
static int combine_plan(Context* c, size_t rows, size_t cols, size_t pad, size_t combinations, CombinePlan* p,
                        size_t chunk = 0) {
    p->msg_len = cols + pad;
    p->col_blocks = (cols + CI_TILE - 1) / CI_TILE;
    p->chunk = chunk ? chunk : comb_chunk(rows, p->col_blocks, CI_CHUNK);
    p->chunks = (rows + p->chunk - 1) / p->chunk;
    size_t bytes = 0;
    if (!mul_ok(combinations, p->msg_len, &p->per_chunk) || !mul_ok(p->per_chunk * sizeof(Fp2), p->chunks, &bytes) ||
        !mul_ok(p->chunks * combinations, 2 * sizeof(uint64_t) + sizeof(uint32_t), &p->sum_bytes))
        return fail_msg(c, "PCS combination partials overflow size_t");
    if (p->chunks > 65535 || combinations > 65535)
        return fail_msg(c, "PCS combination row or combination count exceeds the supported maximum");
    p->part_bytes = p->chunks > 1 ? bytes : 0;
    return 0;
}

// The coefficient sums and flags are written first in the same call; a
// partial is written for every (chunk, combination) the flags mark nonzero
// (and for all of them when the partials are the output), and the reduction
// reads exactly those, so the buffers need no clearing.
static int combine_launch(Context* c, const int16_t* w, const uint64_t* pads, const Fp2* coeffs, size_t rows,
                          size_t cols, size_t pad, size_t combinations, Fp2* out, const CombinePlan& pl, Fp2* part,
                          uint64_t* sums) {
    const size_t chunk = pl.chunk, chunks = pl.chunks, msg_len = pl.msg_len;
    uint32_t* nz = reinterpret_cast<uint32_t*>(sums + chunks * combinations * 2);
    const int direct = chunks == 1;
    if (direct) part = out;  // one chunk: the partials are the result
    hipLaunchKernelGGL(coeff_chunk_sums, dim3(static_cast<unsigned>(chunks), static_cast<unsigned>(combinations)),
                       dim3(256), 0, c->stream, coeffs, sums, nz, rows, chunk);
    VMX_HIP(c, hipGetLastError());
    // Vector row loads need a base and a row pitch aligned to CI_COLS i16.
    const int vec_ok = (reinterpret_cast<uintptr_t>(w) % (2 * CI_COLS) == 0) && (cols % CI_COLS == 0);
    const size_t pairs = combinations / 2;
    if (pairs) {  // every pair of combinations in one launch
        const dim3 grid(static_cast<unsigned>(pl.col_blocks), static_cast<unsigned>(chunks),
                        static_cast<unsigned>(pairs));
        hipLaunchKernelGGL(combine_i16_partial<2>, grid, dim3(COMB_THREADS), 0, c->stream, w, coeffs,
                           static_cast<const uint64_t*>(sums), static_cast<const uint32_t*>(nz), part, rows, cols,
                           msg_len, size_t{0}, combinations, chunk, vec_ok, direct);
        VMX_HIP(c, hipGetLastError());
    }
    if (combinations & 1) {  // the last, odd one
        const dim3 grid(static_cast<unsigned>(pl.col_blocks), static_cast<unsigned>(chunks), 1u);
        hipLaunchKernelGGL(combine_i16_partial<1>, grid, dim3(COMB_THREADS), 0, c->stream, w, coeffs,
                           static_cast<const uint64_t*>(sums), static_cast<const uint32_t*>(nz), part, rows, cols,
                           msg_len, combinations - 1, combinations, chunk, vec_ok, direct);
        VMX_HIP(c, hipGetLastError());
    }
    if (pad) {
        const dim3 g(static_cast<unsigned>((pad + 63) / 64), static_cast<unsigned>(chunks),
                     static_cast<unsigned>(combinations));
        hipLaunchKernelGGL(combine_pads_partial, g, dim3(64 * PAD_WAVES), 0, c->stream, pads, coeffs,
                           static_cast<const uint32_t*>(nz), part, rows, cols, pad, msg_len, combinations, chunk,
                           direct);
        VMX_HIP(c, hipGetLastError());
    }
    if (direct) return 0;
    hipLaunchKernelGGL(reduce_partials, dim3(static_cast<unsigned>((pl.per_chunk + RED_Z - 1) / RED_Z)),
                       dim3(RED_Z * RED_LANES), 0, c->stream, static_cast<const Fp2*>(part), out, chunks,
                       pl.per_chunk, static_cast<const uint32_t*>(nz), combinations, msg_len);
    VMX_HIP(c, hipGetLastError());
    return 0;
}

int pcs_combine_rows(Context* c, const int16_t* w, const uint64_t* pads, const Fp2* coeffs, size_t rows,
                     size_t cols, size_t pad, size_t combinations, Fp2* out) {
    CombinePlan pl{};
    if (combine_plan(c, rows, cols, pad, combinations, &pl)) return -1;
    if ((pl.part_bytes && ensure_ws(c, WS_PARTIALS, pl.part_bytes)) || ensure_ws(c, WS_AUX2, pl.sum_bytes)) return -1;
    return combine_launch(c, w, pads, coeffs, rows, cols, pad, combinations, out, pl,
                          pl.part_bytes ? ws<Fp2>(c, WS_PARTIALS) : nullptr, ws<uint64_t>(c, WS_AUX2));
}

// ---- the allocation-free combination ------------------------------------------------
// A file-scope scratch array serves the partials and coefficient sums of
// pcs_combine_rows_noalloc, so that entry point allocates nothing.  Host code
// never uses the array's name as an address: combine_scratch_attach resolves
// this device's copy once (hipGetSymbolAddress, with the device current) and
// every launch takes that pointer.  All contexts on one GPU share its array:
// each use records a per-device event after its last launch, and the next use
// (from any context of that device) makes its own stream wait on that event
// first, so uses on one GPU run one after another on the device.
static __device__ __align__(256) unsigned char combine_scratch[COMBINE_SCRATCH_BYTES];

namespace {
struct ScratchDevice {
    void* ptr = nullptr;
    hipEvent_t last = nullptr;  // recorded after the latest use's launches
    bool used = false;
};
std::mutex scratch_mu;
std::map<int, ScratchDevice> scratch_by_device;  // each device's copy of combine_scratch
}  // namespace

int combine_scratch_attach(Context* c) {
    std::lock_guard<std::mutex> lock(scratch_mu);
    auto it = scratch_by_device.find(c->device);
    if (it == scratch_by_device.end()) {
        ScratchDevice d;
        hipError_t e = hipGetSymbolAddress(&d.ptr, HIP_SYMBOL(combine_scratch));
        if (e == hipSuccess && d.ptr) e = hipEventCreateWithFlags(&d.last, hipEventDisableTiming);
        if (e != hipSuccess || !d.ptr) {
            c->scratch = nullptr;
            c->scratch_error = std::string("resolving combine_scratch failed: ") +
                               (e != hipSuccess ? hipGetErrorString(e) : "null address");
            return -1;
        }
        it = scratch_by_device.emplace(c->device, d).first;
    }
    c->scratch = it->second.ptr;
    return 0;
}

int pcs_combine_rows_noalloc(Context* c, const int16_t* w, const uint64_t* pads, const Fp2* coeffs, size_t rows,
                             size_t cols, size_t pad, size_t combinations, Fp2* out) {
    CombinePlan pl{};
    if (combine_plan(c, rows, cols, pad, combinations, &pl)) return -1;
    if (!c->scratch) {
        std::string m = "allocation-free PCS combination unavailable on this device: " + c->scratch_error;
        return fail_msg(c, m.c_str());
    }
    auto span = [](const CombinePlan& q) { return (q.part_bytes + 255) / 256 * 256; };
    // A plan whose partials do not fit the array takes larger row chunks
    // (fewer partials, the same sums) up to CI_CHUNK_MAX rows per chunk.
    while (span(pl) + pl.sum_bytes > COMBINE_SCRATCH_BYTES && pl.chunks > 1 && pl.chunk < CI_CHUNK_MAX)
        if (combine_plan(c, rows, cols, pad, combinations, &pl, std::min(pl.chunk * 2, CI_CHUNK_MAX))) return -1;
    const size_t part_span = span(pl);
    if (part_span + pl.sum_bytes > COMBINE_SCRATCH_BYTES) {
        std::string m = "allocation-free PCS combination needs " + std::to_string(part_span + pl.sum_bytes) +
                        " bytes of scratch at " + std::to_string(CI_CHUNK_MAX) +
                        " rows per partial chunk; its fixed array holds " + std::to_string(COMBINE_SCRATCH_BYTES);
        return fail_msg(c, m.c_str());
    }
    unsigned char* base = static_cast<unsigned char*>(c->scratch);
    std::lock_guard<std::mutex> lock(scratch_mu);
    ScratchDevice& d = scratch_by_device.at(c->device);
    if (d.used) VMX_HIP(c, hipStreamWaitEvent(c->stream, d.last, 0));
    if (combine_launch(c, w, pads, coeffs, rows, cols, pad, combinations, out, pl,
                       pl.part_bytes ? reinterpret_cast<Fp2*>(base) : nullptr,
                       reinterpret_cast<uint64_t*>(base + part_span)))
        return -1;
    VMX_HIP(c, hipEventRecord(d.last, c->stream));
    d.used = true;
    return 0;
}

int combine_rows_fp(Context* c, const uint64_t* m, size_t rows, size_t cols, const Fp2* coeffs,
                    size_t combinations, Fp2* out) {
    const size_t col_threads = (cols + FP_COLS - 1) / FP_COLS;
    const size_t col_blocks = (col_threads + COMB_THREADS - 1) / COMB_THREADS;
    const size_t chunk = comb_chunk(rows, col_blocks);
    const size_t chunks = (rows + chunk - 1) / chunk;
    size_t per_chunk = 0, bytes = 0;
    if (!mul_ok(combinations, cols, &per_chunk) || !mul_ok(per_chunk * sizeof(Fp2), chunks, &bytes))
        return fail_msg(c, "combination partials overflow size_t");
    if (chunks > 65535) return fail_msg(c, "combination row count exceeds the supported maximum");
    if (chunks > 1 && ensure_ws(c, WS_PARTIALS, bytes)) return -1;
    Fp2* part = chunks > 1 ? ws<Fp2>(c, WS_PARTIALS) : out;  // one chunk: straight into out
    const dim3 grid(static_cast<unsigned>(col_blocks), static_cast<unsigned>(chunks));
    if (launch_comb_groups(combinations, [&](size_t c0, int kc) {
            if (kc == 2)
                hipLaunchKernelGGL(combine_fp_partial<2>, grid, dim3(COMB_THREADS), 0, c->stream, m, coeffs, part,
                                   rows, cols, c0, combinations, chunk);
            else
                hipLaunchKernelGGL(combine_fp_partial<1>, grid, dim3(COMB_THREADS), 0, c->stream, m, coeffs, part,
                                   rows, cols, c0, combinations, chunk);
            VMX_HIP(c, hipGetLastError());
            return 0;
        }))
        return -1;
    if (chunks == 1) return 0;
    hipLaunchKernelGGL(reduce_partials, dim3(static_cast<unsigned>((per_chunk + RED_Z - 1) / RED_Z)),
                       dim3(RED_Z * RED_LANES), 0, c->stream, static_cast<const Fp2*>(part), out, chunks, per_chunk,
                       static_cast<const uint32_t*>(nullptr), size_t{0}, size_t{1});
    VMX_HIP(c, hipGetLastError());
    return 0;
}

// ---- Fp2 powers [c^1..c^count] (reference fp2_powers_kernel runs serially) ---------------

// c^(2^k) for k < 64, computed on the host from the by-value base and passed
// as a kernel argument (1 KiB of the 4 KiB argument space).
struct Fp2Squares {
    Fp2 p[64];
};

// out[i] = c^(i+1) as the product of c^(2^k) over the set bits of i + 1.  The
// products go to two accumulators (even and odd k), so the dependent chain is
// half the bit count; no thread repeats another's squarings.
__global__ void fp2_powers_kernel(Fp2Squares sq, Fp2* out, size_t count, int bits) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride) {
        const uint64_t e = i + 1;
        Fp2 a{1, 0}, b{1, 0};
        for (int k = 0; k < bits; k += 2) {
            if ((e >> k) & 1) a = gl::fp2_mul(a, sq.p[k]);
            if (k + 1 < bits && ((e >> (k + 1)) & 1)) b = gl::fp2_mul(b, sq.p[k + 1]);
        }
        out[i] = gl::fp2_mul(a, b);
    }
}

// Below 2^18 powers: c^e = T0[e mod 64] T1[(e >> 6) mod 64] T2[e >> 12] with
// T_l[j] = c^(j 64^l), built on the host and passed by value (3 KiB of the
// 4 KiB argument space); two products per element, no divergence.
constexpr int POW_LEVELS = 3;
constexpr size_t POW_TABLE_LIMIT = size_t{1} << (6 * POW_LEVELS);
struct Fp2PowTable {
    Fp2 t[POW_LEVELS][64];
};

__global__ void fp2_powers_table_kernel(Fp2PowTable tb, Fp2* out, size_t count) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride) {
        const size_t e = i + 1;  // < 2^18
        out[i] = gl::fp2_mul(gl::fp2_mul(tb.t[0][e & 63], tb.t[1][(e >> 6) & 63]), tb.t[2][e >> 12]);
    }
}

int fp2_powers(Context* c, Fp2 base, Fp2* out, size_t count) {
    if (count < POW_TABLE_LIMIT) {
        Fp2PowTable tb;
        Fp2 step = base;  // c^(64^l)
        for (int l = 0; l < POW_LEVELS; ++l) {
            tb.t[l][0] = Fp2{1, 0};
            for (int j = 1; j < 64; ++j) tb.t[l][j] = gl::fp2_mul(tb.t[l][j - 1], step);
            step = gl::fp2_mul(tb.t[l][63], step);
        }
        hipLaunchKernelGGL(fp2_powers_table_kernel, dim3(grid_for(count, 256, 8192)), dim3(256), 0, c->stream, tb,
                           out, count);
        VMX_HIP(c, hipGetLastError());
        return 0;
    }
    Fp2Squares sq{};
    int bits = 0;
    while (bits < 64 && (count >> bits) != 0) ++bits;  // bit length of count >= bit length of i + 1
    sq.p[0] = base;
    for (int k = 1; k < bits; ++k) sq.p[k] = gl::fp2_mul(sq.p[k - 1], sq.p[k - 1]);
    hipLaunchKernelGGL(fp2_powers_kernel, dim3(grid_for(count, 256, 8192)), dim3(256), 0, c->stream, sq, out, count,
                       bits);
    VMX_HIP(c, hipGetLastError());
    return 0;
}

__global__ void fp2_add_kernel(Fp2* t, const Fp2* a, size_t n) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        t[i] = gl::fp2_add(t[i], a[i]);
}

int fp2_add_inplace(Context* c, Fp2* target, const Fp2* add, size_t n) {
    hipLaunchKernelGGL(fp2_add_kernel, dim3(grid_for(n, 256, 1 << 16)), dim3(256), 0, c->stream, target, add, n);
    VMX_HIP(c, hipGetLastError());
    return 0;
}

// ---- column gathers (reference .cu:3008-3024) ------------------------------------------------

template <typename T>
__global__ void gather_kernel(const T* m, const uint32_t* idx, T* out, size_t rows, size_t cols, size_t queries) {
    const size_t total = rows * queries;
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t z = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; z < total; z += stride) {
        const size_t q = z / rows, i = z - q * rows;
        const uint32_t col = idx[q];
        // Out-of-range indices read as zero instead of faulting; the Rust seam
        // validates indices before upload (rust/volta-accel/src/lib.rs:6773-6827).
        out[z] = col < cols ? m[i * cols + col] : T{};
    }
}

int gather_columns(Context* c, const uint64_t* m, const uint32_t* idx, uint64_t* out, size_t rows, size_t cols,
                   size_t queries, bool fp2) {
    const unsigned g = grid_for(rows * queries, 256, 1 << 16);
    if (fp2)
        hipLaunchKernelGGL(gather_kernel<Fp2>, dim3(g), dim3(256), 0, c->stream, reinterpret_cast<const Fp2*>(m), idx,
                           reinterpret_cast<Fp2*>(out), rows, cols, queries);
    else
        hipLaunchKernelGGL(gather_kernel<uint64_t>, dim3(g), dim3(256), 0, c->stream, m, idx, out, rows, cols,
                           queries);
    VMX_HIP(c, hipGetLastError());
    return 0;
}

// ---- ChaCha8 FpStream rows (reference .cu:1345-1372; one stream per row) ---------------------
//
// A row's stream is ChaCha8 in counter mode: block k (16 words, 8 u64 draws)
// depends only on (key, stream, k).  One wave fills one row: in each round
// lane t makes block k0 + t, keeps its draws below p, and an exclusive scan of
// the lanes' kept counts gives every kept draw its place in the row, exactly
// as the sequential sampler (next_u64 in block order, rejecting draws >= p)
// would place it.  Rounds continue until the row has `draws` kept values; a
// rejection (probability 2^-32 per draw) only shifts later places, and may
// take one more round.  Draw m goes to out[r * stride + m]; the lanes of a
// round write one contiguous run.
constexpr int CHACHA_WAVES = 4;  // rows per 256-thread workgroup

__global__ __launch_bounds__(64 * CHACHA_WAVES) void chacha8_rows_kernel(chacha8::Key key, uint64_t base_domain,
                                                                         size_t rows, size_t draws, size_t stride,
                                                                         size_t zero_from, uint64_t* out) {
    const int lane = threadIdx.x & 63;
    const size_t row_step = static_cast<size_t>(gridDim.x) * CHACHA_WAVES;
    for (size_t r = static_cast<size_t>(blockIdx.x) * CHACHA_WAVES + (threadIdx.x >> 6); r < rows; r += row_step) {
        uint64_t* o = out + r * stride;
        size_t done = 0;  // kept draws so far (uniform over the wave)
        for (uint64_t k0 = 0; done < draws; k0 += 64) {
            uint32_t w[16];
            chacha8::block(key, base_domain + r, k0 + static_cast<uint64_t>(lane), w);
            uint64_t v[8];
            int kept = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                v[i] = static_cast<uint64_t>(w[2 * i]) | (static_cast<uint64_t>(w[2 * i + 1]) << 32);
                kept += v[i] < chacha8::P ? 1 : 0;
            }
            int incl = kept;  // inclusive scan over the lanes
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const int y = __shfl_up(incl, d);
                if (lane >= d) incl += y;
            }
            size_t m = done + static_cast<size_t>(incl - kept);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (v[i] < chacha8::P) {
                    if (m < draws) o[m] = v[i];
                    ++m;
                }
            }
            done += static_cast<size_t>(__shfl(incl, 63));
        }
        for (size_t z = zero_from + lane; z < stride; z += 64) o[z] = 0;  // Fp2 rows' padding
    }
}

// Few long rows (an opening's mask rows: claims + 1 rows of tens of
// thousands of draws) would leave most of the GPU idle with one wave per row
// and serialise a hundred rounds.  Here a workgroup of CHACHA_WIDE waves fills
// one row: a round takes 64 CHACHA_WIDE consecutive blocks (wave w, lane t:
// block k0 + 64 w + t), each wave scans its lanes' kept counts, and the waves'
// totals (in LDS) place each wave's run after those of the waves before it --
// the same places as the one-wave kernel, in 1/CHACHA_WIDE of the rounds.
constexpr int CHACHA_WIDE = 16;

__global__ __launch_bounds__(64 * CHACHA_WIDE) void chacha8_rows_wide_kernel(chacha8::Key key, uint64_t base_domain,
                                                                             size_t rows, size_t draws, size_t stride,
                                                                             size_t zero_from, uint64_t* out) {
    __shared__ int wave_total[CHACHA_WIDE];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (size_t r = blockIdx.x; r < rows; r += gridDim.x) {
        uint64_t* o = out + r * stride;
        size_t done = 0;  // kept draws so far (uniform over the workgroup)
        for (uint64_t k0 = 0; done < draws; k0 += 64 * CHACHA_WIDE) {
            uint32_t w[16];
            chacha8::block(key, base_domain + r, k0 + static_cast<uint64_t>(64 * wave + lane), w);
            uint64_t v[8];
            int kept = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                v[i] = static_cast<uint64_t>(w[2 * i]) | (static_cast<uint64_t>(w[2 * i + 1]) << 32);
                kept += v[i] < chacha8::P ? 1 : 0;
            }
            int incl = kept;  // inclusive scan over the wave's lanes
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const int y = __shfl_up(incl, d);
                if (lane >= d) incl += y;
            }
            if (lane == 63) wave_total[wave] = incl;
            __syncthreads();
            int before = 0, total = 0;
#pragma unroll
            for (int q = 0; q < CHACHA_WIDE; ++q) {
                const int t = wave_total[q];
                before += q < wave ? t : 0;
                total += t;
            }
            size_t m = done + static_cast<size_t>(before + incl - kept);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (v[i] < chacha8::P) {
                    if (m < draws) o[m] = v[i];
                    ++m;
                }
            }
            done += static_cast<size_t>(total);
            __syncthreads();  // wave_total is rewritten by the next round
        }
        for (size_t z = zero_from + threadIdx.x; z < stride; z += 64 * CHACHA_WIDE) o[z] = 0;
    }
}

// Rows of `draws` kept values at `stride` words, zero from zero_from: one wave
// per row, or a workgroup per row for few long rows.
static int chacha8_rows(Context* c, const uint8_t seed[32], uint64_t base_domain, size_t rows, size_t draws,
                        size_t stride, size_t zero_from, uint64_t* out) {
    const chacha8::Key key = chacha8::key_from_seed(seed);
    if (rows <= 1024 && draws >= 8192)
        hipLaunchKernelGGL(chacha8_rows_wide_kernel, dim3(static_cast<unsigned>(rows)), dim3(64 * CHACHA_WIDE), 0,
                           c->stream, key, base_domain, rows, draws, stride, zero_from, out);
    else
        hipLaunchKernelGGL(chacha8_rows_kernel, dim3(grid_for(rows, CHACHA_WAVES, size_t{1} << 20)),
                           dim3(64 * CHACHA_WAVES), 0, c->stream, key, base_domain, rows, draws, stride, zero_from,
                           out);
    VMX_HIP(c, hipGetLastError());
    return 0;
}

int chacha8_fp_rows(Context* c, const uint8_t seed[32], uint64_t base_domain, size_t rows, size_t count,
                    uint64_t* out) {
    return chacha8_rows(c, seed, base_domain, rows, count, count, count, out);
}

// Fp2 rows: element j of a row is (draw 2j, draw 2j + 1); elements count ..
// padded - 1 are zero.
int chacha8_fp2_rows_padded(Context* c, const uint8_t seed[32], uint64_t base_domain, size_t rows, size_t count,
                            size_t padded, Fp2* out) {
    return chacha8_rows(c, seed, base_domain, rows, 2 * count, 2 * padded, 2 * count,
                        reinterpret_cast<uint64_t*>(out));
}

// ---- measurement probes ---------------------------------------------------------------------------

// Streaming copy with 16-byte accesses: the achievable-bandwidth yardstick.
__global__ __launch_bounds__(256) void copy_kernel(const uint4* src, uint4* dst, size_t n16) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += stride)
        dst[i] = src[i];
}

// The encode's traffic shape as a yardstick: every 4 bytes read become 64
// bytes written (1:16, as i16 messages at rate 1/4 become u64 codewords), with
// the encode's stores: 8 bytes per lane, 512 contiguous bytes per wave
// instruction, non-temporal.
__global__ __launch_bounds__(256) void expand_kernel(const uint32_t* src, uint64_t* dst, size_t n32) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n32; i += stride) {
        const uint64_t v = src[i];
        uint64_t* o = dst + (i / 64) * 512 + (i % 64);
#pragma unroll
        for (int k = 0; k < 8; ++k) __builtin_nontemporal_store(v + k, o + 64 * k);
    }
}

int probe_expand(Context* c, const void* src, void* dst, size_t src_bytes) {
    const size_t n32 = src_bytes / 4;
    hipLaunchKernelGGL(expand_kernel, dim3(grid_for(n32, 256 * 4, 256 * 64)), dim3(256), 0, c->stream,
                       static_cast<const uint32_t*>(src), static_cast<uint64_t*>(dst), n32);
    VMX_HIP(c, hipGetLastError());
    return 0;
}

int probe_copy(Context* c, const void* src, void* dst, size_t bytes) {
    const size_t n16 = bytes / 16;
    hipLaunchKernelGGL(copy_kernel, dim3(grid_for(n16, 256 * 8, 256 * 64)), dim3(256), 0, c->stream,
                       static_cast<const uint4*>(src), static_cast<uint4*>(dst), n16);
    VMX_HIP(c, hipGetLastError());
    return 0;
}

// The reference's Fp2 roofline probes (cuda/p7_goldilocks_roofline.cu:74-89).
__global__ void fp2_stream_kernel(const Fp2* a, const Fp2* b, Fp2* out, size_t n) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = gl::fp2_mul(a[i], b[i]);
}

__global__ void fp2_chain_kernel(const Fp2* a, const Fp2* b, Fp2* out, size_t n, int rounds) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        Fp2 x = a[i];
        const Fp2 y = b[i];
        for (int j = 0; j < rounds; ++j)
            x = gl::fp2_add(gl::fp2_mul(x, y), Fp2{static_cast<uint64_t>(j + 1), static_cast<uint64_t>(2 * j + 3)});
        out[i] = x;
    }
}

int probe_fp2_stream(Context* c, const Fp2* a, const Fp2* b, Fp2* out, size_t n) {
    hipLaunchKernelGGL(fp2_stream_kernel, dim3(grid_for(n, 256, 1 << 16)), dim3(256), 0, c->stream, a, b, out, n);
    VMX_HIP(c, hipGetLastError());
    return 0;
}

int probe_fp2_chain(Context* c, const Fp2* a, const Fp2* b, Fp2* out, size_t n, int rounds) {
    hipLaunchKernelGGL(fp2_chain_kernel, dim3(grid_for(n, 256, 1 << 16)), dim3(256), 0, c->stream, a, b, out, n,
                       rounds);
    VMX_HIP(c, hipGetLastError());
    return 0;
}

}  // namespace vmx

namespace vmx {

// ---- opening-path helpers -------------------------------------------------------------------

namespace {

__device__ __forceinline__ Fp2 fp2_one_minus(Fp2 p) { return Fp2{gl::sub(1, p.c0), gl::neg(p.c1)}; }
__device__ __forceinline__ Fp2 fp2_sub(Fp2 a, Fp2 b) { return Fp2{gl::sub(a.c0, b.c0), gl::sub(a.c1, b.c1)}; }

// out[r][x] = prod_k (bit k of x ? p[r][k] : 1 - p[r][k]) for x < 2^dims
// (reference eq_rows_expand, .cu:2860-2871).  Thread (r, hi) owns the 2^LOW
// consecutive x = hi 2^LOW + i: one product over the high bits, then the low
// bits expanded in registers from the highest down, v -> (v - v p, v p), which
// is the reference's expansion order; two products per output.
template <int LOW>
__global__ __launch_bounds__(256) void eq_rows_kernel(const Fp2* __restrict__ points, size_t rows, int dims,
                                                      Fp2* __restrict__ out) {
    const size_t per_row = size_t{1} << (dims - LOW);
    const size_t total = rows * per_row;
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t z = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; z < total; z += stride) {
        const size_t r = z / per_row, hi = z - r * per_row;
        const Fp2* p = points + r * dims;
        Fp2 v[1 << LOW];
        v[0] = Fp2{1, 0};
        for (int k = LOW; k < dims; ++k) {
            const Fp2 pk = p[k];
            v[0] = gl::fp2_mul(v[0], ((hi >> (k - LOW)) & 1) ? pk : fp2_one_minus(pk));
        }
#pragma unroll
        for (int k = LOW - 1; k >= 0; --k) {
            const Fp2 pk = p[k];
            const int cnt = 1 << (LOW - 1 - k);
#pragma unroll
            for (int i = cnt - 1; i >= 0; --i) {
                const Fp2 t = gl::fp2_mul(v[i], pk);
                const Fp2 s = fp2_sub(v[i], t);
                v[2 * i + 1] = t;
                v[2 * i] = s;
            }
        }
        Fp2* o = out + (r << dims) + (hi << LOW);
#pragma unroll
        for (int i = 0; i < (1 << LOW); ++i) o[i] = v[i];
    }
}

constexpr int DOT_THREADS = 1024;  // 16 waves per row: a claim's mask row is 2^13..2^17 long
constexpr int DOT_UNROLL = 4;      // products whose loads are in flight together

__device__ __forceinline__ Fp2 fp2_shfl_xor(Fp2 x, int m) {
    const uint64_t c0 = __shfl_xor(x.c0, m), c1 = __shfl_xor(x.c1, m);
    return Fp2{c0, c1};
}

// out[r] = sum_j a[r a_stride + j] b[r b_stride + j] (reference .cu:1374-1391):
// one workgroup per row, strided partial sums, a shuffle reduction inside each
// wave and one LDS step across the four waves.
__global__ __launch_bounds__(DOT_THREADS) void fp2_row_dots_kernel(const Fp2* __restrict__ a, size_t a_stride,
                                                                   const Fp2* __restrict__ b, size_t b_stride,
                                                                   Fp2* __restrict__ out, size_t rows, size_t len) {
    __shared__ Fp2 part[DOT_THREADS / 64];
    const int t = threadIdx.x;
    for (size_t row = blockIdx.x; row < rows; row += gridDim.x) {
        Fp2 acc{0, 0};
        const Fp2* ar = a + row * a_stride;
        const Fp2* br = b + row * b_stride;
        size_t j = t;
        for (; j + (DOT_UNROLL - 1) * DOT_THREADS < len; j += DOT_UNROLL * DOT_THREADS) {
            Fp2 x[DOT_UNROLL], y[DOT_UNROLL];
#pragma unroll
            for (int u = 0; u < DOT_UNROLL; ++u) {
                x[u] = ar[j + u * DOT_THREADS];
                y[u] = br[j + u * DOT_THREADS];
            }
#pragma unroll
            for (int u = 0; u < DOT_UNROLL; ++u) acc = gl::fp2_add(acc, gl::fp2_mul(x[u], y[u]));
        }
        for (; j < len; j += DOT_THREADS) acc = gl::fp2_add(acc, gl::fp2_mul(ar[j], br[j]));
#pragma unroll
        for (int m = 32; m > 0; m >>= 1) acc = gl::fp2_add(acc, fp2_shfl_xor(acc, m));
        if ((t & 63) == 0) part[t >> 6] = acc;
        __syncthreads();
        if (t == 0) {
            Fp2 s = part[0];
#pragma unroll
            for (int w = 1; w < DOT_THREADS / 64; ++w) s = gl::fp2_add(s, part[w]);
            out[row] = s;
        }
        __syncthreads();
    }
}

}  // namespace

int eq_rows(Context* c, const Fp2* points, size_t rows, size_t dims, Fp2* out) {
    const int d = static_cast<int>(dims);
    // Up to 16 outputs per thread, fewer when that would leave under 256
    // threads (a single block claim's 2^9 weights: 256 threads of two,
    // instead of 32 threads of sixteen running one serial wave).
    int low = d < 4 ? d : 4;
    while (low > 0 && (rows << (dims - low)) < 256) --low;
    const size_t threads = rows << (dims - low);
    const dim3 grid(grid_for(threads, 256, 1 << 16));
    switch (low) {
        case 0: hipLaunchKernelGGL(eq_rows_kernel<0>, grid, dim3(256), 0, c->stream, points, rows, d, out); break;
        case 1: hipLaunchKernelGGL(eq_rows_kernel<1>, grid, dim3(256), 0, c->stream, points, rows, d, out); break;
        case 2: hipLaunchKernelGGL(eq_rows_kernel<2>, grid, dim3(256), 0, c->stream, points, rows, d, out); break;
        case 3: hipLaunchKernelGGL(eq_rows_kernel<3>, grid, dim3(256), 0, c->stream, points, rows, d, out); break;
        default: hipLaunchKernelGGL(eq_rows_kernel<4>, grid, dim3(256), 0, c->stream, points, rows, d, out); break;
    }
    VMX_HIP(c, hipGetLastError());
    return 0;
}

int fp2_row_dots(Context* c, const Fp2* a, size_t a_stride, const Fp2* b, size_t b_stride, Fp2* out, size_t rows,
                 size_t len) {
    const unsigned blocks = static_cast<unsigned>(rows < 65535 ? rows : 65535);
    hipLaunchKernelGGL(fp2_row_dots_kernel, dim3(blocks), dim3(DOT_THREADS), 0, c->stream, a, a_stride, b, b_stride,
                       out, rows, len);
    VMX_HIP(c, hipGetLastError());
    return 0;
}

}  // namespace vmx
