// kernels.hpp -- host-side launchers for the device kernels.  All launch on
// the context stream and return 0 or a context error; the callers in
// abi_pcs.cpp do geometry validation and stats accounting.
#pragma once

#include <stdint.h>

#include <cstddef>

#include "context.hpp"
#include "gl64.hpp"

namespace vmx {

int zero_bytes(Context* c, void* dst, size_t bytes);

// rows x n forward (or inverse, n^-1 scaled) NTT of u64 rows: input row r is
// in[r*in_stride .. +msg_len), zero beyond; output rows are n wide.  t is
// ensure_twiddles(n)'s set; the inverse needs t->inv unless t->reg is present
// (the pass engine, n >= 2^13).
int ntt_fp_rows(Context* c, const uint64_t* in, size_t in_stride, size_t msg_len, size_t rows, size_t n,
                uint64_t* out, TwiddleSet* t, bool inverse);
// Componentwise NTT of rows x n Fp2 (u64 pairs) with base-field twiddles.
int ntt_fp2_rows(Context* c, const uint64_t* in, size_t rows, size_t n, uint64_t* out, const TwiddleSet* t);
// Fused PCS encode: messages lift(w) || pads || 0 transformed without
// materialising the message rows.
int ntt_msg_i16_rows(Context* c, const int16_t* w, const uint64_t* pads, size_t rows, size_t cols, size_t pad,
                     size_t n, uint64_t* out, TwiddleSet* t);
// Fast path for the Ligero shapes (i16 messages with rate <= 1/2 and
// n in [2^11, 2^14]); returns 1 when the shape is not covered.
// Forward NTT of rows of n = 2^15 in one pass (ntt15.hip): u64 rows as for
// ntt13r_u64_rows (len <= n), or message rows lift(w) || pads || 0 with
// cols = 2^12 or 2^13 and pad <= 1024.  Returns 1 (nothing done) for other
// shapes, 0 on success, -1 on error.
int ntt15_u64_rows(Context* c, const uint64_t* in, size_t stride, size_t len, size_t rows, size_t n, uint64_t* out,
                   TwiddleSet* t);
int ntt15_msg_rows(Context* c, const int16_t* w, const uint64_t* pads, size_t cols, size_t pad, size_t rows,
                   size_t n, uint64_t* out, TwiddleSet* t);
// Forward NTT of rows of n = 2^13 (ntt13r) or 2^14 (ntt14r) canonical u64 in
// one pass (ntt_rr.hip): row r is in[r * stride .. r * stride + len), zero
// beyond len (len <= n).  Returns 1 (nothing done) for other sizes, 0 on
// success, -1 on error.
int ntt13r_u64_rows(Context* c, const uint64_t* in, size_t stride, size_t len, size_t rows, size_t n, uint64_t* out,
                    TwiddleSet* t);
int ntt14r_u64_rows(Context* c, const uint64_t* in, size_t stride, size_t len, size_t rows, size_t n, uint64_t* out,
                    TwiddleSet* t);
// The n = 2^13 tables of ntt13r inside the encode's device table (built on
// first use; null on error), and their builder.
const uint64_t* enc13_rr_table(Context* c, TwiddleSet* t);
int build_rr13_table(Context* c, const uint64_t* fwd, uint64_t* tab);
int encode_i16_fast(Context* c, const int16_t* w, size_t rows, size_t cols, size_t n, uint64_t* out,
                    TwiddleSet* t);

int pcs_messages(Context* c, const int16_t* w, const uint64_t* pads, size_t rows, size_t cols, size_t pad,
                 size_t code_len, uint64_t* out);
// out[comb][j], j < cols+pad, over message rows lift(w) || pads.
int pcs_combine_rows(Context* c, const int16_t* w, const uint64_t* pads, const gl::Fp2* coeffs, size_t rows,
                     size_t cols, size_t pad, size_t combinations, gl::Fp2* out);
// The same combination over dense u64 (Fp) rows.
// The same combination with its partials and coefficient sums in a fixed
// device array of COMBINE_SCRATCH_BYTES (no allocation), with larger row
// chunks when the usual ones need more; fails with a clear error when even
// chunks of 2^16 rows need more.  combine_scratch_attach resolves the
// array's address on the context's device (called by volta_cuda_create).
constexpr size_t COMBINE_SCRATCH_BYTES = size_t{16} << 20;
int pcs_combine_rows_noalloc(Context* c, const int16_t* w, const uint64_t* pads, const gl::Fp2* coeffs, size_t rows,
                             size_t cols, size_t pad, size_t combinations, gl::Fp2* out);
int combine_scratch_attach(Context* c);
int combine_rows_fp(Context* c, const uint64_t* m, size_t rows, size_t cols, const gl::Fp2* coeffs,
                    size_t combinations, gl::Fp2* out);
int fp2_powers(Context* c, gl::Fp2 base, gl::Fp2* out, size_t count);
int fp2_add_inplace(Context* c, gl::Fp2* target, const gl::Fp2* add, size_t n);
int gather_columns(Context* c, const uint64_t* m, const uint32_t* idx, uint64_t* out, size_t rows,
                   size_t cols, size_t queries, bool fp2);
int chacha8_fp_rows(Context* c, const uint8_t seed[32], uint64_t base_domain, size_t rows, size_t count,
                    uint64_t* out);
int chacha8_fp2_rows_padded(Context* c, const uint8_t seed[32], uint64_t base_domain, size_t rows,
                            size_t count, size_t padded, gl::Fp2* out);

// Opening-path helpers: equality rows (rows x 2^dims, LSB-first) and strided
// Fp2 row dot products.
int eq_rows(Context* c, const gl::Fp2* points, size_t rows, size_t dims, gl::Fp2* out);
int fp2_row_dots(Context* c, const gl::Fp2* a, size_t a_stride, const gl::Fp2* b, size_t b_stride, gl::Fp2* out,
                 size_t rows, size_t len);

// BLAKE3 column leaves of a rows x cols Fp (fp2 = false) or Fp2 matrix into
// leaves[cols][8 words]; the Merkle levels above cols leaves stored after
// them (tree = leaves, then each level, root last); sibling paths.
int merkle_column_leaves(Context* c, const uint64_t* m, size_t rows, size_t cols, bool fp2, uint32_t* leaves);
int merkle_tree_levels(Context* c, uint32_t* tree, size_t leaves);
int merkle_paths(Context* c, const uint32_t* tree, size_t leaves, const uint32_t* idx, size_t queries,
                 uint32_t* paths);

// Batched NTTs of 2^13 .. 2^33 points as passes of register four-steps
// (ntt_reg.hip).  rows transforms of n = 2^nb elements of `planes` u64 (1: Fp,
// 2: Fp2); input row r starts at in + r in_stride planes and holds len
// elements (zero beyond), output rows are contiguous.  Roots are the X4 roots
// (the base field's up to 2^31).  inverse: a_i = n^-1 sum_j A_j w^-ij (n <= 2^31).
struct RegTables {
    const uint64_t* inner = nullptr;  // w_4096^j, j < 2048
    const uint64_t* split = nullptr;  // two-level table of b_min(nb,32)
    int split_h = 0;
};
int reg_ntt(Context* c, const RegTables& tb, const uint64_t* in, uint64_t in_stride, uint64_t len, uint64_t* out,
            uint64_t rows, int nb, int planes, bool inverse);
// The same forward transform of Ligero message rows lift(w) || pads || 0
// (cols i16 weights and pad u64 pads per row), without materialising them.
int reg_ntt_msg_i16(Context* c, const RegTables& tb, const int16_t* w, const uint64_t* pads, uint64_t cols,
                    uint64_t pad, uint64_t* out, uint64_t rows, int nb);

// X4 extension-field transforms (x4.hip).  Tables for transforms and folds of
// 2^nb points, nb in [1, 33]; uploaded once per size (adds to *h2d), so call
// before the primitive's timing begins.
struct X4Tables {
    const uint64_t* inner = nullptr;  // w_4096^j, j < 2048
    const uint64_t* split = nullptr;  // two-level table of b_min(nb,32)
    int split_h = 0;
    int nb = 0;
};
int x4_tables(Context* c, int nb, uint64_t* h2d, X4Tables* out);
// 2^nb-point X4 Fp2 NTT of the len coefficients at in (zero beyond len) into
// out (2^nb elements, natural order; must not overlap in).
int x4_ntt(Context* c, const X4Tables& tb, const gl::Fp2* in, uint64_t len, gl::Fp2* out);
// Codeword fold of a 2^nb codeword: out[j] for absolute index j0 + j, j < count,
// from pos[j] = v[j0 + j] and neg[j] = v[j0 + j + 2^(nb-1)].
int x4_fold(Context* c, const X4Tables& tb, const gl::Fp2* pos, const gl::Fp2* neg, gl::Fp2* out, uint64_t j0,
            uint64_t count, gl::Fp2 ch);
// In-place Moebius transform of n = 2^k values (inverse: upper += lower).
int fp2_mobius(Context* c, gl::Fp2* values, uint64_t n, bool inverse);

// Measurement probes.
int probe_copy(Context* c, const void* src, void* dst, size_t bytes);
int probe_expand(Context* c, const void* src, void* dst, size_t src_bytes);
int probe_fp2_stream(Context* c, const gl::Fp2* a, const gl::Fp2* b, gl::Fp2* out, size_t n);
int probe_fp2_chain(Context* c, const gl::Fp2* a, const gl::Fp2* b, gl::Fp2* out, size_t n, int rounds);

}  // namespace vmx
