/*
 * volta_oracle.h -- CPU restatement of the reference's Ligero commit arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP path: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * The product (libvolta_mi355x_backend.so) never links or calls it.
 *
 * Every function cites the reference file:line whose behaviour it restates
 * (paths relative to the okrame/volta-zk checkout).  Field elements are
 * canonical u64 in [0, p), p = 2^64 - 2^32 + 1; an Fp2 is two u64 (c0, c1),
 * the layout of the reference's #[repr(C)] Fp2Repr.
 */
#ifndef VOLTA_ORACLE_H
#define VOLTA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    uint64_t c0;
    uint64_t c1;
} vo_fp2;

/* ---- field (rust/volta-field/src/lib.rs) ------------------------------- */
uint64_t vo_fp_new(uint64_t x);                  /* lib.rs:22-25   */
uint64_t vo_fp_from_i64(int64_t x);              /* lib.rs:32-40   */
uint64_t vo_fp_add(uint64_t a, uint64_t b);      /* lib.rs:42-47   */
uint64_t vo_fp_sub(uint64_t a, uint64_t b);      /* lib.rs:49-53   */
uint64_t vo_fp_neg(uint64_t a);                  /* lib.rs:55-62   */
uint64_t vo_fp_mul(uint64_t a, uint64_t b);      /* lib.rs:64-67, 89-103 */
uint64_t vo_fp_pow(uint64_t a, uint64_t e);      /* lib.rs:69-80   */
uint64_t vo_fp_inv(uint64_t a);                  /* lib.rs:83-86   */
vo_fp2 vo_fp2_add(vo_fp2 a, vo_fp2 b);           /* lib.rs:163-166 */
vo_fp2 vo_fp2_mul(vo_fp2 a, vo_fp2 b);           /* lib.rs:173-177 */
vo_fp2 vo_fp2_mul_base(vo_fp2 a, uint64_t x);    /* lib.rs:181-184 */

/* element-wise batch forms, for differential tests */
void vo_fp_mul_vec(const uint64_t* a, const uint64_t* b, uint64_t* out, size_t n);
void vo_fp_add_vec(const uint64_t* a, const uint64_t* b, uint64_t* out, size_t n);
void vo_fp_sub_vec(const uint64_t* a, const uint64_t* b, uint64_t* out, size_t n);

/* ---- NTT (rust/volta-pcs/src/ntt.rs) ------------------------------------ */
uint64_t vo_root_of_unity(uint32_t bits);                          /* ntt.rs:9-12  */
void vo_ntt_twiddles(size_t n, uint64_t* tw);                      /* ntt.rs:21-32 */
void vo_ntt_forward(uint64_t* a, size_t n, const uint64_t* tw);    /* ntt.rs:36-61 */
/* Batched encode of compact rows (msg_len per row) into rows x n codewords:
 * NttPlan::encode per row (ntt.rs:63-70), OpenMP over rows like the
 * reference's rayon par_chunks_mut (ligero.rs:584-592). */
void vo_ntt_encode_batch(const uint64_t* msgs, size_t rows, size_t msg_len, size_t n,
                         uint64_t* out, int threads);
/* In-place batched forward NTT of rows x n (already zero-padded). */
void vo_ntt_forward_batch(uint64_t* data, size_t rows, size_t n, int threads);
/* Inverse NTT: a_i = n^-1 sum_j A_j w^-ij.  Absent from the reference; defined
 * as the forward transform with w^-1 followed by a scale by n^-1. */
void vo_ntt_inverse_batch(uint64_t* data, size_t rows, size_t n, int threads);

/* ---- PCS message rows and combinations (rust/volta-pcs/src/ligero.rs) -- */
/* msg = lift(w) || pads || 0 up to code_len (ligero.rs:584-592; .cu:2950-2958) */
void vo_pcs_messages(const int16_t* w, const uint64_t* pads, size_t rows, size_t cols,
                     size_t pad, size_t code_len, uint64_t* out, int threads);
/* commit_impl encode step: messages + NttPlan::forward per row (ligero.rs:584-592) */
void vo_pcs_encode_i16(const int16_t* w, const uint64_t* pads, size_t rows, size_t cols,
                       size_t pad, size_t code_len, uint64_t* out, int threads);
/* u[c][j] = sum_i coeffs[c*rows+i] * msg_i[j] over message rows lift(w)||pads,
 * with combine_rows' loop order (ligero.rs:680-720: column chunks, each walking
 * all rows once, all combinations fused; the pad block after); the sums equal
 * combine_row_range's (ligero.rs:1114-1135).  Coefficient layout lib.rs:6522-6569. */
void vo_pcs_combine_rows(const int16_t* w, const uint64_t* pads, const vo_fp2* coeffs,
                         size_t rows, size_t cols, size_t pad, size_t combinations,
                         vo_fp2* out, int threads);
/* The same combination over u64 (Fp) message rows, as in the reference's own
 * arithmetic benchmark (cuda/p7_pcs_arithmetic.cu:275-288). */
void vo_combine_rows_fp(const uint64_t* msgs, const vo_fp2* coeffs, size_t rows, size_t cols,
                        size_t combinations, vo_fp2* out, int threads);
/* [c^1 .. c^count] (ligero.rs:772-778, 1630-1636; .cu:1394-1401) */
void vo_fp2_powers(vo_fp2 base, size_t count, vo_fp2* out);
/* target[i] += add[i] (.cu:2960-2963) */
void vo_fp2_add_inplace(vo_fp2* target, const vo_fp2* add, size_t n);
/* out[q*rows + i] = M[i*cols + idx[q]] (.cu:3008-3015) */
void vo_gather_columns(const uint64_t* m, size_t rows, size_t cols, const uint32_t* idx,
                       size_t queries, uint64_t* out);
void vo_gather_fp2_columns(const vo_fp2* m, size_t rows, size_t cols, const uint32_t* idx,
                           size_t queries, vo_fp2* out);

/* ---- FpStream = rand_chacha 0.3.1 ChaCha8Rng (lib.rs:224-258) ----------- */
typedef struct {
    uint32_t key[8];
    uint64_t stream;
    uint64_t counter;
    uint32_t index; /* next u64 index within the 16-word block, 8 = empty */
    uint32_t words[16];
} vo_fpstream;

void vo_chacha8_block(const uint32_t key[8], uint64_t stream, uint64_t counter, uint32_t out[16]);
void vo_fpstream_init(vo_fpstream* s, const uint8_t seed[32], uint64_t domain); /* lib.rs:235-242 */
uint64_t vo_fpstream_next_u64(vo_fpstream* s);
uint64_t vo_fpstream_next_fp(vo_fpstream* s);                                   /* lib.rs:245-253 */
vo_fp2 vo_fpstream_next_fp2(vo_fpstream* s);                                    /* lib.rs:255-258 */
/* Row r: FpStream::domain_separated(seed, base_domain + r), count draws
 * (chacha8_prover_secret_fp_rows_device, .cu:1345-1355, 3991-4047). */
void vo_fp_rows(const uint8_t seed[32], uint64_t base_domain, size_t rows, size_t count,
                uint64_t* out, int threads);
void vo_fp2_rows_padded(const uint8_t seed[32], uint64_t base_domain, size_t rows, size_t count,
                        size_t padded_count, vo_fp2* out, int threads);
void vo_raw_u64(const uint8_t seed[32], uint64_t domain, size_t count, uint64_t* out);

/* ---- checksums and spike kernels (cuda/p7_*.cu) ------------------------- */
/* FNV-style fold over u64 words (p7_pcs_arithmetic.cu:160-176) */
uint64_t vo_fnv_u64(const uint64_t* v, size_t n, uint64_t h);
/* out = a*b elementwise (p7_goldilocks_roofline.cu:74-77) */
void vo_fp2_mul_stream(const vo_fp2* a, const vo_fp2* b, vo_fp2* out, size_t n, int threads);
/* x = a; repeat R: x = x*b + (j+1, 2j+3) (p7_goldilocks_roofline.cu:79-89) */
void vo_fp2_chain(const vo_fp2* a, const vo_fp2* b, vo_fp2* out, size_t n, int rounds,
                  int threads);

/* ---- opening-path helpers ------------------------------------------------ */
/* out[r][x] = prod_k (bit k of x ? p[r][k] : 1 - p[r][k]), x < 2^dims
 * (cuda/volta_cuda_backend.cu:2860-2871, 6884-6911) */
void vo_eq_rows(const vo_fp2* points, size_t rows, size_t dims, vo_fp2* out);
/* out[r] = sum_j a[r a_stride + j] b[r b_stride + j] (.cu:1374-1391) */
void vo_fp2_row_dots(const vo_fp2* a, size_t a_stride, const vo_fp2* b, size_t b_stride, size_t rows,
                     size_t len, vo_fp2* out);

/* ---- BLAKE3 column leaves and Merkle tree (volta_oracle_blake3.c) -------
 * blake3 1.8.5 (rust/Cargo.lock:51-53) restated from the BLAKE3 specification;
 * merkle.rs:9-51, ligero.rs:595-621. Hashes are 32 bytes. */
void vo_blake3(const uint8_t* in, size_t len, uint8_t out[32]);               /* blake3::hash */
void vo_hash_fp_columns(const uint64_t* m, size_t rows, size_t cols, uint8_t* leaves, int threads);
void vo_hash_fp2_columns(const vo_fp2* m, size_t rows, size_t cols, uint8_t* leaves, int threads);
void vo_merkle_tree(const uint8_t* leaves, size_t n, uint8_t* tree);         /* merkle.rs:27-37 */
void vo_merkle_paths(const uint8_t* tree, size_t leaves, const uint32_t* idx, size_t queries,
                     uint8_t* paths);                                          /* merkle.rs:43-51 */
void vo_merkle_bench_matrix(size_t rows, size_t cols, uint64_t* m, int threads); /* p7_blake3_merkle.cu:243 */
/* commit_impl (ligero.rs:543-624) composed: pads -> messages -> per-row NTT ->
 * column leaves -> Merkle root.  encoded/pads may be NULL. */
int vo_commit_root(const int16_t* w, size_t rows, size_t cols, size_t pad, size_t code_len,
                   const uint8_t seed[32], uint8_t root[32], uint64_t* encoded, uint64_t* pads,
                   int threads);

/* ---- X4 extension-field transforms (volta_oracle_x4.c) -------------------
 * rust/volta-pcs/src/x4/ntt.rs; cuda/volta_x4b.cuh. */
vo_fp2 vo_fp2_pow(vo_fp2 base, uint64_t e);                                   /* ntt.rs:15-26 */
vo_fp2 vo_fp2_inv(vo_fp2 a);                                                   /* volta_x4b.cuh:107-115 */
vo_fp2 vo_x4_root_of_unity(uint32_t bits);                                     /* ntt.rs:28-57 */
void vo_x4_ntt(const vo_fp2* coeffs, size_t len, size_t n, vo_fp2* out);      /* ntt.rs:66-122 */
void vo_x4_fold_codeword(const vo_fp2* v, size_t n, vo_fp2 challenge, vo_fp2* out); /* ntt.rs:238-256 */
void vo_x4_fold_coefficients(const vo_fp2* c, size_t n, vo_fp2 challenge, vo_fp2* out); /* ntt.rs:230-235 */
void vo_fp2_mobius(vo_fp2* v, size_t n, int inverse);                          /* ntt.rs:147-188 */
vo_fp2 vo_mle_eval_coefficients(const vo_fp2* c, size_t n, const vo_fp2* point, size_t dims); /* ntt.rs:190-207 */
vo_fp2 vo_mle_eval_table(const vo_fp2* t, size_t n, const vo_fp2* point, size_t dims);        /* ntt.rs:209-228 */

#ifdef __cplusplus
}
#endif

#endif
