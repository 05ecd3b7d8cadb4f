/*
 * volta_oracle.c -- CPU restatement of the reference's Ligero commit arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (see volta_oracle.h).  It exists to check the HIP
 * product path and to time a CPU baseline; nothing in the product links it.
 *
 * The reference implementation is Rust (rust/volta-field, rust/volta-pcs),
 * which cannot be built in this environment, so this file restates it in C.
 * Pins (tests/test_oracle.py):
 *   - field ops: differential against Python big-int arithmetic, the edge cases
 *     of rust/volta-field/src/lib.rs:309-320, 7 a non-residue (lib.rs:331-335);
 *   - NTT: root order (ntt.rs:78-87), naive DFT (ntt.rs:89-104), Horner
 *     evaluation (ntt.rs:106-121), and the reference-recorded checksums
 *     0xa87a560725f2d016 / 0xbe7b90425a4c7229 (benchmarks/results/
 *     p7-gpu-pcs-arithmetic[-quick]-2026-07-11-366ec4a.json);
 *   - combinations: checksums 0x0852323a5805ed2c / 0x856f9a96d8e01901 (same
 *     files) and a brute-force double loop;
 *   - Fp2 mul: checksums of p7-gpu-roofline[-quick]-2026-07-11-a43d105.json;
 *   - FpStream: the reference KAT (rust/volta-accel/src/lib.rs:7517-7528) and
 *     the published ChaCha8 keystream for the all-zero key.
 *   - inverse NTT: round trip and naive inverse DFT (no reference exists).
 */
#include "volta_oracle.h"

#include <omp.h>
#include <stdlib.h>
#include <string.h>

#define VO_P 0xFFFFFFFF00000001ULL
#define VO_EPS 0x00000000FFFFFFFFULL

typedef unsigned __int128 u128;

/* ------------------------------------------------------------------------ */
/* field                                                                    */
/* ------------------------------------------------------------------------ */

/* lib.rs:22-25: one conditional subtraction canonicalises any u64. */
uint64_t vo_fp_new(uint64_t x) { return x >= VO_P ? x - VO_P : x; }

/* lib.rs:32-40: negative values embed as p - |x|. */
uint64_t vo_fp_from_i64(int64_t x) {
    if (x >= 0) return vo_fp_new((uint64_t)x);
    uint64_t mag = (uint64_t)0 - (uint64_t)x; /* |x| without overflow at INT64_MIN */
    return VO_P - mag;
}

/* lib.rs:42-47: wrap-around carry is worth 2^64 = eps (mod p). */
uint64_t vo_fp_add(uint64_t a, uint64_t b) {
    uint64_t r = a + b;
    if (r < a) r += VO_EPS;
    if (r >= VO_P) r -= VO_P;
    return r;
}

/* lib.rs:49-53: a borrow is worth -2^64 = -eps. */
uint64_t vo_fp_sub(uint64_t a, uint64_t b) {
    uint64_t r = a - b;
    if (a < b) r -= VO_EPS;
    return r;
}

/* lib.rs:55-62 */
uint64_t vo_fp_neg(uint64_t a) { return a == 0 ? 0 : VO_P - a; }

/* lib.rs:89-103: x = lo + 2^64 hi, hi = hh*2^32 + hl, 2^64 = eps, 2^96 = -1,
 * so x = lo - hh + eps*hl (mod p). */
static inline uint64_t vo_reduce128(u128 x) {
    uint64_t lo = (uint64_t)x;
    uint64_t hi = (uint64_t)(x >> 64);
    uint64_t hh = hi >> 32;
    uint64_t hl = hi & VO_EPS;
    uint64_t t = lo - hh;
    if (lo < hh) t -= VO_EPS;
    uint64_t m = hl * VO_EPS;
    uint64_t r = t + m;
    if (r < t) r += VO_EPS;
    if (r >= VO_P) r -= VO_P;
    return r;
}

/* lib.rs:64-67 */
uint64_t vo_fp_mul(uint64_t a, uint64_t b) { return vo_reduce128((u128)a * b); }

/* lib.rs:69-80: square-and-multiply, LSB first. */
uint64_t vo_fp_pow(uint64_t a, uint64_t e) {
    uint64_t acc = 1;
    while (e) {
        if (e & 1) acc = vo_fp_mul(acc, a);
        a = vo_fp_mul(a, a);
        e >>= 1;
    }
    return acc;
}

/* lib.rs:83-86: Fermat inverse. */
uint64_t vo_fp_inv(uint64_t a) { return vo_fp_pow(a, VO_P - 2); }

/* lib.rs:163-166 */
vo_fp2 vo_fp2_add(vo_fp2 a, vo_fp2 b) {
    vo_fp2 r = {vo_fp_add(a.c0, b.c0), vo_fp_add(a.c1, b.c1)};
    return r;
}

/* lib.rs:173-177: (a0 + a1 phi)(b0 + b1 phi), phi^2 = 7. */
vo_fp2 vo_fp2_mul(vo_fp2 a, vo_fp2 b) {
    vo_fp2 r;
    r.c0 = vo_fp_add(vo_fp_mul(a.c0, b.c0), vo_fp_mul(7, vo_fp_mul(a.c1, b.c1)));
    r.c1 = vo_fp_add(vo_fp_mul(a.c0, b.c1), vo_fp_mul(a.c1, b.c0));
    return r;
}

/* lib.rs:181-184 */
vo_fp2 vo_fp2_mul_base(vo_fp2 a, uint64_t x) {
    vo_fp2 r = {vo_fp_mul(a.c0, x), vo_fp_mul(a.c1, x)};
    return r;
}

void vo_fp_mul_vec(const uint64_t* a, const uint64_t* b, uint64_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = vo_fp_mul(a[i], b[i]);
}
void vo_fp_add_vec(const uint64_t* a, const uint64_t* b, uint64_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = vo_fp_add(a[i], b[i]);
}
void vo_fp_sub_vec(const uint64_t* a, const uint64_t* b, uint64_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = vo_fp_sub(a[i], b[i]);
}

/* ------------------------------------------------------------------------ */
/* NTT                                                                      */
/* ------------------------------------------------------------------------ */

static int vo_log2(size_t n) {
    int b = 0;
    while (((size_t)1 << b) < n) ++b;
    return b;
}

/* ntt.rs:9-12: generator 7, 2-adicity 32. */
uint64_t vo_root_of_unity(uint32_t bits) {
    if (bits > 32) return 0;
    return vo_fp_pow(7, (VO_P - 1) >> bits);
}

/* ntt.rs:21-32: w^0 .. w^(n/2-1) by repeated multiplication. */
void vo_ntt_twiddles(size_t n, uint64_t* tw) {
    uint64_t w = vo_root_of_unity((uint32_t)vo_log2(n));
    uint64_t acc = 1;
    for (size_t i = 0; i < n / 2; ++i) {
        tw[i] = acc;
        acc = vo_fp_mul(acc, w);
    }
}

static size_t vo_bitrev(size_t x, int bits) {
    size_t r = 0;
    for (int i = 0; i < bits; ++i) {
        r = (r << 1) | (x & 1);
        x >>= 1;
    }
    return r;
}

/* ntt.rs:36-61: bit-reversal permutation, then radix-2 DIT stages with
 * twiddle stride n/len; output in natural order, out[j] = sum_i a_i w^ij. */
void vo_ntt_forward(uint64_t* a, size_t n, const uint64_t* tw) {
    int bits = vo_log2(n);
    for (size_t i = 0; i < n; ++i) {
        size_t j = vo_bitrev(i, bits);
        if (i < j) {
            uint64_t t = a[i];
            a[i] = a[j];
            a[j] = t;
        }
    }
    for (size_t len = 2; len <= n; len <<= 1) {
        size_t step = n / len, half = len / 2;
        for (size_t start = 0; start < n; start += len) {
            for (size_t k = 0; k < half; ++k) {
                uint64_t u = a[start + k];
                uint64_t v = vo_fp_mul(a[start + k + half], tw[k * step]);
                a[start + k] = vo_fp_add(u, v);
                a[start + k + half] = vo_fp_sub(u, v);
            }
        }
    }
}

void vo_ntt_encode_batch(const uint64_t* msgs, size_t rows, size_t msg_len, size_t n,
                         uint64_t* out, int threads) {
    uint64_t* tw = (uint64_t*)malloc((n / 2 + 1) * sizeof(uint64_t));
    vo_ntt_twiddles(n, tw);
#pragma omp parallel for schedule(static) num_threads(threads)
    for (size_t r = 0; r < rows; ++r) {
        uint64_t* row = out + r * n;
        memcpy(row, msgs + r * msg_len, msg_len * sizeof(uint64_t));
        memset(row + msg_len, 0, (n - msg_len) * sizeof(uint64_t));
        vo_ntt_forward(row, n, tw);
    }
    free(tw);
}

void vo_ntt_forward_batch(uint64_t* data, size_t rows, size_t n, int threads) {
    uint64_t* tw = (uint64_t*)malloc((n / 2 + 1) * sizeof(uint64_t));
    vo_ntt_twiddles(n, tw);
#pragma omp parallel for schedule(static) num_threads(threads)
    for (size_t r = 0; r < rows; ++r) vo_ntt_forward(data + r * n, n, tw);
    free(tw);
}

void vo_ntt_inverse_batch(uint64_t* data, size_t rows, size_t n, int threads) {
    uint64_t* tw = (uint64_t*)malloc((n / 2 + 1) * sizeof(uint64_t));
    uint64_t w_inv = vo_fp_inv(vo_root_of_unity((uint32_t)vo_log2(n)));
    uint64_t acc = 1;
    for (size_t i = 0; i < n / 2; ++i) {
        tw[i] = acc;
        acc = vo_fp_mul(acc, w_inv);
    }
    uint64_t n_inv = vo_fp_inv(vo_fp_new((uint64_t)n));
#pragma omp parallel for schedule(static) num_threads(threads)
    for (size_t r = 0; r < rows; ++r) {
        uint64_t* row = data + r * n;
        vo_ntt_forward(row, n, tw);
        for (size_t j = 0; j < n; ++j) row[j] = vo_fp_mul(row[j], n_inv);
    }
    free(tw);
}

/* ------------------------------------------------------------------------ */
/* PCS messages and combinations                                            */
/* ------------------------------------------------------------------------ */

static void vo_message_row(const int16_t* w, const uint64_t* pads, size_t r, size_t cols,
                           size_t pad, size_t code_len, uint64_t* out) {
    for (size_t j = 0; j < cols; ++j) out[j] = vo_fp_from_i64((int64_t)w[r * cols + j]);
    for (size_t j = 0; j < pad; ++j) out[cols + j] = pads[r * pad + j];
    for (size_t j = cols + pad; j < code_len; ++j) out[j] = 0;
}

void vo_pcs_messages(const int16_t* w, const uint64_t* pads, size_t rows, size_t cols,
                     size_t pad, size_t code_len, uint64_t* out, int threads) {
#pragma omp parallel for schedule(static) num_threads(threads)
    for (size_t r = 0; r < rows; ++r)
        vo_message_row(w, pads, r, cols, pad, code_len, out + r * code_len);
}

void vo_pcs_encode_i16(const int16_t* w, const uint64_t* pads, size_t rows, size_t cols,
                       size_t pad, size_t code_len, uint64_t* out, int threads) {
    uint64_t* tw = (uint64_t*)malloc((code_len / 2 + 1) * sizeof(uint64_t));
    vo_ntt_twiddles(code_len, tw);
#pragma omp parallel for schedule(static) num_threads(threads)
    for (size_t r = 0; r < rows; ++r) {
        uint64_t* row = out + r * code_len;
        vo_message_row(w, pads, r, cols, pad, code_len, row);
        vo_ntt_forward(row, code_len, tw);
    }
    free(tw);
}

/* combine_rows (ligero.rs:680-720) for any number of coefficient rows: the
 * data block is split into threads*4 column chunks, each task walks every
 * row once over its chunk and accumulates all combinations (the reference
 * fuses u_q and u_c the same way); the pad block (rows x pad) is summed
 * serially afterwards.  combine_row_range (ligero.rs:1114-1135) gives the
 * same sums: field addition is exact, so the order does not matter. */
void vo_pcs_combine_rows(const int16_t* w, const uint64_t* pads, const vo_fp2* coeffs,
                         size_t rows, size_t cols, size_t pad, size_t combinations,
                         vo_fp2* out, int threads) {
    const size_t msg_len = cols + pad;
    for (size_t k = 0; k < combinations * msg_len; ++k) out[k] = (vo_fp2){0, 0};
    const size_t n_chunks = (size_t)(threads > 0 ? threads : 1) * 4;
    const size_t chunk = (cols + n_chunks - 1) / n_chunks;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
    for (size_t ci = 0; ci < n_chunks; ++ci) {
        const size_t j0 = ci * chunk;
        if (j0 >= cols) continue;
        const size_t len = cols - j0 < chunk ? cols - j0 : chunk;
        for (size_t i = 0; i < rows; ++i) {
            const int16_t* row = w + i * cols + j0;
            for (size_t dj = 0; dj < len; ++dj) {
                const uint64_t x = vo_fp_from_i64((int64_t)row[dj]);
                for (size_t c = 0; c < combinations; ++c) {
                    vo_fp2* u = out + c * msg_len + j0 + dj;
                    *u = vo_fp2_add(*u, vo_fp2_mul_base(coeffs[c * rows + i], x));
                }
            }
        }
    }
    for (size_t i = 0; i < rows; ++i)
        for (size_t q = 0; q < pad; ++q) {
            const uint64_t x = pads[i * pad + q];
            for (size_t c = 0; c < combinations; ++c) {
                vo_fp2* u = out + c * msg_len + cols + q;
                *u = vo_fp2_add(*u, vo_fp2_mul_base(coeffs[c * rows + i], x));
            }
        }
}

void vo_combine_rows_fp(const uint64_t* msgs, const vo_fp2* coeffs, size_t rows, size_t cols,
                        size_t combinations, vo_fp2* out, int threads) {
#pragma omp parallel for schedule(static) num_threads(threads)
    for (size_t j = 0; j < cols; ++j) {
        for (size_t c = 0; c < combinations; ++c) {
            vo_fp2 acc = {0, 0};
            for (size_t i = 0; i < rows; ++i)
                acc = vo_fp2_add(acc, vo_fp2_mul_base(coeffs[c * rows + i], msgs[i * cols + j]));
            out[c * cols + j] = acc;
        }
    }
}

void vo_fp2_powers(vo_fp2 base, size_t count, vo_fp2* out) {
    vo_fp2 acc = {1, 0};
    for (size_t i = 0; i < count; ++i) {
        acc = vo_fp2_mul(acc, base);
        out[i] = acc;
    }
}

void vo_fp2_add_inplace(vo_fp2* target, const vo_fp2* add, size_t n) {
    for (size_t i = 0; i < n; ++i) target[i] = vo_fp2_add(target[i], add[i]);
}

void vo_gather_columns(const uint64_t* m, size_t rows, size_t cols, const uint32_t* idx,
                       size_t queries, uint64_t* out) {
    for (size_t q = 0; q < queries; ++q)
        for (size_t i = 0; i < rows; ++i) out[q * rows + i] = m[i * cols + idx[q]];
}

void vo_gather_fp2_columns(const vo_fp2* m, size_t rows, size_t cols, const uint32_t* idx,
                           size_t queries, vo_fp2* out) {
    for (size_t q = 0; q < queries; ++q)
        for (size_t i = 0; i < rows; ++i) out[q * rows + i] = m[i * cols + idx[q]];
}

/* Equality rows for the opening's claim and mask points
 * (volta_cuda_logup_eq_rows_device, cuda/volta_cuda_backend.cu:6884-6911 with
 * eq_rows_expand .cu:2860-2871; callers rust/volta-accel/src/lib.rs:3037-3053,
 * 6167-6205): out[r][x] = prod_k (bit k of x ? p[r][k] : 1 - p[r][k]) for
 * x < 2^dims, written here as the direct product. */
void vo_eq_rows(const vo_fp2* points, size_t rows, size_t dims, vo_fp2* out) {
    const size_t width = (size_t)1 << dims;
    const vo_fp2 one = {1, 0};
    for (size_t r = 0; r < rows; ++r)
        for (size_t x = 0; x < width; ++x) {
            vo_fp2 acc = one;
            for (size_t k = 0; k < dims; ++k) {
                const vo_fp2 p = points[r * dims + k];
                const vo_fp2 f = ((x >> k) & 1) ? p : (vo_fp2){vo_fp_sub(1, p.c0), vo_fp_sub(0, p.c1)};
                acc = vo_fp2_mul(acc, f);
            }
            out[r * width + x] = acc;
        }
}

/* out[r] = sum_j a[r a_stride + j] b[r b_stride + j] for j < len
 * (volta_cuda_fp2_row_dots_device, .cu:1374-1391, 4049-4103; caller
 * Backend::fp2_row_dots_device, rust/volta-accel/src/lib.rs:1873-1908). */
void vo_fp2_row_dots(const vo_fp2* a, size_t a_stride, const vo_fp2* b, size_t b_stride, size_t rows, size_t len,
                     vo_fp2* out) {
    for (size_t r = 0; r < rows; ++r) {
        vo_fp2 acc = {0, 0};
        for (size_t j = 0; j < len; ++j) acc = vo_fp2_add(acc, vo_fp2_mul(a[r * a_stride + j], b[r * b_stride + j]));
        out[r] = acc;
    }
}

/* ------------------------------------------------------------------------ */
/* ChaCha8 FpStream                                                          */
/* ------------------------------------------------------------------------ */

static inline uint32_t vo_rotl(uint32_t x, int n) { return (x << n) | (x >> (32 - n)); }

#define VO_QR(a, b, c, d)                 \
    do {                                  \
        a += b; d = vo_rotl(d ^ a, 16);   \
        c += d; b = vo_rotl(b ^ c, 12);   \
        a += b; d = vo_rotl(d ^ a, 8);    \
        c += d; b = vo_rotl(b ^ c, 7);    \
    } while (0)

/* Bernstein's ChaCha with 8 rounds and the original 64-bit block counter +
 * 64-bit nonce layout, which rand_chacha 0.3.1 uses with the nonce carrying
 * the stream id (the reference's device restatement, volta_chacha8_fp.cuh:68-108). */
void vo_chacha8_block(const uint32_t key[8], uint64_t stream, uint64_t counter, uint32_t out[16]) {
    uint32_t s[16];
    s[0] = 0x61707865u;
    s[1] = 0x3320646eu;
    s[2] = 0x79622d32u;
    s[3] = 0x6b206574u;
    for (int i = 0; i < 8; ++i) s[4 + i] = key[i];
    s[12] = (uint32_t)counter;
    s[13] = (uint32_t)(counter >> 32);
    s[14] = (uint32_t)stream;
    s[15] = (uint32_t)(stream >> 32);
    uint32_t x[16];
    memcpy(x, s, sizeof x);
    for (int dr = 0; dr < 4; ++dr) {
        VO_QR(x[0], x[4], x[8], x[12]);
        VO_QR(x[1], x[5], x[9], x[13]);
        VO_QR(x[2], x[6], x[10], x[14]);
        VO_QR(x[3], x[7], x[11], x[15]);
        VO_QR(x[0], x[5], x[10], x[15]);
        VO_QR(x[1], x[6], x[11], x[12]);
        VO_QR(x[2], x[7], x[8], x[13]);
        VO_QR(x[3], x[4], x[9], x[14]);
    }
    for (int i = 0; i < 16; ++i) out[i] = x[i] + s[i];
}

/* lib.rs:235-242: ChaCha8Rng::from_seed(seed) then set_stream(domain); the
 * seed bytes are the key as little-endian words. */
void vo_fpstream_init(vo_fpstream* s, const uint8_t seed[32], uint64_t domain) {
    for (int i = 0; i < 8; ++i)
        s->key[i] = (uint32_t)seed[4 * i] | ((uint32_t)seed[4 * i + 1] << 8) |
                    ((uint32_t)seed[4 * i + 2] << 16) | ((uint32_t)seed[4 * i + 3] << 24);
    s->stream = domain;
    s->counter = 0;
    s->index = 8;
    memset(s->words, 0, sizeof s->words);
}

/* rand_core BlockRng next_u64: two adjacent block words, low word first. */
uint64_t vo_fpstream_next_u64(vo_fpstream* s) {
    if (s->index >= 8) {
        vo_chacha8_block(s->key, s->stream, s->counter, s->words);
        s->counter += 1;
        s->index = 0;
    }
    uint64_t lo = s->words[2 * s->index];
    uint64_t hi = s->words[2 * s->index + 1];
    s->index += 1;
    return lo | (hi << 32);
}

/* lib.rs:245-253: rejection sampling, draws >= p are discarded. */
uint64_t vo_fpstream_next_fp(vo_fpstream* s) {
    for (;;) {
        uint64_t x = vo_fpstream_next_u64(s);
        if (x < VO_P) return x;
    }
}

/* lib.rs:255-258 */
vo_fp2 vo_fpstream_next_fp2(vo_fpstream* s) {
    vo_fp2 r;
    r.c0 = vo_fpstream_next_fp(s);
    r.c1 = vo_fpstream_next_fp(s);
    return r;
}

void vo_fp_rows(const uint8_t seed[32], uint64_t base_domain, size_t rows, size_t count,
                uint64_t* out, int threads) {
#pragma omp parallel for schedule(static) num_threads(threads)
    for (size_t r = 0; r < rows; ++r) {
        vo_fpstream s;
        vo_fpstream_init(&s, seed, base_domain + (uint64_t)r);
        for (size_t j = 0; j < count; ++j) out[r * count + j] = vo_fpstream_next_fp(&s);
    }
}

void vo_fp2_rows_padded(const uint8_t seed[32], uint64_t base_domain, size_t rows, size_t count,
                        size_t padded_count, vo_fp2* out, int threads) {
#pragma omp parallel for schedule(static) num_threads(threads)
    for (size_t r = 0; r < rows; ++r) {
        vo_fpstream s;
        vo_fpstream_init(&s, seed, base_domain + (uint64_t)r);
        for (size_t j = 0; j < count; ++j) out[r * padded_count + j] = vo_fpstream_next_fp2(&s);
        for (size_t j = count; j < padded_count; ++j) {
            out[r * padded_count + j].c0 = 0;
            out[r * padded_count + j].c1 = 0;
        }
    }
}

void vo_raw_u64(const uint8_t seed[32], uint64_t domain, size_t count, uint64_t* out) {
    vo_fpstream s;
    vo_fpstream_init(&s, seed, domain);
    for (size_t i = 0; i < count; ++i) out[i] = vo_fpstream_next_u64(&s);
}

/* ------------------------------------------------------------------------ */
/* checksums and spike kernels                                               */
/* ------------------------------------------------------------------------ */

uint64_t vo_fnv_u64(const uint64_t* v, size_t n, uint64_t h) {
    for (size_t i = 0; i < n; ++i) {
        h ^= v[i];
        h *= 0x00000100000001B3ULL;
    }
    return h;
}

void vo_fp2_mul_stream(const vo_fp2* a, const vo_fp2* b, vo_fp2* out, size_t n, int threads) {
#pragma omp parallel for schedule(static) num_threads(threads)
    for (size_t i = 0; i < n; ++i) out[i] = vo_fp2_mul(a[i], b[i]);
}

void vo_fp2_chain(const vo_fp2* a, const vo_fp2* b, vo_fp2* out, size_t n, int rounds,
                  int threads) {
#pragma omp parallel for schedule(static) num_threads(threads)
    for (size_t i = 0; i < n; ++i) {
        vo_fp2 x = a[i];
        for (int j = 0; j < rounds; ++j) {
            vo_fp2 bias = {(uint64_t)(j + 1), (uint64_t)(2 * j + 3)};
            x = vo_fp2_add(vo_fp2_mul(x, b[i]), bias);
        }
        out[i] = x;
    }
}
