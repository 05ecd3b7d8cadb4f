/*
 * volta_oracle_x4.c -- CPU restatement of the reference's X4 extension-field
 * transforms: the order-2^33 Fp2 root, the Fp2 NTT, codeword folding and the
 * Boolean-hypercube Moebius transform.
 *
 * TEST INFRASTRUCTURE ONLY (see volta_oracle.h): the checker for the HIP path.
 *
 * Every transform is written the way the reference writes it (radix-2 DIT
 * with a full Fp2 twiddle table, one running inverse-x per fold symbol), not
 * the way the HIP path computes it, so a shortcut taken on the device (real
 * twiddles, other factorisations) is checked against the plain definition.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "volta_oracle.h"

#define VO_P 0xFFFFFFFF00000001ull

static vo_fp2 fp2_sub(vo_fp2 a, vo_fp2 b) {
    vo_fp2 r = {vo_fp_sub(a.c0, b.c0), vo_fp_sub(a.c1, b.c1)};
    return r;
}

static int fp2_eq(vo_fp2 a, vo_fp2 b) { return a.c0 == b.c0 && a.c1 == b.c1; }

/* base^e for a 128-bit exponent (rust/volta-pcs/src/x4/ntt.rs:15-26). */
static vo_fp2 fp2_pow128(vo_fp2 base, unsigned __int128 e) {
    vo_fp2 r = {1, 0};
    while (e) {
        if (e & 1) r = vo_fp2_mul(r, base);
        base = vo_fp2_mul(base, base);
        e >>= 1;
    }
    return r;
}

vo_fp2 vo_fp2_pow(vo_fp2 base, uint64_t e) { return fp2_pow128(base, e); }

/* (c0 - c1 phi) / (c0^2 - 7 c1^2) (cuda/volta_x4b.cuh:107-115). */
vo_fp2 vo_fp2_inv(vo_fp2 a) {
    const uint64_t d = vo_fp_sub(vo_fp_mul(a.c0, a.c0), vo_fp_mul(7, vo_fp_mul(a.c1, a.c1)));
    const uint64_t di = vo_fp_inv(d);
    vo_fp2 r = {vo_fp_mul(a.c0, di), vo_fp_mul(vo_fp_neg(a.c1), di)};
    return r;
}

/* The primitive 2^33-th root: the first candidate (c0, 1), c0 = 0, 1, ..., whose
 * power (p^2 - 1) >> 33 has exact order 2^33 (x4/ntt.rs:28-47).  Found once and
 * cached; the search ends at c0 = 0. */
static vo_fp2 primitive_root_2_33(void) {
    static int done = 0;
    static vo_fp2 root;
    if (done) return root;
    const unsigned __int128 order = (unsigned __int128)VO_P * VO_P - 1;
    const unsigned __int128 cofactor = order >> 33;
    const vo_fp2 one = {1, 0};
    for (uint64_t c0 = 0;; ++c0) {
        const vo_fp2 cand = {c0, 1};
        const vo_fp2 r = fp2_pow128(cand, cofactor);
        if (fp2_eq(fp2_pow128(r, (unsigned __int128)1 << 33), one) &&
            !fp2_eq(fp2_pow128(r, (unsigned __int128)1 << 32), one)) {
            root = r;
            done = 1;
            return root;
        }
    }
}

/* root^(2^(33 - bits)), or 1 for bits = 0; bits <= 33 (x4/ntt.rs:49-57). */
vo_fp2 vo_x4_root_of_unity(uint32_t bits) {
    const vo_fp2 one = {1, 0};
    if (bits == 0 || bits > 33) return one;
    return fp2_pow128(primitive_root_2_33(), (unsigned __int128)1 << (33 - bits));
}

/* Fp2NttPlan::encode then forward (x4/ntt.rs:66-122): zero-pad the
 * coefficients to n, bit-reverse, radix-2 DIT with the table root^0..root^(n/2-1)
 * indexed offset * (n / len).  n >= 2 a power of two <= 2^33, len <= n. */
void vo_x4_ntt(const vo_fp2* coeffs, size_t len, size_t n, vo_fp2* out) {
    uint32_t bits = 0;
    while (((size_t)1 << bits) < n) ++bits;
    const vo_fp2 root = vo_x4_root_of_unity(bits);
    vo_fp2* tw = (vo_fp2*)malloc(sizeof(vo_fp2) * (n / 2));
    vo_fp2 v = {1, 0};
    for (size_t i = 0; i < n / 2; ++i) {
        tw[i] = v;
        v = vo_fp2_mul(v, root);
    }
    memset(out, 0, sizeof(vo_fp2) * n);
    memcpy(out, coeffs, sizeof(vo_fp2) * len);
    for (size_t i = 0; i < n; ++i) {
        size_t r = 0;
        for (uint32_t b = 0; b < bits; ++b) r |= ((i >> b) & 1) << (bits - 1 - b);
        if (i < r) {
            const vo_fp2 t = out[i];
            out[i] = out[r];
            out[r] = t;
        }
    }
    for (size_t l = 2; l <= n; l *= 2) {
        const size_t step = n / l;
        for (size_t start = 0; start < n; start += l)
            for (size_t k = 0; k < l / 2; ++k) {
                const vo_fp2 a = out[start + k];
                const vo_fp2 b = vo_fp2_mul(out[start + k + l / 2], tw[k * step]);
                out[start + k] = vo_fp2_add(a, b);
                out[start + k + l / 2] = fp2_sub(a, b);
            }
    }
    free(tw);
}

/* fold_codeword (x4/ntt.rs:238-256; the device form direct_fold_symbol,
 * cuda/volta_x4b.cuh:194-201): with half = n/2 and x = w^j,
 * out[j] = (v[j] + v[j+half])/2 + challenge (v[j] - v[j+half])/2 x^-1. */
void vo_x4_fold_codeword(const vo_fp2* v, size_t n, vo_fp2 challenge, vo_fp2* out) {
    uint32_t bits = 0;
    while (((size_t)1 << bits) < n) ++bits;
    const size_t half = n / 2;
    const vo_fp2 w_inv = vo_fp2_inv(vo_x4_root_of_unity(bits));
    const vo_fp2 inv_two = {vo_fp_inv(2), 0};
    vo_fp2 inv_x = {1, 0};
    for (size_t j = 0; j < half; ++j) {
        const vo_fp2 pos = v[j], neg = v[j + half];
        const vo_fp2 even = vo_fp2_mul(vo_fp2_add(pos, neg), inv_two);
        const vo_fp2 odd = vo_fp2_mul(vo_fp2_mul(fp2_sub(pos, neg), inv_two), inv_x);
        out[j] = vo_fp2_add(even, vo_fp2_mul(challenge, odd));
        inv_x = vo_fp2_mul(inv_x, w_inv);
    }
}

/* fold_coefficients: out[j] = c[2j] + challenge c[2j+1] (x4/ntt.rs:230-235). */
void vo_x4_fold_coefficients(const vo_fp2* c, size_t n, vo_fp2 challenge, vo_fp2* out) {
    for (size_t j = 0; j < n / 2; ++j) out[j] = vo_fp2_add(c[2 * j], vo_fp2_mul(challenge, c[2 * j + 1]));
}

/* Moebius transform over the Boolean hypercube, LSB-first variables: for each
 * bit, upper = upper - lower (evaluations -> monomial coefficients,
 * x4/ntt.rs:147-166) or upper = upper + lower (the inverse, x4/ntt.rs:172-188;
 * the device entry fp2_mobius_inverse_inplace_device, .cu:2965-2972, 7114-7130). */
void vo_fp2_mobius(vo_fp2* v, size_t n, int inverse) {
    for (size_t mask = 1; mask < n; mask <<= 1)
        for (size_t base = 0; base < n; base += 2 * mask)
            for (size_t k = 0; k < mask; ++k) {
                vo_fp2* up = &v[base + mask + k];
                *up = inverse ? vo_fp2_add(*up, v[base + k]) : fp2_sub(*up, v[base + k]);
            }
}

/* evaluate_multilinear_coefficients (x4/ntt.rs:190-207): fold the coefficient
 * table by c[2i] + x c[2i+1], one point coordinate at a time. */
vo_fp2 vo_mle_eval_coefficients(const vo_fp2* c, size_t n, const vo_fp2* point, size_t dims) {
    vo_fp2* f = (vo_fp2*)malloc(sizeof(vo_fp2) * n);
    memcpy(f, c, sizeof(vo_fp2) * n);
    size_t len = n;
    for (size_t d = 0; d < dims; ++d) {
        for (size_t i = 0; i < len / 2; ++i) f[i] = vo_fp2_add(f[2 * i], vo_fp2_mul(point[d], f[2 * i + 1]));
        len /= 2;
    }
    const vo_fp2 r = f[0];
    free(f);
    return r;
}

/* evaluate_multilinear_table (x4/ntt.rs:209-228): l + x (r - l). */
vo_fp2 vo_mle_eval_table(const vo_fp2* t, size_t n, const vo_fp2* point, size_t dims) {
    vo_fp2* f = (vo_fp2*)malloc(sizeof(vo_fp2) * n);
    memcpy(f, t, sizeof(vo_fp2) * n);
    size_t len = n;
    for (size_t d = 0; d < dims; ++d) {
        for (size_t i = 0; i < len / 2; ++i) {
            const vo_fp2 l = f[2 * i], r = f[2 * i + 1];
            f[i] = vo_fp2_add(l, vo_fp2_mul(point[d], fp2_sub(r, l)));
        }
        len /= 2;
    }
    const vo_fp2 r = f[0];
    free(f);
    return r;
}
