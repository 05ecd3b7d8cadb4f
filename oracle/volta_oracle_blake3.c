/*
 * volta_oracle_blake3.c -- CPU restatement of the column commitment that
 * closes the reference's Ligero commit: BLAKE3 leaves over the encoded
 * matrix's columns and a binary BLAKE3 Merkle tree over the leaves.
 *
 * TEST INFRASTRUCTURE ONLY (see volta_oracle.h).
 *
 * The hash is the reference's third-party dependency blake3 1.8.5
 * (rust/Cargo.lock:51-53), called as blake3::hash (rust/volta-pcs/src/merkle.rs:9-18).
 * It is restated here from the published BLAKE3 specification (O'Connor,
 * Aumasson, Neves, Wilcox-O'Hearn, 2020):
 * - the compression function: the SHA-256 IV, 7 rounds of the ChaCha-style G
 *   with rotations 16/12/8/7, and the fixed message permutation;
 * - 1024-byte chunks of 64-byte blocks, flagged CHUNK_START/CHUNK_END;
 * - the binary chunk tree, whose left subtree holds the largest power-of-two
 *   number of chunks that leaves at least one byte to the right, written here
 *   recursively exactly as the specification states it;
 * - the ROOT flag on the final compression.
 * The GPU builds the same tree bottom-up (aligned groups, then a level-wise
 * merge); the recursion here is the independent formulation it is checked
 * against.
 */
#include <stdlib.h>
#include <string.h>

#include "volta_oracle.h"

enum { B3_CHUNK_START = 1, B3_CHUNK_END = 2, B3_PARENT = 4, B3_ROOT = 8 };
enum { B3_BLOCK = 64, B3_CHUNK = 1024 };

static const uint32_t B3_IV[8] = {0x6A09E667u, 0xBB67AE85u, 0x3C6EF372u, 0xA54FF53Au,
                                  0x510E527Fu, 0x9B05688Cu, 0x1F83D9ABu, 0x5BE0CD19u};
/* message word order for round r+1 = order of round r permuted by this table */
static const uint8_t B3_PERMUTE[16] = {2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8};

static inline uint32_t b3_rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

static inline void b3_g(uint32_t* v, int a, int b, int c, int d, uint32_t mx, uint32_t my) {
    v[a] = v[a] + v[b] + mx;
    v[d] = b3_rotr(v[d] ^ v[a], 16);
    v[c] = v[c] + v[d];
    v[b] = b3_rotr(v[b] ^ v[c], 12);
    v[a] = v[a] + v[b] + my;
    v[d] = b3_rotr(v[d] ^ v[a], 8);
    v[c] = v[c] + v[d];
    v[b] = b3_rotr(v[b] ^ v[c], 7);
}

/* compress(cv, block, counter, block_len, flags) -> 16 output words */
static void b3_compress(const uint32_t cv[8], const uint8_t block[B3_BLOCK], uint64_t counter, uint32_t block_len,
                        uint32_t flags, uint32_t out[16]) {
    uint32_t m[16], v[16], t[16];
    for (int i = 0; i < 16; ++i)
        m[i] = (uint32_t)block[4 * i] | ((uint32_t)block[4 * i + 1] << 8) | ((uint32_t)block[4 * i + 2] << 16) |
               ((uint32_t)block[4 * i + 3] << 24);
    for (int i = 0; i < 8; ++i) v[i] = cv[i];
    for (int i = 0; i < 4; ++i) v[8 + i] = B3_IV[i];
    v[12] = (uint32_t)counter;
    v[13] = (uint32_t)(counter >> 32);
    v[14] = block_len;
    v[15] = flags;
    for (int r = 0; r < 7; ++r) {
        /* columns, then diagonals */
        b3_g(v, 0, 4, 8, 12, m[0], m[1]);
        b3_g(v, 1, 5, 9, 13, m[2], m[3]);
        b3_g(v, 2, 6, 10, 14, m[4], m[5]);
        b3_g(v, 3, 7, 11, 15, m[6], m[7]);
        b3_g(v, 0, 5, 10, 15, m[8], m[9]);
        b3_g(v, 1, 6, 11, 12, m[10], m[11]);
        b3_g(v, 2, 7, 8, 13, m[12], m[13]);
        b3_g(v, 3, 4, 9, 14, m[14], m[15]);
        for (int i = 0; i < 16; ++i) t[i] = m[B3_PERMUTE[i]];
        memcpy(m, t, sizeof m);
    }
    for (int i = 0; i < 8; ++i) {
        out[i] = v[i] ^ v[i + 8];
        out[i + 8] = v[i + 8] ^ cv[i];
    }
}

/* Chaining value of one chunk (len <= 1024; an empty input is one empty block).
 * With root set, the last block carries ROOT and its output is the hash. */
static void b3_chunk(const uint8_t* in, size_t len, uint64_t counter, int root, uint32_t cv_out[8]) {
    uint32_t cv[8], out[16];
    memcpy(cv, B3_IV, sizeof cv);
    const size_t blocks = len == 0 ? 1 : (len + B3_BLOCK - 1) / B3_BLOCK;
    for (size_t b = 0; b < blocks; ++b) {
        uint8_t block[B3_BLOCK] = {0};
        const size_t off = b * B3_BLOCK;
        const size_t take = len - off < B3_BLOCK ? len - off : B3_BLOCK;
        if (take) memcpy(block, in + off, take);
        uint32_t flags = 0;
        if (b == 0) flags |= B3_CHUNK_START;
        if (b + 1 == blocks) flags |= B3_CHUNK_END | (root ? B3_ROOT : 0);
        b3_compress(cv, block, counter, (uint32_t)take, flags, out);
        memcpy(cv, out, sizeof cv);
    }
    memcpy(cv_out, cv, 8 * sizeof(uint32_t));
}

static void b3_parent(const uint32_t l[8], const uint32_t r[8], int root, uint32_t cv_out[8]) {
    uint8_t block[B3_BLOCK];
    for (int i = 0; i < 8; ++i)
        for (int k = 0; k < 4; ++k) {
            block[4 * i + k] = (uint8_t)(l[i] >> (8 * k));
            block[32 + 4 * i + k] = (uint8_t)(r[i] >> (8 * k));
        }
    uint32_t out[16];
    b3_compress(B3_IV, block, 0, B3_BLOCK, B3_PARENT | (root ? B3_ROOT : 0), out);
    memcpy(cv_out, out, 8 * sizeof(uint32_t));
}

/* Subtree over in[0..len) whose first chunk has index chunk0. */
static void b3_node(const uint8_t* in, size_t len, uint64_t chunk0, int root, uint32_t cv_out[8]) {
    if (len <= B3_CHUNK) {
        b3_chunk(in, len, chunk0, root, cv_out);
        return;
    }
    size_t left_chunks = 1;  /* largest power of two with left_chunks * 1024 < len */
    while (2 * left_chunks * B3_CHUNK < len) left_chunks *= 2;
    const size_t left_len = left_chunks * B3_CHUNK;
    uint32_t l[8], r[8];
    b3_node(in, left_len, chunk0, 0, l);
    b3_node(in + left_len, len - left_len, chunk0 + left_chunks, 0, r);
    b3_parent(l, r, root, cv_out);
}

static void b3_store(const uint32_t cv[8], uint8_t out[32]) {
    for (int i = 0; i < 8; ++i)
        for (int k = 0; k < 4; ++k) out[4 * i + k] = (uint8_t)(cv[i] >> (8 * k));
}

void vo_blake3(const uint8_t* in, size_t len, uint8_t out[32]) {
    uint32_t cv[8];
    b3_node(in, len, 0, 1, cv);
    b3_store(cv, out);
}

/* Leaf j = blake3 of column j's values as little-endian u64 words, row by row
 * (ligero.rs:595-614 with col_bytes ligero.rs:351-357); an Fp2 value is c0
 * then c1.  words = 1 (Fp) or 2 (Fp2). */
static void columns(const uint64_t* m, size_t rows, size_t cols, size_t words, uint8_t* leaves, int threads) {
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
    {
        uint8_t* buf = (uint8_t*)malloc(rows * words * 8);
#pragma omp for schedule(static)
        for (long j = 0; j < (long)cols; ++j) {
            for (size_t i = 0; i < rows; ++i)
                for (size_t w = 0; w < words; ++w) {
                    const uint64_t x = m[(i * cols + (size_t)j) * words + w];
                    for (int k = 0; k < 8; ++k) buf[(i * words + w) * 8 + k] = (uint8_t)(x >> (8 * k));
                }
            vo_blake3(buf, rows * words * 8, leaves + 32 * (size_t)j);
        }
        free(buf);
    }
}

void vo_hash_fp_columns(const uint64_t* m, size_t rows, size_t cols, uint8_t* leaves, int threads) {
    columns(m, rows, cols, 1, leaves, threads);
}

void vo_hash_fp2_columns(const vo_fp2* m, size_t rows, size_t cols, uint8_t* leaves, int threads) {
    columns((const uint64_t*)m, rows, cols, 2, leaves, threads);
}

/* MerkleTree::from_leaves (merkle.rs:27-37) with hash_pair = blake3(l || r)
 * (merkle.rs:13-18), stored level by level: leaves, then each parent level,
 * the root last (2n - 1 hashes, the reference's resident tree layout,
 * rust/volta-accel/src/lib.rs:6700-6725). */
void vo_merkle_tree(const uint8_t* leaves, size_t n, uint8_t* tree) {
    memcpy(tree, leaves, 32 * n);
    size_t off = 0;
    for (size_t len = n; len > 1; len /= 2) {
        for (size_t i = 0; i < len / 2; ++i) vo_blake3(tree + 32 * (off + 2 * i), 64, tree + 32 * (off + len + i));
        off += len;
    }
}

/* MerkleTree::open (merkle.rs:43-51) for each query: the sibling at every
 * level from the leaves up.  An index outside [0, leaves) yields zero hashes
 * (the seam validates indices first). */
void vo_merkle_paths(const uint8_t* tree, size_t leaves, const uint32_t* idx, size_t queries, uint8_t* paths) {
    size_t bits = 0;
    while (((size_t)1 << bits) < leaves) ++bits;
    for (size_t q = 0; q < queries; ++q) {
        size_t i = idx[q], off = 0, len = leaves;
        for (size_t l = 0; l < bits; ++l) {
            uint8_t* dst = paths + 32 * (q * bits + l);
            if (idx[q] < leaves) memcpy(dst, tree + 32 * (off + (i ^ 1)), 32);
            else memset(dst, 0, 32);
            off += len;
            len /= 2;
            i /= 2;
        }
    }
}

/* The reference's synthetic Merkle benchmark matrix, M[i] = (i 0x9E3779B9 + 17) mod p
 * (cuda/p7_blake3_merkle.cu:243), for the P4_LAYER root pins. */
void vo_merkle_bench_matrix(size_t rows, size_t cols, uint64_t* m, int threads) {
    const uint64_t p = 0xFFFFFFFF00000001ull;
    /* the reference evaluates i * 0x9E3779B9 + 17 in wrapping 64-bit arithmetic */
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
    for (long i = 0; i < (long)(rows * cols); ++i) m[i] = ((uint64_t)i * 0x9E3779B9ull + 17) % p;
}

/* commit_impl (ligero.rs:543-624) end to end, without a backend: per-row pads
 * FpStream::domain_separated(seed, r) (ligero.rs:555-563), each row encoded
 * as NttPlan::forward of lift(w) || pads || 0 (ligero.rs:584-592), blake3
 * column leaves (ligero.rs:596-616) and MerkleTree::from_leaves (ligero.rs:620);
 * writes the 32-byte root.  `encoded` (rows x code_len) and `pads` (rows x pad)
 * receive the intermediate matrices when non-null.  Returns 0, or -1 when the
 * geometry is invalid (code_len not a power of two, cols + pad > code_len) or
 * memory runs out. */
int vo_commit_root(const int16_t* w, size_t rows, size_t cols, size_t pad, size_t code_len,
                   const uint8_t seed[32], uint8_t root[32], uint64_t* encoded, uint64_t* pads,
                   int threads) {
    if (!rows || !cols || code_len < 1 || (code_len & (code_len - 1)) || cols + pad > code_len) return -1;
    uint64_t* enc = encoded ? encoded : (uint64_t*)malloc(rows * code_len * sizeof(uint64_t));
    uint64_t* pd = pads ? pads : (uint64_t*)malloc((rows * pad + 1) * sizeof(uint64_t));
    uint8_t* leaves = (uint8_t*)malloc(code_len * 32);
    uint8_t* tree = (uint8_t*)malloc((2 * code_len - 1) * 32);
    int rc = 0;
    if (!enc || !pd || !leaves || !tree) {
        rc = -1;
    } else {
        if (pad) vo_fp_rows(seed, 0, rows, pad, pd, threads);
        vo_pcs_encode_i16(w, pd, rows, cols, pad, code_len, enc, threads);
        vo_hash_fp_columns(enc, rows, code_len, leaves, threads);
        vo_merkle_tree(leaves, code_len, tree);
        memcpy(root, tree + 32 * (2 * code_len - 2), 32);
    }
    if (!encoded) free(enc);
    if (!pads) free(pd);
    free(leaves);
    free(tree);
    return rc;
}
