// merkle.hip -- BLAKE3 column leaves and the binary Merkle tree over them,
// the commitment that closes the reference's Ligero commit
// (rust/volta-pcs/src/ligero.rs:595-621, rust/volta-pcs/src/merkle.rs:9-51).
//
// Leaf j is blake3 (the blake3 1.8.5 crate's unkeyed hash) of column j of the
// row-major matrix, read as little-endian u64 words row by row; an Fp2
// element contributes c0 then c1.  Inner nodes are blake3(left || right).
// The tree buffer holds 2 cols - 1 hashes level by level, root last.
//
// BLAKE3 cuts a column's byte stream into 1024-byte chunks (128 Fp rows or 64
// Fp2 rows) and joins chunk chaining values in a binary tree whose left
// subtrees are complete power-of-two blocks.  Any aligned power-of-two run of
// chunks is therefore an exact subtree, and a short run at the end is the
// left-complete subtree over what remains; the GPU builds the tree in such
// runs, bottom up:
//   column_groups: one thread per (column, run of up to 4 chunks).  A wave's
//     lanes are 64 consecutive columns, so every row read is one coalesced
//     512-byte (Fp) or 1 KiB (Fp2) segment.  The thread hashes its chunks in
//     order, loading the next block while it compresses the current one, and
//     joins them with two registers of pending values (no LDS, so occupancy
//     is set by registers alone).
//   merge_pass: one thread per (column, run of 16 values) folds them with an
//     eager join stack in LDS, repeated until one value per column is left;
//     the column's last join carries the ROOT flag.
//   merkle_level / merkle_top: the pair hashes of the Merkle tree.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>

#include "context.hpp"
#include "gl64_shift.hpp"
#include "kernels.hpp"

namespace vmx {

namespace b3 {

constexpr uint32_t CHUNK_START = 1, CHUNK_END = 2, PARENT = 4, ROOT = 8;
constexpr std::array<uint32_t, 8> IV = {0x6A09E667u, 0xBB67AE85u, 0x3C6EF372u, 0xA54FF53Au,
                                        0x510E527Fu, 0x9B05688Cu, 0x1F83D9ABu, 0x5BE0CD19u};

// Message word order of each of the 7 rounds: round r + 1 reads word
// SCHED[r][PERM[i]] at position i (the specification's fixed permutation).
constexpr std::array<std::array<uint8_t, 16>, 7> make_schedule() {
    constexpr uint8_t perm[16] = {2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8};
    std::array<std::array<uint8_t, 16>, 7> s{};
    for (int i = 0; i < 16; ++i) s[0][i] = static_cast<uint8_t>(i);
    for (int r = 1; r < 7; ++r)
        for (int i = 0; i < 16; ++i) s[r][i] = s[r - 1][perm[i]];
    return s;
}
constexpr auto SCHED = make_schedule();

__device__ __forceinline__ uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

__device__ __forceinline__ void g(uint32_t& a, uint32_t& b, uint32_t& c, uint32_t& d, uint32_t x, uint32_t y) {
    a = a + b + x;
    d = rotr(d ^ a, 16);
    c = c + d;
    b = rotr(b ^ c, 12);
    a = a + b + y;
    d = rotr(d ^ a, 8);
    c = c + d;
    b = rotr(b ^ c, 7);
}

// cv[s] <- the chaining value of compress(cv[s], m[s], counter, block_len,
// flags) for S independent states, their G functions interleaved so one
// lane keeps several dependency chains in flight.
template <int S>
__device__ __forceinline__ void compress_n(uint32_t (*cv)[8], const uint32_t (*m)[16], uint64_t counter,
                                           uint32_t block_len, uint32_t flags) {
    uint32_t v[S][16];
#pragma unroll
    for (int q = 0; q < S; ++q) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[q][i] = cv[q][i];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[q][8 + i] = IV[i];
        v[q][12] = static_cast<uint32_t>(counter);
        v[q][13] = static_cast<uint32_t>(counter >> 32);
        v[q][14] = block_len;
        v[q][15] = flags;
    }
    gl::static_for<0, 7>([&](auto rr) {
        constexpr auto s = SCHED[decltype(rr)::value];
#pragma unroll
        for (int q = 0; q < S; ++q) {
            g(v[q][0], v[q][4], v[q][8], v[q][12], m[q][s[0]], m[q][s[1]]);
            g(v[q][1], v[q][5], v[q][9], v[q][13], m[q][s[2]], m[q][s[3]]);
            g(v[q][2], v[q][6], v[q][10], v[q][14], m[q][s[4]], m[q][s[5]]);
            g(v[q][3], v[q][7], v[q][11], v[q][15], m[q][s[6]], m[q][s[7]]);
        }
#pragma unroll
        for (int q = 0; q < S; ++q) {
            g(v[q][0], v[q][5], v[q][10], v[q][15], m[q][s[8]], m[q][s[9]]);
            g(v[q][1], v[q][6], v[q][11], v[q][12], m[q][s[10]], m[q][s[11]]);
            g(v[q][2], v[q][7], v[q][8], v[q][13], m[q][s[12]], m[q][s[13]]);
            g(v[q][3], v[q][4], v[q][9], v[q][14], m[q][s[14]], m[q][s[15]]);
        }
    });
#pragma unroll
    for (int q = 0; q < S; ++q)
#pragma unroll
        for (int i = 0; i < 8; ++i) cv[q][i] = v[q][i] ^ v[q][i + 8];
}

__device__ __forceinline__ void compress(uint32_t* cv, const uint32_t* m, uint64_t counter, uint32_t block_len,
                                         uint32_t flags) {
    compress_n<1>(reinterpret_cast<uint32_t(*)[8]>(cv), reinterpret_cast<const uint32_t(*)[16]>(m), counter,
                  block_len, flags);
}

// out[s] <- compress(IV, l[s] || r[s], 0, 64, flags) for S pairs: BLAKE3
// parent nodes (flags PARENT [| ROOT]) or, with CHUNK_START | CHUNK_END |
// ROOT, the hash of the 64 bytes l || r as a message (the Merkle pair hash).
template <int S>
__device__ __forceinline__ void join_n(uint32_t (*out)[8], const uint32_t (*l)[8], const uint32_t (*r)[8],
                                       uint32_t flags) {
    uint32_t m[S][16], cv[S][8];
#pragma unroll
    for (int q = 0; q < S; ++q)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            m[q][i] = l[q][i];
            m[q][8 + i] = r[q][i];
            cv[q][i] = IV[i];
        }
    compress_n<S>(cv, m, 0, 64, flags);
#pragma unroll
    for (int q = 0; q < S; ++q)
#pragma unroll
        for (int i = 0; i < 8; ++i) out[q][i] = cv[q][i];
}

__device__ __forceinline__ void join(uint32_t* out, const uint32_t* l, const uint32_t* r, uint32_t flags) {
    join_n<1>(reinterpret_cast<uint32_t(*)[8]>(out), reinterpret_cast<const uint32_t(*)[8]>(l),
              reinterpret_cast<const uint32_t(*)[8]>(r), flags);
}

__device__ __forceinline__ void store_hash(uint32_t* dst, const uint32_t* h) {
    using u32x4 = uint32_t __attribute__((ext_vector_type(4)));
    reinterpret_cast<u32x4*>(dst)[0] = u32x4{h[0], h[1], h[2], h[3]};
    reinterpret_cast<u32x4*>(dst)[1] = u32x4{h[4], h[5], h[6], h[7]};
}

__device__ __forceinline__ void load_hash(uint32_t* h, const uint32_t* src) {
    using u32x4 = uint32_t __attribute__((ext_vector_type(4)));
    const u32x4 a = reinterpret_cast<const u32x4*>(src)[0], b = reinterpret_cast<const u32x4*>(src)[1];
    h[0] = a.x, h[1] = a.y, h[2] = a.z, h[3] = a.w, h[4] = b.x, h[5] = b.y, h[6] = b.z, h[7] = b.w;
}

constexpr int LANES = 64;          // columns per column_groups workgroup (one wave)
constexpr size_t CHUNK_WORDS = 128; // u64 words per 1024-byte chunk

// W = u64 words per matrix element: 1 for Fp, 2 for Fp2.  Thread (column,
// g) hashes the chunks [g G, min(g G + G, chunks)) of its column, G <= 4, and
// joins them left-complete with two registers of pending values: chunks 0+1
// and 2+3 pair up, then the pairs; a short last group of 3 joins (0+1)+2.
// Writes the group's chaining value to out[(g cols + col) 8 ..], or with
// root set (one group per column) the column's leaf hash to out[col 8 ..].
// OFF32: a row of the matrix spans less than 4 GiB, so a lane's element is
// addressed as the uniform row pointer plus a 32-bit byte offset.
template <int W, bool OFF32>
__global__ __launch_bounds__(LANES, 6) void column_groups(const uint64_t* __restrict__ m, size_t rows, size_t cols,
                                                       size_t chunks, size_t group, int root,
                                                       uint32_t* __restrict__ out) {
    const int lane = threadIdx.x;
    const size_t col = static_cast<size_t>(blockIdx.x) * LANES + lane;
    if (col >= cols) return;
    const size_t gi = blockIdx.y;
    const size_t c_begin = gi * group;
    const size_t c_end = min(chunks, c_begin + group);
    const size_t n_local = c_end - c_begin;  // 1..4
    const size_t words = rows * W;            // the column's u64 word stream
    const size_t row_stride = cols * W;
    const uint32_t lane_bytes = static_cast<uint32_t>(col * W * sizeof(uint64_t));  // used when OFF32
    // blocks of the group in stream order: only the column's last chunk can
    // be short, and it comes last, so block k starts at word (c_begin 16 + k) 8
    const size_t last_words = words - (c_end - 1) * CHUNK_WORDS;
    const size_t total = (n_local - 1) * 16 + (min(CHUNK_WORDS, last_words) + 7) / 8;

    auto element = [&](size_t row, int part) -> const uint64_t* {
        const uint64_t* rowp = m + row * row_stride;
        if constexpr (OFF32)
            return reinterpret_cast<const uint64_t*>(reinterpret_cast<const char*>(rowp) + lane_bytes) + part;
        else
            return rowp + col * W + part;
    };
    auto load_block = [&](size_t k, uint32_t* mw) {
        const size_t w0 = (c_begin * 16 + k) * 8;
        if (w0 + 8 <= words) {
            if constexpr (W == 1) {
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const uint64_t x = *element(w0 + i, 0);
                    mw[2 * i] = static_cast<uint32_t>(x);
                    mw[2 * i + 1] = static_cast<uint32_t>(x >> 32);
                }
            } else {
                using u32x4 = uint32_t __attribute__((ext_vector_type(4)));
#pragma unroll
                for (int i = 0; i < 4; ++i) {  // one 16-byte (c0, c1) load per row
                    const u32x4 x = *reinterpret_cast<const u32x4*>(element(w0 / 2 + i, 0));
                    mw[4 * i] = x.x, mw[4 * i + 1] = x.y, mw[4 * i + 2] = x.z, mw[4 * i + 3] = x.w;
                }
            }
        } else {  // the column's last, partial block: zero past the end
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const size_t w = w0 + i;
                const uint64_t x = w < words ? *element(w / W, static_cast<int>(w % W)) : 0;
                mw[2 * i] = static_cast<uint32_t>(x);
                mw[2 * i + 1] = static_cast<uint32_t>(x >> 32);
            }
        }
    };

    const uint32_t top = root ? PARENT | ROOT : PARENT;  // flags of the group's last join
    uint32_t cv[8], p0[8], p1[8];
    auto compress_block = [&](const uint32_t* mw, size_t k, int cb, int nb) {
        const size_t left = words - (c_begin * 16 + k) * 8;
        const uint32_t len = static_cast<uint32_t>(min<size_t>(8, left) * 8);
        uint32_t flags = (cb == 0 ? CHUNK_START : 0u) | (cb + 1 == nb ? CHUNK_END : 0u);
        if (chunks == 1 && cb + 1 == nb) flags |= ROOT;  // a one-chunk column: this block is the root
        compress(cv, mw, c_begin + k / 16, len, flags);
    };

    // Two block buffers alternate: the next block loads while the current one
    // compresses.  A full chunk has 16 blocks, so the next chunk's first block
    // always lands in `a`; only the column's last chunk can be shorter.
    uint32_t a[16], b[16];
    load_block(0, a);
    for (size_t lc = 0; lc < n_local; ++lc) {
        const size_t k0 = lc * 16;
        const int nb = static_cast<int>(min<size_t>(16, total - k0));
#pragma unroll
        for (int i = 0; i < 8; ++i) cv[i] = IV[i];
        for (int cb = 0; cb < nb; cb += 2) {
            if (k0 + cb + 1 < total) load_block(k0 + cb + 1, b);
            compress_block(a, k0 + cb, cb, nb);
            if (cb + 1 == nb) break;
            if (k0 + cb + 2 < total) load_block(k0 + cb + 2, a);
            compress_block(b, k0 + cb + 1, cb + 1, nb);
        }
        // chunk lc done: chunks 0 and 2 wait in p0 / p1, chunks 1 and 3 join them
        if ((lc & 1) == 0) {
#pragma unroll
            for (int i = 0; i < 8; ++i) (lc == 0 ? p0 : p1)[i] = cv[i];
        } else {
            uint32_t l[8], j[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) l[i] = lc == 1 ? p0[i] : p1[i];
            join(j, l, cv, lc == 1 && n_local == 2 ? top : PARENT);
#pragma unroll
            for (int i = 0; i < 8; ++i) (lc == 1 ? p0 : p1)[i] = j[i];
        }
    }
    if (chunks == 1) {  // the single block chain already carried ROOT
        store_hash(out + col * 8, cv);
        return;
    }
    if (n_local >= 3) join(p0, p0, p1, top);  // (0+1) + 2  or  (0+1) + (2+3)
    store_hash(out + (root ? col : gi * cols + col) * 8, p0);
}

constexpr int FAN_IN = 16;      // values one merge_pass thread folds
constexpr int MERGE_DEPTH = 5;  // pending values of a left-complete fold of 16

// Thread (column, j) folds values [16 j, min(16 j + 16, k_in)) of its column
// (in[(i cols + col) 8 ..]) left-complete, joining complete power-of-two runs
// eagerly on a per-lane LDS stack; with final set this is the column's last
// fold and its top join carries ROOT.  k_in >= 2.
__global__ __launch_bounds__(LANES) void merge_pass(const uint32_t* __restrict__ in, size_t k_in, size_t cols,
                                                    int final, uint32_t* __restrict__ out) {
    __shared__ uint32_t stack[MERGE_DEPTH][8][LANES];
    const int lane = threadIdx.x;
    const size_t col = static_cast<size_t>(blockIdx.x) * LANES + lane;
    if (col >= cols) return;
    const size_t j = blockIdx.y;
    const size_t i0 = j * FAN_IN;
    const size_t n = min<size_t>(FAN_IN, k_in - i0);
    auto push = [&](int d, const uint32_t* h) {
#pragma unroll
        for (int i = 0; i < 8; ++i) stack[d][i][lane] = h[i];
    };
    auto peek = [&](int d, uint32_t* h) {
#pragma unroll
        for (int i = 0; i < 8; ++i) h[i] = stack[d][i][lane];
    };
    int depth = 0;
    for (size_t t = 1; t <= n; ++t) {
        uint32_t h[8];
        load_hash(h, in + ((i0 + t - 1) * cols + col) * 8);
        push(depth++, h);
        if (t == n) break;  // the last value is joined in the fold below
        for (size_t u = t; (u & 1) == 0; u >>= 1) {
            uint32_t l[8], r[8], p[8];
            peek(depth - 1, r);
            peek(depth - 2, l);
            join(p, l, r, PARENT);
            depth -= 2;
            push(depth++, p);
        }
    }
    uint32_t acc[8];
    peek(--depth, acc);
    while (depth > 0) {
        uint32_t l[8];
        peek(--depth, l);
        join(acc, l, acc, PARENT | (depth == 0 && final ? ROOT : 0u));
    }
    store_hash(out + (final ? col : j * cols + col) * 8, acc);
}

constexpr int MERGE_THREADS = 256;
constexpr int MERGE_MAX = 2 * MERGE_THREADS;  // values per column merge_final handles

// The column's last fold when it has k_in <= 512 values (in[(i cols + col) 8
// ..]): the workgroup holds cpw = 256 / tpc columns (tpc = ceil(k_in / 2)
// rounded up to a power of two) and joins each column's values level by
// level in LDS, carrying an odd last value up unchanged (which builds the
// same left-complete tree); the last join carries ROOT.  Each level is one
// join deep.
__global__ __launch_bounds__(MERGE_THREADS) void merge_final(const uint32_t* __restrict__ in, int k_in, size_t cols,
                                                             int cpw, uint32_t* __restrict__ leaves) {
    __shared__ uint32_t node[MERGE_MAX][9];  // odd pitch: a join reads two neighbouring nodes
    const int t = threadIdx.x;
    const int per = MERGE_MAX / cpw;          // node slots per column
    const int tpc = MERGE_THREADS / cpw;      // threads per column
    // columns interleave across threads: a level's active threads (r < pairs)
    // are the first pairs * cpw, packed into as few waves as possible
    const int q = t % cpw, r = t / cpw;       // column within the workgroup, thread within the column
    const size_t col = static_cast<size_t>(blockIdx.x) * cpw + q;
    const bool live = q < cpw && col < cols;
    uint32_t(*mine)[9] = node + q * per;
    if (live)
        for (int i = r; i < k_in; i += tpc) {
            uint32_t h[8];
            load_hash(h, in + (static_cast<size_t>(i) * cols + col) * 8);
#pragma unroll
            for (int w = 0; w < 8; ++w) mine[i][w] = h[w];
        }
    __syncthreads();
    for (int count = k_in; count > 1;) {
        const int pairs = count / 2;
        uint32_t p[8];
        const bool act = live && r < pairs;
        if (act) {
            uint32_t l[8], rr[8];
#pragma unroll
            for (int w = 0; w < 8; ++w) {
                l[w] = mine[2 * r][w];
                rr[w] = mine[2 * r + 1][w];
            }
            join(p, l, rr, PARENT | (count == 2 ? ROOT : 0u));
        }
        __syncthreads();
        if (act)
#pragma unroll
            for (int w = 0; w < 8; ++w) mine[r][w] = p[w];
        if (live && (count & 1) && r == pairs)  // carry the odd last value up unchanged
#pragma unroll
            for (int w = 0; w < 8; ++w) mine[pairs][w] = mine[count - 1][w];
        __syncthreads();
        count = pairs + (count & 1);
    }
    if (live && r == 0) {
        uint32_t h[8];
#pragma unroll
        for (int w = 0; w < 8; ++w) h[w] = mine[0][w];
        store_hash(leaves + col * 8, h);
    }
}

constexpr uint32_t PAIR_FLAGS = CHUNK_START | CHUNK_END | ROOT;  // blake3 of a 64-byte message

// parents[i] = blake3(child[2i] || child[2i+1])
__global__ __launch_bounds__(256) void merkle_level(const uint32_t* __restrict__ child, uint32_t* __restrict__ parent,
                                                    size_t parents) {
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= parents) return;
    uint32_t l[8], r[8], p[8];
    load_hash(l, child + 2 * i * 8);
    load_hash(r, child + (2 * i + 1) * 8);
    join(p, l, r, PAIR_FLAGS);
    store_hash(parent + i * 8, p);
}

constexpr int TOP_THREADS = 512;
constexpr size_t TOP_MAX = 2 * TOP_THREADS;  // nodes a single workgroup finishes

// The last levels in one workgroup: level (at tree + off 8, len <= TOP_MAX
// nodes) up to the root, staged through LDS and written level by level.
__global__ __launch_bounds__(TOP_THREADS) void merkle_top(uint32_t* __restrict__ tree, size_t off, int len) {
    __shared__ uint32_t cur[TOP_MAX][9];
    const int t = threadIdx.x;
    for (int i = t; i < len; i += TOP_THREADS) {
        uint32_t h[8];
        load_hash(h, tree + (off + i) * 8);
#pragma unroll
        for (int k = 0; k < 8; ++k) cur[i][k] = h[k];
    }
    __syncthreads();
    while (len > 1) {
        const int parents = len / 2;  // len is a power of two
        uint32_t p[8];
        if (t < parents) {
            uint32_t l[8], r[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                l[k] = cur[2 * t][k];
                r[k] = cur[2 * t + 1][k];
            }
            join(p, l, r, PAIR_FLAGS);
            store_hash(tree + (off + len + t) * 8, p);
        }
        __syncthreads();
        if (t < parents)
#pragma unroll
            for (int k = 0; k < 8; ++k) cur[t][k] = p[k];
        __syncthreads();
        off += len;
        len = parents;
    }
}

// paths[(q bits + l) 8 ..] = the level-l sibling of leaf idx[q]; zero for an
// index outside [0, leaves).
__global__ __launch_bounds__(256) void merkle_paths_kernel(const uint32_t* __restrict__ tree,
                                                           const uint32_t* __restrict__ idx,
                                                           uint32_t* __restrict__ paths, size_t leaves,
                                                           size_t queries, int bits) {
    const size_t z = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (z >= queries * bits) return;
    const size_t q = z / bits;
    const int level = static_cast<int>(z - q * bits);
    size_t i = idx[q];
    uint32_t h[8] = {};
    if (i < leaves) {
        size_t off = 0, len = leaves;
        for (int l = 0; l < level; ++l) {
            off += len;
            len >>= 1;
            i >>= 1;
        }
        load_hash(h, tree + (off + (i ^ 1)) * 8);
    }
    store_hash(paths + z * 8, h);
}

}  // namespace b3


int merkle_column_leaves(Context* c, const uint64_t* m, size_t rows, size_t cols, bool fp2, uint32_t* leaves) {
    const size_t w = fp2 ? 2 : 1;
    const size_t words = rows * w;
    const size_t chunks = (words + b3::CHUNK_WORDS - 1) / b3::CHUNK_WORDS;
    const size_t group = std::min<size_t>(4, chunks);  // chunks per column_groups thread
    size_t k = (chunks + group - 1) / group;           // values per column after column_groups
    if (k > 65535) return fail_msg(c, "Merkle column too long (more than 2^18 BLAKE3 chunks)");
    // workspace: column_groups' values, then each non-final merge pass's (16x fewer)
    size_t slots = 0;
    for (size_t kk = k; kk > 1; kk = (kk + b3::FAN_IN - 1) / b3::FAN_IN) slots += kk;
    uint32_t* buf = nullptr;
    if (k > 1) {
        size_t bytes = 0;
        if (!mul_ok(slots, cols * 32, &bytes)) return fail_msg(c, "Merkle workspace overflows size_t");
        if (ensure_ws(c, WS_HASH, bytes)) return -1;
        buf = ws<uint32_t>(c, WS_HASH);
    }
    const dim3 grid(static_cast<unsigned>((cols + b3::LANES - 1) / b3::LANES), static_cast<unsigned>(k));
    const int is_root = k == 1 ? 1 : 0;
    uint32_t* gout = k == 1 ? leaves : buf;
    const bool off32 = cols * w * sizeof(uint64_t) <= 0xFFFFFFFFull;
    auto launch = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, dim3(b3::LANES), 0, c->stream, m, rows, cols, chunks, group, is_root, gout);
    };
    if (fp2) off32 ? launch(b3::column_groups<2, true>) : launch(b3::column_groups<2, false>);
    else off32 ? launch(b3::column_groups<1, true>) : launch(b3::column_groups<1, false>);
    VMX_HIP(c, hipGetLastError());
    const uint32_t* in = buf;
    uint32_t* next = buf ? buf + k * cols * 8 : nullptr;
    while (k > static_cast<size_t>(b3::MERGE_MAX)) {  // 16-way passes down to a single workgroup's worth
        const size_t k_out = (k + b3::FAN_IN - 1) / b3::FAN_IN;
        hipLaunchKernelGGL(b3::merge_pass, dim3(static_cast<unsigned>((cols + b3::LANES - 1) / b3::LANES),
                                                static_cast<unsigned>(k_out)),
                           dim3(b3::LANES), 0, c->stream, in, k, cols, 0, next);
        VMX_HIP(c, hipGetLastError());
        in = next;
        next += k_out * cols * 8;
        k = k_out;
    }
    if (k > 1) {
        // threads per column: the first level's joins, rounded up to a power of two
        size_t tpc = 1;
        while (tpc < (k + 1) / 2) tpc *= 2;
        const int cpw = static_cast<int>(b3::MERGE_THREADS / tpc);
        hipLaunchKernelGGL(b3::merge_final, dim3(static_cast<unsigned>((cols + cpw - 1) / cpw)),
                           dim3(b3::MERGE_THREADS), 0, c->stream, in, static_cast<int>(k), cols, cpw, leaves);
        VMX_HIP(c, hipGetLastError());
    }
    return 0;
}

int merkle_tree_levels(Context* c, uint32_t* tree, size_t leaves) {
    size_t off = 0, len = leaves;
    while (len > b3::TOP_MAX) {
        const size_t parents = len / 2;
        hipLaunchKernelGGL(b3::merkle_level, dim3(static_cast<unsigned>((parents + 255) / 256)), dim3(256), 0,
                           c->stream, static_cast<const uint32_t*>(tree + off * 8), tree + (off + len) * 8, parents);
        VMX_HIP(c, hipGetLastError());
        off += len;
        len = parents;
    }
    if (len > 1) {
        hipLaunchKernelGGL(b3::merkle_top, dim3(1), dim3(b3::TOP_THREADS), 0, c->stream, tree, off,
                           static_cast<int>(len));
        VMX_HIP(c, hipGetLastError());
    }
    return 0;
}

int merkle_paths(Context* c, const uint32_t* tree, size_t leaves, const uint32_t* idx, size_t queries,
                 uint32_t* paths) {
    int bits = 0;
    while ((size_t{1} << bits) < leaves) ++bits;
    const size_t total = queries * bits;
    hipLaunchKernelGGL(b3::merkle_paths_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0,
                       c->stream, tree, idx, paths, leaves, queries, bits);
    VMX_HIP(c, hipGetLastError());
    return 0;
}

}  // namespace vmx
