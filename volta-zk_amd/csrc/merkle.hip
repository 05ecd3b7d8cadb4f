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
// subtrees are complete power-of-two blocks.  On the GPU:
//   column_groups: one thread per (column, aligned group of G chunks).  A
//     wave's lanes are 64 consecutive columns, so every row read is one
//     coalesced 512-byte (Fp) or 1 KiB (Fp2) segment.  The thread hashes its
//     chunks in order, prefetching the next block's 8 words while it
//     compresses the current one, and merges chunk values eagerly on a small
//     per-lane stack in LDS.  Aligned groups of a power-of-two size are exact
//     subtrees of the BLAKE3 tree, and a short last group is the subtree over
//     the remaining chunks.
//   merge_groups: one workgroup per column joins its group values level by
//     level, carrying an odd last node up unchanged; that pairing builds the
//     same left-complete tree, and the last join carries the ROOT flag.
//   merkle_level / merkle_top: the pair hashes of the Merkle tree.
#include <hip/hip_runtime.h>

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

// cv <- the chaining value of compress(cv, m, counter, block_len, flags).
__device__ __forceinline__ void compress(uint32_t* cv, const uint32_t* m, uint64_t counter, uint32_t block_len,
                                         uint32_t flags) {
    uint32_t v[16] = {cv[0],  cv[1],  cv[2],  cv[3],  cv[4],  cv[5],
                      cv[6],  cv[7],  IV[0],  IV[1],  IV[2],  IV[3],
                      static_cast<uint32_t>(counter), static_cast<uint32_t>(counter >> 32), block_len, flags};
    gl::static_for<0, 7>([&](auto rr) {
        constexpr auto s = SCHED[decltype(rr)::value];
        g(v[0], v[4], v[8], v[12], m[s[0]], m[s[1]]);
        g(v[1], v[5], v[9], v[13], m[s[2]], m[s[3]]);
        g(v[2], v[6], v[10], v[14], m[s[4]], m[s[5]]);
        g(v[3], v[7], v[11], v[15], m[s[6]], m[s[7]]);
        g(v[0], v[5], v[10], v[15], m[s[8]], m[s[9]]);
        g(v[1], v[6], v[11], v[12], m[s[10]], m[s[11]]);
        g(v[2], v[7], v[8], v[13], m[s[12]], m[s[13]]);
        g(v[3], v[4], v[9], v[14], m[s[14]], m[s[15]]);
    });
#pragma unroll
    for (int i = 0; i < 8; ++i) cv[i] = v[i] ^ v[i + 8];
}

// out <- compress(IV, l || r, 0, 64, flags): a BLAKE3 parent node (flags
// PARENT [| ROOT]) or, with CHUNK_START | CHUNK_END | ROOT, the hash of the
// 64 bytes l || r as a message (the Merkle pair hash).
__device__ __forceinline__ void join(uint32_t* out, const uint32_t* l, const uint32_t* r, uint32_t flags) {
    uint32_t m[16], cv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        m[i] = l[i];
        m[8 + i] = r[i];
        cv[i] = IV[i];
    }
    compress(cv, m, 0, 64, flags);
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = cv[i];
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
constexpr size_t MAX_GROUPS = 256;  // merge_groups handles up to this many groups per column
constexpr size_t MAX_GROUP = 4096;  // chunks per group (LDS stack depth 13)

// W = u64 words per matrix element: 1 for Fp, 2 for Fp2.  Writes the group's
// chaining value to out[(g cols + col) 8 ..], or with root set (one group
// per column) the column's leaf hash to out[col 8 ..].
template <int W>
__global__ __launch_bounds__(LANES) void column_groups(const uint64_t* __restrict__ m, size_t rows, size_t cols,
                                                       size_t chunks, size_t group, int root,
                                                       uint32_t* __restrict__ out) {
    extern __shared__ uint32_t stack[];  // [depth][8 words][LANES]
    const int lane = threadIdx.x;
    const size_t col = static_cast<size_t>(blockIdx.x) * LANES + lane;
    if (col >= cols) return;  // no barriers below: the stack is per lane
    const size_t gi = blockIdx.y;
    const size_t c_begin = gi * group;
    const size_t c_end = min(chunks, c_begin + group);
    const size_t words = rows * W;  // the column's u64 word stream
    const size_t row_stride = cols * W;
    const uint64_t* base = m + col * W;

    auto blocks_in = [&](size_t c) -> int {
        const size_t w = min(CHUNK_WORDS, words - c * CHUNK_WORDS);
        return static_cast<int>((w + 7) / 8);
    };
    // block b of chunk c: stream words [c 128 + 8 b, + 8), zero past the end
    auto load_block = [&](size_t c, int b, uint32_t* mw) {
        const size_t w0 = c * CHUNK_WORDS + static_cast<size_t>(b) * 8;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const size_t w = w0 + k;
            const size_t row = w / W, part = w - row * W;
            const uint64_t x = w < words ? base[row * row_stride + part] : 0;
            mw[2 * k] = static_cast<uint32_t>(x);
            mw[2 * k + 1] = static_cast<uint32_t>(x >> 32);
        }
    };
    auto push = [&](int d, const uint32_t* h) {
#pragma unroll
        for (int i = 0; i < 8; ++i) stack[(d * 8 + i) * LANES + lane] = h[i];
    };
    auto peek = [&](int d, uint32_t* h) {
#pragma unroll
        for (int i = 0; i < 8; ++i) h[i] = stack[(d * 8 + i) * LANES + lane];
    };

    int depth = 0;
    uint32_t cv[8], nxt[16];
    size_t c = c_begin;
    int b = 0, blocks = blocks_in(c);
    load_block(c, 0, nxt);
    while (c < c_end) {
        uint32_t cur[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) cur[i] = nxt[i];
        const size_t cc = c;
        const int cb = b, cblocks = blocks;
        if (++b == blocks) {
            ++c;
            b = 0;
            if (c < c_end) blocks = blocks_in(c);
        }
        if (c < c_end) load_block(c, b, nxt);  // in flight during the compression below

        const size_t left = words - cc * CHUNK_WORDS - static_cast<size_t>(cb) * 8;
        const uint32_t len = static_cast<uint32_t>(min<size_t>(8, left) * 8);
        if (cb == 0)
#pragma unroll
            for (int i = 0; i < 8; ++i) cv[i] = IV[i];
        uint32_t flags = (cb == 0 ? CHUNK_START : 0u) | (cb + 1 == cblocks ? CHUNK_END : 0u);
        if (chunks == 1 && cb + 1 == cblocks) flags |= ROOT;  // a one-chunk column: this block is the root
        compress(cv, cur, cc, len, flags);
        if (cb + 1 != cblocks) continue;
        if (chunks == 1) {
            store_hash(out + col * 8, cv);
            return;
        }
        push(depth++, cv);
        size_t t = cc - c_begin + 1;  // chunks of this group done
        if (t < c_end - c_begin) {
            // eager joins of complete power-of-two runs; the group's last
            // chunk is joined in the final fold so the root join can be flagged
            while ((t & 1) == 0) {
                uint32_t l[8], r[8], p[8];
                peek(depth - 1, r);
                peek(depth - 2, l);
                join(p, l, r, PARENT);
                depth -= 2;
                push(depth++, p);
                t >>= 1;
            }
        }
    }
    uint32_t acc[8];
    peek(--depth, acc);
    while (depth > 0) {
        uint32_t l[8];
        peek(--depth, l);
        join(acc, l, acc, PARENT | (depth == 0 && root ? ROOT : 0u));
    }
    store_hash(out + (root ? col : gi * cols + col) * 8, acc);
}

// One workgroup per column: joins the column's `groups` chaining values
// (gcv[(g cols + col) 8 ..]) level by level into the leaf hash.
__global__ __launch_bounds__(MAX_GROUPS) void merge_groups(const uint32_t* __restrict__ gcv, size_t groups,
                                                           size_t cols, uint32_t* __restrict__ leaves) {
    __shared__ uint32_t node[MAX_GROUPS][9];  // odd pitch: a join reads two nodes per lane
    const size_t col = blockIdx.x;
    const int t = threadIdx.x;
    if (static_cast<size_t>(t) < groups) {
        uint32_t h[8];
        load_hash(h, gcv + (t * cols + col) * 8);
#pragma unroll
        for (int i = 0; i < 8; ++i) node[t][i] = h[i];
    }
    __syncthreads();
    int count = static_cast<int>(groups);
    while (count > 1) {
        const int pairs = count / 2;
        uint32_t p[8];
        if (t < pairs) {
            uint32_t l[8], r[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                l[i] = node[2 * t][i];
                r[i] = node[2 * t + 1][i];
            }
            join(p, l, r, PARENT | (count == 2 ? ROOT : 0u));
        }
        __syncthreads();
        if (t < pairs)
#pragma unroll
            for (int i = 0; i < 8; ++i) node[t][i] = p[i];
        if ((count & 1) && t == pairs)  // carry the odd last node up unchanged
#pragma unroll
            for (int i = 0; i < 8; ++i) node[pairs][i] = node[count - 1][i];
        __syncthreads();
        count = pairs + (count & 1);
    }
    if (t == 0) {
        uint32_t h[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) h[i] = node[0][i];
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

namespace {

size_t log2_exact(size_t n) {
    size_t b = 0;
    while ((size_t{1} << b) < n) ++b;
    return b;
}

}  // namespace

int merkle_column_leaves(Context* c, const uint64_t* m, size_t rows, size_t cols, bool fp2, uint32_t* leaves) {
    const size_t w = fp2 ? 2 : 1;
    const size_t words = rows * w;
    const size_t chunks = (words + b3::CHUNK_WORDS - 1) / b3::CHUNK_WORDS;
    // Groups: enough threads to fill the GPU (about 16 waves per CU), at most
    // MAX_GROUPS per column for merge_groups.
    constexpr size_t TARGET_THREADS = size_t{1} << 18;
    size_t group = 1;
    while (group < chunks && cols * ((chunks + 2 * group - 1) / (2 * group)) >= TARGET_THREADS) group *= 2;
    while ((chunks + group - 1) / group > b3::MAX_GROUPS) group *= 2;
    if (group > b3::MAX_GROUP) return fail_msg(c, "Merkle column too long (more than 2^20 BLAKE3 chunks)");
    const size_t groups = (chunks + group - 1) / group;
    const int depth = static_cast<int>(log2_exact(group)) + 1;
    const size_t lds = static_cast<size_t>(depth) * 8 * b3::LANES * sizeof(uint32_t);
    uint32_t* gout = leaves;
    if (groups > 1) {
        size_t bytes = 0;
        if (!mul_ok(groups * cols, 32, &bytes)) return fail_msg(c, "Merkle group buffer overflows size_t");
        if (ensure_ws(c, WS_HASH, bytes)) return -1;
        gout = ws<uint32_t>(c, WS_HASH);
    }
    const dim3 grid(static_cast<unsigned>((cols + b3::LANES - 1) / b3::LANES), static_cast<unsigned>(groups));
    if (fp2)
        hipLaunchKernelGGL(b3::column_groups<2>, grid, dim3(b3::LANES), lds, c->stream, m, rows, cols, chunks, group,
                           groups == 1 ? 1 : 0, gout);
    else
        hipLaunchKernelGGL(b3::column_groups<1>, grid, dim3(b3::LANES), lds, c->stream, m, rows, cols, chunks, group,
                           groups == 1 ? 1 : 0, gout);
    VMX_HIP(c, hipGetLastError());
    if (groups > 1) {
        const unsigned threads = groups <= 64 ? 64u : groups <= 128 ? 128u : 256u;
        hipLaunchKernelGGL(b3::merge_groups, dim3(static_cast<unsigned>(cols)), dim3(threads), 0, c->stream,
                           static_cast<const uint32_t*>(gout), groups, cols, leaves);
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
    const int bits = static_cast<int>(log2_exact(leaves));
    const size_t total = queries * bits;
    hipLaunchKernelGGL(b3::merkle_paths_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0,
                       c->stream, tree, idx, paths, leaves, queries, bits);
    VMX_HIP(c, hipGetLastError());
    return 0;
}

}  // namespace vmx
