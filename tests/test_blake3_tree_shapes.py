"""Multi-chunk BLAKE3 inputs whose chunk count is not a power of two.

The oracle's blake3 (oracle/volta_oracle_blake3.c, restating blake3 1.8.5 of
rust/Cargo.lock:51-53 from the BLAKE3 specification) builds the chunk tree by
recursive splits: the left subtree takes the largest power-of-two number of
chunks smaller than the total.  The reference repository holds no vector for
such counts (its recorded roots have 1, 8 and 512 chunks per column).  This
file pins them with an independent formulation written here: the
specification's incremental hasher, which pushes each finished chunk's
chaining value on a stack and merges while the chunk count is even, in plain
Python integers.  A wrong split point, a misplaced ROOT flag or a wrong chunk
counter in either formulation fails the comparison.  The pure-Python
compression is itself checked against the published digests of "" and "abc".

Column leaves of the commit (ligero.rs:595-616: LE u64 words, row by row) hit
these counts for row counts that are not powers of two times 128, e.g. the
reference's production layer (24,576 rows: 192 chunks per column)."""
import numpy as np
import pytest

IV = [0x6A09E667, 0xBB67AE85, 0x3C6EF372, 0xA54FF53A, 0x510E527F, 0x9B05688C, 0x1F83D9AB, 0x5BE0CD19]
PERM = [2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8]
CHUNK_START, CHUNK_END, PARENT, ROOT = 1, 2, 4, 8
M32 = 0xFFFFFFFF


def _rotr(x, n):
    return ((x >> n) | (x << (32 - n))) & M32


def _g(s, a, b, c, d, mx, my):
    s[a] = (s[a] + s[b] + mx) & M32
    s[d] = _rotr(s[d] ^ s[a], 16)
    s[c] = (s[c] + s[d]) & M32
    s[b] = _rotr(s[b] ^ s[c], 12)
    s[a] = (s[a] + s[b] + my) & M32
    s[d] = _rotr(s[d] ^ s[a], 8)
    s[c] = (s[c] + s[d]) & M32
    s[b] = _rotr(s[b] ^ s[c], 7)


def _compress(cv, words, counter, block_len, flags):
    s = list(cv) + IV[:4] + [counter & M32, (counter >> 32) & M32, block_len, flags]
    m = list(words)
    for r in range(7):
        _g(s, 0, 4, 8, 12, m[0], m[1])
        _g(s, 1, 5, 9, 13, m[2], m[3])
        _g(s, 2, 6, 10, 14, m[4], m[5])
        _g(s, 3, 7, 11, 15, m[6], m[7])
        _g(s, 0, 5, 10, 15, m[8], m[9])
        _g(s, 1, 6, 11, 12, m[10], m[11])
        _g(s, 2, 7, 8, 13, m[12], m[13])
        _g(s, 3, 4, 9, 14, m[14], m[15])
        if r < 6:
            m = [m[i] for i in PERM]
    return [s[i] ^ s[i + 8] for i in range(8)] + [s[i + 8] ^ cv[i] for i in range(8)]


def _words(block: bytes):
    block = block.ljust(64, b"\0")
    return [int.from_bytes(block[4 * i:4 * i + 4], "little") for i in range(16)]


class _Output:
    def __init__(self, cv, words, counter, block_len, flags):
        self.cv, self.words, self.counter, self.block_len, self.flags = cv, words, counter, block_len, flags

    def chaining_value(self):
        return _compress(self.cv, self.words, self.counter, self.block_len, self.flags)[:8]

    def root_bytes(self):
        out = _compress(self.cv, self.words, 0, self.block_len, self.flags | ROOT)[:8]
        return b"".join(w.to_bytes(4, "little") for w in out)


def _chunk_output(data: bytes, counter: int) -> _Output:
    """All blocks of one chunk but the last compressed; the last kept as an
    output (it may become the root)."""
    cv = IV
    blocks = [data[i:i + 64] for i in range(0, len(data), 64)] or [b""]
    for k, blk in enumerate(blocks[:-1]):
        flags = CHUNK_START if k == 0 else 0
        cv = _compress(cv, _words(blk), counter, 64, flags)[:8]
    last = blocks[-1]
    flags = (CHUNK_START if len(blocks) == 1 else 0) | CHUNK_END
    return _Output(cv, _words(last), counter, len(last), flags)


def _parent_output(left, right):
    return _Output(IV, left + right, 0, 64, PARENT)


def blake3_incremental(data: bytes) -> bytes:
    """The specification's hasher: each finished chunk's chaining value goes
    on a stack, merged with the top while the number of chunks so far is
    even; at the end the stack folds into the last chunk's output."""
    stack = []
    chunks = [data[i:i + 1024] for i in range(0, len(data), 1024)] or [b""]
    for counter, chunk in enumerate(chunks[:-1]):
        cv = _chunk_output(chunk, counter).chaining_value()
        total = counter + 1
        while total & 1 == 0:
            cv = _parent_output(stack.pop(), cv).chaining_value()
            total >>= 1
        stack.append(cv)
    out = _chunk_output(chunks[-1], len(chunks) - 1)
    while stack:
        out = _parent_output(stack.pop(), out.chaining_value())
    return out.root_bytes()


def test_incremental_formulation_reproduces_published_digests():
    assert blake3_incremental(b"").hex() == "af1349b9f5f9a1a6a0404dea36dcc9499bcb25c9adc112b7cc9a93cae41f3262"
    assert blake3_incremental(b"abc").hex() == "6437b3ac38465133ffb63b75273a8db548c558465d79db03fd359c6cd5bd9d85"


@pytest.mark.parametrize("length", [1023, 1024, 1025, 2048, 2049, 3072, 3073, 5 * 1024, 6 * 1024 + 7, 7 * 1024,
                                    9 * 1024 - 1, 13 * 1024 + 512, 17 * 1024 + 1, 31 * 1024 + 64])
def test_oracle_blake3_matches_incremental_tree(oracle, length):
    data = bytes((i * 31 + 7) % 251 for i in range(length))
    assert oracle.blake3(data) == blake3_incremental(data)


@pytest.mark.parametrize("rows", [3 * 128, 5 * 128 + 9, 6 * 128, 192 * 128 // 16])
def test_column_leaves_with_uneven_chunk_counts(oracle, rows):
    """Column leaves over rows that give 3, 6 (5 + a partial), 6 and 12
    chunks per column, against the incremental tree of the column bytes."""
    cols = 4
    g = np.random.Generator(np.random.PCG64(rows))
    m = g.integers(0, 0xFFFF_FFFF_0000_0001, size=(rows, cols), dtype=np.uint64)
    leaves = oracle.hash_fp_columns(m, rows, cols)
    for j in range(cols):
        col = b"".join(int(m[r, j]).to_bytes(8, "little") for r in range(rows))
        assert leaves[j].tobytes() == blake3_incremental(col)
