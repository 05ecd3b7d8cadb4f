"""The reference's production commitment layouts, restated in
volta_mi355x/workloads.py, against the values the reference itself asserts
for them (rust/volta-pcs/src/layer_layout.rs):

* one GPT-2 layer: blocks at [0, 3 * 2^22, 2^22, 2^23], 2^24 in all
  (layer_layout.rs:140-141, and the table at :110-117);
* the consolidated weights tree: twelve 2^24 layer blocks, exactly
  C3_WEIGHTS.rows() * C3_WEIGHTS.cols() = 24,576 x 2^13 (:170-177, :30);
* the P5 embedding tree: wte at 0, wpe at 2^26, 2^27 in all (:199-204);
* the exact-block C3 embedding tree: the same offsets, 2^26 + 2^20 =
  C3_EMBED.rows() * C3_EMBED.cols() = 2,080 x 2^15 (:209-214, :34)."""
from volta_mi355x import workloads as W


def test_layer_layout_matches_the_reference_asserts():
    slots, total = W.block_layout(W.GPT2_LAYER_SHAPES)
    assert total == 1 << 24
    assert [s.offset for s in slots] == [0, 3 << 22, 1 << 22, 1 << 23]
    assert [s.stride for s in slots] == [4096, 1024, 4096, 1024]


def test_consolidated_weights_layout():
    slots, total = W.c3_weights_slots()
    assert total == 24576 * (1 << 13)
    assert len(slots) == 48
    assert [s.offset for s in slots[4:8]] == [(1 << 24) + o for o in (0, 3 << 22, 1 << 22, 1 << 23)]
    # every tensor ends inside its own block, and the blocks do not overlap
    spans = sorted((s.offset, s.offset + (s.k - 1) * s.stride + s.n) for s in slots)
    assert all(a[1] <= b[0] for a, b in zip(spans, spans[1:]))
    assert spans[-1][1] <= total
    assert sum(s.k * s.n for s in slots) == 12 * (768 * 4096 + 768 * 768 + 768 * 3072 + 3072 * 768)


def test_embedding_layouts():
    full, total = W.block_layout((("wte", 50257, 768), ("wpe", 1024, 768)))
    assert [s.offset for s in full] == [0, 1 << 26] and total == 1 << 27
    exact, total = W.c3_embed_slots()
    assert [s.offset for s in exact] == [0, 1 << 26] and total == (1 << 26) + (1 << 20) == 2080 * (1 << 15)
    assert [s.stride for s in exact] == [1024, 1024]
