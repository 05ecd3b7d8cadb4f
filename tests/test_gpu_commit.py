"""End-to-end resident commitment and opening through the C ABI, against the
oracle's CPU commit (commit_impl, rust/volta-pcs/src/ligero.rs:543-624).

These follow the reference's drop-in acceptance tests
(rust/volta-pcs/tests/cuda.rs:186-497): strided device placements of
several tensors, the device chain pads -> messages -> NTT -> BLAKE3 tree ->
root equal to the CPU root, the exact stats of a cold commit
(tests/cuda.rs:228-244, 381-441), overlap and alignment rejection, no leaked
memory, and every device step of the resident opening
(ligero.rs:1216-1551) equal to the same steps composed from the oracle."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

P = 0xFFFF_FFFF_0000_0001


def packed_from(params_rows, cols, tensors):
    """Host restatement of the placements: zero target, tensor row r at
    offset + r * stride (ligero.rs:439-451)."""
    packed = np.zeros(params_rows * cols, np.int16)
    for t, off, stride in tensors:
        for r in range(t.shape[0]):
            packed[off + r * stride:off + r * stride + t.shape[1]] = t[r]
    return packed


def commit_on_device(b, params, tensors, seed, fused):
    """Upload every tensor into one source buffer with gaps (the reference's
    DeviceSlice sources), then place them and commit."""
    from volta_mi355x import ligero
    gap = 5
    offsets, parts, pos = [], [], gap
    for t, _, _ in tensors:
        offsets.append(pos)
        parts.append(np.full(gap, -901, np.int16) if not parts else np.full(gap, -903, np.int16))
        parts.append(t.reshape(-1))
        pos += t.size + gap
    parts.append(np.full(gap, -907, np.int16))
    source = b.upload_device(np.concatenate(parts))
    placements = [ligero.ResidentWeightPlacement(source, so, t.shape[0], t.shape[1], off, stride,
                                                 params.rows * params.cols)
                  for (t, off, stride), so in zip(tensors, offsets)]
    b.reset_stats()
    root, pm = ligero.commit_resident_from_device(b, placements, params, seed, fused=fused)
    stats = b.get_stats()
    return source, placements, root, pm, stats


@pytest.mark.parametrize("fused", [False, True])
def test_device_placements_commit_to_the_cpu_root(oracle, fused):
    """tests/cuda.rs:381-497: two tensors (3x3 at stride 4, 2x2 at stride 2
    from offset 32) into an 8 x 8 matrix, pad 2, code length 16."""
    from volta_mi355x import Backend, InvalidInput, ligero
    params = ligero.LigeroParams(rows=8, col_bits=3, pad=2, code_bits=4, n_queries=2)
    a = np.arange(1, 10, dtype=np.int16).reshape(3, 3)
    bt = np.arange(101, 105, dtype=np.int16).reshape(2, 2)
    tensors = [(a, 0, 4), (bt, 32, 2)]
    packed = packed_from(params.rows, params.cols, tensors)
    seed = bytes([0x79] * 32)
    with Backend() as b:
        base = b.memory_breakdown()[1]
        source, (pa, pb), root, pm, s = commit_on_device(b, params, tensors, seed, fused)
        assert root == oracle.commit_root(packed, params.rows, params.cols, params.pad, params.code_len, seed)
        assert s["h2d_bytes"] == params.code_len // 2 * 8
        assert s["d2d_bytes"] == (a.size + bt.size) * 2
        assert s["device_zeroed_bytes"] == packed.size * 2
        assert s["device_generated_bytes"] == params.rows * params.pad * 8
        assert s["d2h_bytes"] == 32
        assert s["calls"]["pcs_ntt"] == 1 and s["calls"]["pcs_merkle"] == 1 and s["calls"]["pcs_rows"] > 0
        # overlap and geometry rejection allocate nothing
        over = ligero.ResidentWeightPlacement(source, pb.source_offset, 2, 2, 8, 2, packed.size)
        live = b.memory_breakdown()[1]
        with pytest.raises(InvalidInput, match="overlap"):
            ligero.commit_resident_from_device(b, [pa, over], params, seed)
        assert b.memory_breakdown()[1] == live
        with pytest.raises(InvalidInput, match="not aligned"):
            ligero.ResidentWeightPlacement(source, pb.source_offset, 2, 2, 1, 2, packed.size)
        with pytest.raises(InvalidInput, match="exceeds packed target"):
            ligero.ResidentWeightPlacement(source, pb.source_offset, 2, 2, packed.size, 2, packed.size)
        with pytest.raises(InvalidInput, match="wrong PCS geometry"):
            ligero.commit_resident_from_device(
                b, [ligero.ResidentWeightPlacement(source, 0, 2, 2, 0, 2, 2 * packed.size)], params, seed)
        ligero.free_resident_matrix(b, pm)
        b.free_device(source)
        assert b.memory_breakdown()[1] == base


# Production-size layouts: the pass engine and the n = 2^13 paths build their
# tables on the device, so a cold commit still uploads exactly n/2 words.
LAYOUTS = [
    # rows, col_bits, pad, code_bits, tensors (rows, cols, offset, stride)
    (256, 11, 512, 13, [(100, 1500, 0, 2048), (50, 700, 262144, 1024), (7, 300, 327680, 512)]),
    (64, 13, 512, 15, [(30, 8000, 0, 8192), (30, 3000, 393216, 4096)]),
    (8, 15, 512, 17, [(3, 32768, 0, 32768), (3, 1000, 196608, 1024)]),
]


@pytest.mark.parametrize("rows,col_bits,pad,code_bits,shapes", LAYOUTS)
@pytest.mark.parametrize("fused", [False, True])
def test_production_layout_commit_root_and_stats(oracle, rows, col_bits, pad, code_bits, shapes, fused):
    from volta_mi355x import Backend, ligero
    params = ligero.LigeroParams(rows=rows, col_bits=col_bits, pad=pad, code_bits=code_bits)
    g = np.random.Generator(np.random.PCG64(rows * code_bits))
    tensors = [(g.integers(-(1 << 15), 1 << 15, size=(r, c), dtype=np.int16), off, st) for r, c, off, st in shapes]
    for t, _, _ in tensors:
        t.reshape(-1)[:2] = [-32768, 32767]
    packed = packed_from(rows, params.cols, tensors)
    seed = bytes(range(32))
    with Backend() as b:
        base = b.memory_breakdown()[1]
        source, _, root, pm, s = commit_on_device(b, params, tensors, seed, fused)
        want_root, want_enc, want_pads = oracle.commit_root(packed, rows, params.cols, pad, params.code_len, seed,
                                                            keep=True)
        if root != want_root:  # name the first differing row before failing
            got = b.download_device(pm.encoded).reshape(rows, params.code_len)
            bad = np.nonzero((got != want_enc).any(axis=1))[0]
            raise AssertionError(f"root differs; first differing encoded rows {bad[:8].tolist()}")
        assert s["h2d_bytes"] == params.code_len // 2 * 8
        assert s["d2d_bytes"] == sum(t.size for t, _, _ in tensors) * 2
        assert s["device_zeroed_bytes"] == packed.size * 2
        assert s["device_generated_bytes"] == rows * pad * 8
        assert s["d2h_bytes"] == 32
        assert (b.download_device(pm.pads).reshape(rows, pad) == want_pads).all()
        ligero.free_resident_matrix(b, pm)
        b.free_device(source)
        assert b.memory_breakdown()[1] == base


def oracle_opening(oracle, packed, params, enc, pads, claims, c, js, mask_seed):
    """The device steps of open_multi_zk_resident (ligero.rs:1216-1551)
    composed from oracle functions."""
    rows, cols, msg_len, n, cb = params.rows, params.cols, params.msg_len, params.code_len, params.col_bits
    g_count = len(claims)
    mask_rows = g_count + 1
    masks = oracle.fp2_rows_padded(mask_seed, 0, mask_rows, msg_len, n)  # (mask_rows, n, 2)
    compact = masks[:, :msg_len]
    menc = np.stack([oracle.ntt_forward_batch(masks[:, :, k].copy()) for k in (0, 1)], axis=-1)
    mtree = oracle.merkle_tree(oracle.hash_fp2_columns(menc, mask_rows, n))
    tree = oracle.merkle_tree(oracle.hash_fp_columns(enc, rows, n))
    u_c = oracle.pcs_combine_rows(packed, pads, oracle.fp2_powers(c, rows), rows, cols, params.pad, 1)[0]
    u_c = oracle.fp2_add_inplace(u_c, compact[0])
    co = np.zeros((g_count * rows, 2), np.uint64)
    for g, (off, pt) in enumerate(claims):
        eq = oracle.eq_rows(pt[cb:], 1, len(pt) - cb).reshape(-1, 2)
        row0 = off >> cb
        co[g * rows + row0:g * rows + row0 + eq.shape[0]] = eq
    u_gs = oracle.pcs_combine_rows(packed, pads, co, rows, cols, params.pad, g_count)
    u_gs = np.stack([oracle.fp2_add_inplace(u_gs[g], compact[1 + g]) for g in range(g_count)])
    qeq = np.concatenate([oracle.eq_rows(pt[:cb], 1, cb).reshape(-1, 2) for _, pt in claims])
    s_vals = oracle.fp2_row_dots(compact[1:].reshape(-1, 2), msg_len, qeq, cols, g_count, cols)
    idx = np.asarray(js, np.uint32)
    return {
        "mask_root": mtree[-1].tobytes(),
        "u_c": u_c, "u_gs": u_gs, "s_values": s_vals,
        "data_columns": oracle.gather_columns(enc, idx),
        "mask_columns": oracle.gather_fp2_columns(menc, idx),
        "data_paths": oracle.merkle_paths(tree, n, idx),
        "mask_paths": oracle.merkle_paths(mtree, n, idx),
    }


OPEN_CASES = [
    # rows, col_bits, pad, code_bits, claims as (row0, row_bits), queries
    (8, 3, 2, 4, [(0, 3), (4, 2), (6, 1)], 3),
    (64, 11, 512, 13, [(0, 2), (8, 3), (63, 0)], 7),
    (32, 13, 512, 15, [(16, 4), (0, 1)], 5),
]


@pytest.mark.parametrize("rows,col_bits,pad,code_bits,claim_rows,queries", OPEN_CASES)
def test_resident_opening_steps_match_oracle(backend, oracle, rows, col_bits, pad, code_bits, claim_rows,
                                             queries):
    """Mask rows and their Fp2 NTT at the code length (rows = claims + 1),
    the mask tree, u_c, the block-claim combinations, the mask dots, gathers
    and paths, each bit-exact against the oracle."""
    from volta_mi355x import ligero
    params = ligero.LigeroParams(rows=rows, col_bits=col_bits, pad=pad, code_bits=code_bits)
    g = np.random.Generator(np.random.PCG64(rows + code_bits))
    packed = g.integers(-(1 << 15), 1 << 15, size=rows * params.cols, dtype=np.int16)
    seed, mask_seed = bytes([0x71] * 32), bytes([0x75] * 32)
    src = backend.upload_device(packed)
    root, pm = ligero.commit_resident_from_device(
        backend, [ligero.ResidentWeightPlacement(src, 0, rows, params.cols, 0, params.cols, packed.size)],
        params, seed)
    backend.free_device(src)
    try:
        want_root, enc, pads = oracle.commit_root(packed, rows, params.cols, pad, params.code_len, seed, keep=True)
        assert root == want_root
        claims = [((r0 << col_bits), g.integers(0, P, size=(col_bits + rb, 2), dtype=np.uint64))
                  for r0, rb in claim_rows]
        c = tuple(int(x) for x in g.integers(0, P, size=2, dtype=np.uint64))
        js = g.integers(0, params.code_len, size=queries, dtype=np.uint32)
        got = ligero.open_rows_resident(backend, pm, claims, c, js, mask_seed)
        want = oracle_opening(oracle, packed, params, enc, pads.reshape(-1), claims, c, js, mask_seed)
        for k, v in want.items():
            if isinstance(v, bytes):
                assert got[k] == v, k
            else:
                assert np.array_equal(np.asarray(got[k]), np.asarray(v)), k
    finally:
        ligero.free_resident_matrix(backend, pm)


@pytest.mark.parametrize("name", ["embed", "weights"])
def test_reference_production_commitments(oracle, name):
    """C3_EMBED (2 tensors) and C3_WEIGHTS (48 tensors) in the reference's own
    layouts, committed as its report commits them (p6_report.rs:2584-2615,
    2929-2952): each tensor a resident buffer, one strided placement per
    tensor, pad 512, the seeds 0x51/0x52.  The root equals the oracle's CPU
    commit of the packed matrix, and the stats carry exactly the placements'
    bytes."""
    from volta_mi355x import Backend, ligero, workloads as W
    slots, total = W.c3_weights_slots() if name == "weights" else W.c3_embed_slots()
    rows, col_bits, code_bits = (24576, 13, 15) if name == "weights" else (2080, 15, 17)
    params = ligero.LigeroParams(rows=rows, col_bits=col_bits, pad=512, code_bits=code_bits)
    seed = bytes([0x51 if name == "weights" else 0x52]) * 32
    g = np.random.Generator(np.random.PCG64(rows))
    tensors = [g.integers(-(1 << 15), 1 << 15, size=(s.k, s.n), dtype=np.int16) for s in slots]
    tensors[0].reshape(-1)[:2] = [-32768, 32767]
    packed = np.zeros(total, np.int16)
    for t, s in zip(tensors, slots):
        packed[s.offset:s.offset + s.k * s.stride].reshape(s.k, s.stride)[:, :s.n] = t
    with Backend() as b:
        base = b.memory_breakdown()[1]
        sources = [b.upload_device(t.reshape(-1)) for t in tensors]
        placements = [ligero.ResidentWeightPlacement(src, 0, s.k, s.n, s.offset, s.stride, total)
                      for src, s in zip(sources, slots)]
        b.reset_stats()
        root, pm = ligero.commit_resident_from_device(b, placements, params, seed)
        st = b.get_stats()
        ligero.free_resident_matrix(b, pm)
        for src in sources:
            b.free_device(src)
        assert b.memory_breakdown()[1] == base
    del tensors
    assert st["d2d_bytes"] == sum(s.k * s.n for s in slots) * 2
    assert st["device_zeroed_bytes"] == total * 2
    assert st["device_generated_bytes"] == rows * 512 * 8
    assert root == oracle.commit_root(packed, rows, params.cols, 512, params.code_len, seed)
