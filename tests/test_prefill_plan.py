"""Key-piece planning of the prefill entry points, on the host (no GPU): which
chunks are cut, into how many pieces, and the piece map of the batched launch.
The library sizes the plan for 256 CUs when no GPU is present (512 workgroup
slots, two per CU)."""
import numpy as np
import pytest

import atomflow_amd
from atomflow_amd import kv

NQ = 24
COUNTERS = 64 * 1024
REC = 128 * 128 * 4 + 2 * 128 * 4  # one piece's o and (m, l) records


def lib():
    return atomflow_amd.lib()


def test_workspace_size_follows_the_cut_rule():
    # 4 tiles x 24 heads = 96 workgroups: cut; key tiles 98..104 per tile over
    # ceil(9696 / 512) = 19 per piece -> 4 pieces (the cap)
    nbytes = lib().af_prefill_workspace_size(6144, 512, 6656, NQ, 0)
    assert nbytes >= COUNTERS + 4 * NQ * 4 * REC
    # key_pieces = 1, or a grid that fills the device (32 tiles x 24 heads): no records
    assert lib().af_prefill_workspace_size(6144, 512, 6656, NQ, 1) == COUNTERS
    assert lib().af_prefill_workspace_size(0, 4096, 4096, NQ, 0) == COUNTERS
    # too little work per tile (a 200-token prompt: at most 4 key tiles, 12 per piece)
    assert lib().af_prefill_workspace_size(0, 200, 200, NQ, 0) == COUNTERS
    # a cap of 2 pieces sizes for 2
    two = lib().af_prefill_workspace_size(6144, 512, 6656, NQ, 2)
    assert COUNTERS + 4 * NQ * 2 * REC <= two < nbytes
    # bad arguments
    assert lib().af_prefill_workspace_size(0, 512, 512, NQ, 5) == 0
    assert lib().af_prefill_workspace_size(-1, 512, 512, NQ, 0) == 0


def test_piece_map_covers_every_piece_heaviest_first():
    chunks = [(3000, 300, 3300, 0), (0, 300, 300, 300), (1000, 100, 1100, 600), (0, 1, 1, 700),
              (2000, 200, 2150, 701)]
    pmap, groups, most, nbytes = kv.prefill_piece_map(chunks, NQ, 0)
    tiles = [(c, t) for c, (_, n, _, _) in enumerate(chunks) for t in range((n + 127) // 128)]
    assert groups == len(tiles) == 10
    assert 1 < most <= 4
    assert nbytes >= COUNTERS + groups * NQ * most * REC
    pieces = {}
    for c, t, pp, g in pmap:
        p, n = int(pp) & 0xff, int(pp) >> 8
        assert 0 <= p < n <= most
        assert tiles[g] == (c, t)  # the record group is the tile's index
        pieces.setdefault((int(c), int(t)), set()).add(p)
        assert pieces[(int(c), int(t))] <= set(range(n))
    assert set(pieces) == set(tiles)
    for (c, t), ps in pieces.items():
        assert ps == set(range(len(ps)))  # every piece of a tile once
    # heaviest piece first: the piece's key tiles never grow along the map
    def units(c, t):
        p0, n, kvl, _ = chunks[c]
        return -(-min(p0 + min((t + 1) * 128, n), kvl) // 64)
    work = [units(int(c), int(t)) / (int(pp) >> 8) for c, t, pp, _ in pmap]
    assert all(a >= b for a, b in zip(work, work[1:]))
    # the first chunk's tiles (49..52 key tiles) are cut; the one-token chunk is not
    assert len(pieces[(0, 0)]) > 1 and len(pieces[(3, 0)]) == 1


def test_piece_map_without_cuts_matches_tile_map():
    chunks = [(0, 300, 300, 0), (1000, 100, 1100, 300)]
    pmap, groups, most, nbytes = kv.prefill_piece_map(chunks, NQ, 1)
    tmap = kv.prefill_tile_map(chunks)
    assert most == 1 and nbytes == COUNTERS
    assert [(int(c), int(t)) for c, t, _, _ in pmap] == [tuple(map(int, x)) for x in tmap]
    # a launch whose tiles fill the device is not cut either
    big = [(0, 4096, 4096, 0)]
    pmap, groups, most, nbytes = kv.prefill_piece_map(big, NQ, 0)
    assert most == 1 and len(pmap) == 32


def test_piece_map_errors():
    chunks = np.array([[3000, 300, 3300, 0]], np.int32)
    out = np.zeros((2, 4), np.int32)
    import ctypes
    g, m, nb = ctypes.c_int(), ctypes.c_int(), ctypes.c_size_t()
    st = lib().af_prefill_piece_map(chunks.ctypes.data, 1, NQ, 0, out.ctypes.data, 2,
                                    ctypes.byref(g), ctypes.byref(m), ctypes.byref(nb))
    assert st == atomflow_amd.AF_ERR_WORKSPACE  # more entries than max_entries
    st = lib().af_prefill_piece_map(chunks.ctypes.data, 1, NQ, 9, out.ctypes.data, 2,
                                    ctypes.byref(g), ctypes.byref(m), ctypes.byref(nb))
    assert st == atomflow_amd.AF_ERR_INVALID_ARG
    with pytest.raises(atomflow_amd.AfError):
        kv.prefill_piece_map([(-1, 10, 10, 0)], NQ)
