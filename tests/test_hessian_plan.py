"""Host planning of the grouped Hessian launch (mgq_hessian_plan, host code
only: runs without a GPU).

Every plan must cover each lower-triangle 256x256 tile of every group once
per token chunk, with the chunks partitioning the group's token range; a
diagonal tile is covered either alone or in a pair with another diagonal
tile of the same group; split items write each partial slot exactly once
(a pair writes slot and slot + 1) and the split-tile list sums exactly those
slots. Launches of several groups split the groups longer than the average
per-CU load and leave the others whole.
"""

from __future__ import annotations

import ctypes
from collections import defaultdict

import numpy as np
import pytest

TILE = 256
HEADER = np.dtype([("n_items", "<i8"), ("n_split", "<i8"), ("n_slots", "<i8"), ("C", "<i8"),
                   ("n_groups", "<i8"), ("items_off", "<i8"), ("split_off", "<i8"),
                   ("plan_bytes", "<i8"), ("k_end_max", "<i8")])
ITEM = np.dtype([("g", "<i4"), ("ti", "<i4"), ("tj", "<i4"), ("slot", "<i4"), ("k0", "<i8"),
                 ("k1", "<i8")])
SPLIT = np.dtype([("g", "<i4"), ("ti", "<i4"), ("tj", "<i4"), ("slot0", "<i4"), ("nslots", "<i4"),
                  ("stride", "<i4")])


def _lib():
    from mlx_gptq import _native

    if not _native.LIB_PATH.exists():
        pytest.fail(f"{_native.LIB_PATH} not built (python mlx-gptq-mxfp_amd/build.py)")
    return ctypes.CDLL(str(_native.LIB_PATH))


def plan(C: int, offsets, target_items: int = 0):
    lib = _lib()
    off = np.ascontiguousarray(np.asarray(offsets, dtype=np.int64))
    pb, wb = ctypes.c_int64(0), ctypes.c_int64(0)
    args = (ctypes.c_int64(C), ctypes.c_int64(off.size - 1), ctypes.c_void_p(off.ctypes.data),
            ctypes.c_int64(target_items))
    assert lib.mgq_hessian_plan(*args, None, ctypes.c_int64(0), ctypes.byref(pb),
                                ctypes.byref(wb)) == 0
    buf = np.zeros(pb.value, dtype=np.uint8)
    assert lib.mgq_hessian_plan(*args, ctypes.c_void_p(buf.ctypes.data), ctypes.c_int64(pb.value),
                                None, None) == 0
    h = buf[:HEADER.itemsize].view(HEADER)[0]
    items = buf[h["items_off"]:h["items_off"] + h["n_items"] * ITEM.itemsize].view(ITEM)
    split = buf[h["split_off"]:h["split_off"] + h["n_split"] * SPLIT.itemsize].view(SPLIT)
    return h, items, split, wb.value


def check(C: int, offsets, target_items: int = 0):
    h, items, split, ws = plan(C, offsets, target_items)
    nt = -(-C // TILE)
    G = len(offsets) - 1
    assert h["C"] == C and h["n_groups"] == G and h["k_end_max"] == offsets[-1]
    zero_row = -(-2 * C // 256) * 256
    assert ws == h["plan_bytes"] + zero_row + h["n_slots"] * TILE * TILE * 4
    real = items[items["g"] >= 0]
    # coverage: (group, output tile) -> token chunks; diagonal tiles alone or paired
    cover = defaultdict(list)
    writes = defaultdict(int)
    for it in real:
        g, ti, tj, slot, k0, k1 = (int(it[f]) for f in ITEM.names)
        assert 0 <= g < G and 0 <= tj < nt and 0 <= ti < nt
        assert offsets[g] <= k0 <= k1 <= offsets[g + 1]
        outs = [(ti, tj)] if ti > tj else ([(ti, ti), (tj, tj)] if ti < tj else [(ti, ti)])
        for k, t in enumerate(outs):
            cover[(g, t)].append((k0, k1))
            if slot >= 0:
                writes[slot + k] += 1
    for g in range(G):
        for i in range(nt):
            for j in range(i + 1):
                chunks = sorted(cover.pop((g, (i, j)), []))
                assert chunks, (g, i, j)
                assert chunks[0][0] == offsets[g] and chunks[-1][1] == offsets[g + 1]
                assert all(a[1] == b[0] for a, b in zip(chunks, chunks[1:])), chunks
    assert not cover  # nothing outside the lower triangle
    # partial slots: each written once, each summed by exactly one split tile
    assert sorted(writes) == list(range(h["n_slots"])) and set(writes.values()) <= {1}
    summed = []
    for st in split:
        summed += [int(st["slot0"]) + int(st["stride"]) * i for i in range(int(st["nslots"]))]
        assert st["stride"] in (1, 2) and st["ti"] >= st["tj"]
        assert (st["stride"] == 2) == (st["ti"] == st["tj"] and any(
            it["slot"] >= 0 and it["ti"] < it["tj"] and st["ti"] in (it["ti"], it["tj"])
            and it["g"] == st["g"] for it in real))
    assert sorted(summed) == list(range(h["n_slots"]))
    return h, real, split


@pytest.mark.parametrize("C,offsets", [
    (2048, [0, 8192]),              # one group, split: pairs in split mode
    (4096, [0, 32768]),
    (768, [0, 5000]),               # one pair and one odd diagonal tile
    (1000, [0, 300, 9300, 9300, 14300, 14420]),  # ragged C, an empty group
    (264, [0, 10]),
    (96, [0, 5000]),                # one partial tile
    (256, [0, 20000]),
])
def test_plan_covers_every_tile_once(C, offsets):
    check(C, offsets)


def test_plan_explicit_split():
    h, real, split = check(256, [0, 20000], target_items=64)
    assert h["n_split"] >= 1 and h["n_slots"] > 1


def test_direct_groups_pair_their_diagonal_tiles():
    # 128 groups of C = 2048: 32 items per group (28 off-diagonal + 4 pairs)
    n = np.full(128, 8192, dtype=np.int64)
    h, real, split = check(2048, np.concatenate([[0], np.cumsum(n)]).tolist())
    assert h["n_split"] == 0
    per_group = np.bincount(real["g"], minlength=128)
    assert (per_group == 32).all()
    assert int((real["ti"] < real["tj"]).sum()) == 4 * 128 and int((real["ti"] == real["tj"]).sum()) == 0


def test_heavy_groups_are_split_and_light_ones_are_not():
    # C = 768: 5 items per group; one group holds far more than the average
    # per-CU load (tokens x items / 256) and is cut along K, the others not
    n = np.array([4000] * 60 + [60000], dtype=np.int64)
    offsets = np.concatenate([[0], np.cumsum(n)]).tolist()
    h, real, split = check(768, offsets)
    split_groups = set(int(g) for g in real["g"][real["slot"] >= 0])
    assert split_groups == {60}
    avg = int(n.sum()) * 5 // 256
    chunks = real[(real["g"] == 60) & (real["ti"] > real["tj"])]
    assert int((chunks["k1"] - chunks["k0"]).max()) <= max(avg, 4096) + 64
