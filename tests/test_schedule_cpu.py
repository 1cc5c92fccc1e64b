"""The bf16 logits launch's tile schedule, restated on the host and checked
over many shapes: every tile of a tiles_m x vt_total grid runs exactly once,
and the partial last vocabulary column adds at most one tile to the busiest
workgroup.

Restated from the device code (csrc): `xcd_remap` and `grouped_tile`
(flce_device.h), `TileSeq` and `fwd_group` / `fwd_bf16_kernel`
(flce_kernels_bf16.h), `fwd_grid` / `persistent_grid` (flce_capi.hip).
The GPU tests run the kernels themselves on shapes that take each branch
(V below one tile, a 2- and 3-workgroup grid cap, uneven last columns); this
file covers the index arithmetic over shapes no GPU test reaches.
"""
from __future__ import annotations

import itertools

import pytest


def xcd_remap(bid: int, nwg: int) -> int:
    q, r = divmod(nwg, 8)
    x, i = bid % 8, bid // 8
    return x * (q + 1) + i if x < r else r * (q + 1) + (x - r) * q + i


def grouped_tile(lid: int, tiles_m: int, tiles_n: int, group_m: int) -> tuple[int, int]:
    per_group = group_m * tiles_n
    g = lid // per_group
    first_m = g * group_m
    gm = min(group_m, tiles_m - first_m)
    inner = lid - g * per_group
    return first_m + inner % gm, inner // gm


def fwd_group(tiles_m: int) -> int:
    return tiles_m if tiles_m <= 12 else 8


def persistent_grid(tiles: int, cus: int, cap: int = 0) -> int:
    return min(tiles, min(cap, cus) if cap > 0 else cus)


def fwd_grid(tiles_m: int, vt_total: int, tail: bool, cus: int, cap: int = 0) -> int:
    full = tiles_m * (vt_total - (1 if tail else 0))
    return persistent_grid(full, cus, cap) if full > 0 else persistent_grid(tiles_m, cus, cap)


def schedule(tiles_m: int, vt_total: int, tail: bool, P: int) -> list[list[tuple[int, int]]]:
    """Tiles each of the P workgroups runs, in order (fwd_bf16_kernel)."""
    vt_full = vt_total - (1 if tail else 0)
    total = tiles_m * vt_full
    out = []
    for b in range(P):
        first = xcd_remap(b, P)
        mine = []
        if tail:
            r = total % P
            rel = first - r if first >= r else first + P - r
            mine += [(tm, vt_full) for tm in range(rel, tiles_m, P)]
        count = (total - first + P - 1) // P if first < total else 0
        for k in range(count):
            mine.append(grouped_tile(first + k * P, tiles_m, vt_full, fwd_group(tiles_m)))
        out.append(mine)
    return out


def test_xcd_remap_is_a_bijection():
    for nwg in range(1, 300):
        assert sorted(xcd_remap(b, nwg) for b in range(nwg)) == list(range(nwg))


@pytest.mark.parametrize("cus", [256, 2, 3, 8, 37])
def test_every_tile_once_and_tail_balance(cus):
    for tiles_m, vt_total, tail in itertools.product(range(1, 31), (1, 2, 5, 17, 501, 594),
                                                     (False, True)):
        if vt_total == 1 and not tail:
            continue
        P = fwd_grid(tiles_m, vt_total, tail, cus)
        sched = schedule(tiles_m, vt_total, tail, P)
        seen = [t for mine in sched for t in mine]
        assert len(seen) == len(set(seen)) == tiles_m * vt_total, (tiles_m, vt_total, tail, P)
        assert set(seen) == {(m, v) for m in range(tiles_m) for v in range(vt_total)}
        full = tiles_m * (vt_total - (1 if tail else 0))
        base = -(-full // P) if full else 0
        busiest = max(len(mine) for mine in sched)
        # the tail tiles go to the workgroups with one full tile fewer: the
        # busiest one gains a tile only when they outnumber those workgroups
        r = full % P
        spare = P - r if r else 0
        extra = -(-max(tiles_m - spare, 0) // P) if tail else 0
        assert busiest <= base + max(extra, 0 if spare >= tiles_m else 1), (tiles_m, vt_total, P)


def test_grouped_tile_covers_each_group():
    for tiles_m, tiles_n in itertools.product(range(1, 40), (1, 3, 16, 51)):
        g = fwd_group(tiles_m)
        got = {grouped_tile(l, tiles_m, tiles_n, g) for l in range(tiles_m * tiles_n)}
        assert got == {(m, n) for m in range(tiles_m) for n in range(tiles_n)}
