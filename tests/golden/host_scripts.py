"""Call sequences for the loader's host-side entry points.

The layer-coordinate and slot-manager exports (genome / geo) are pure host
bookkeeping whose observable results are fixed by the reference.  The same
functions drive the reference library (in make_golden.py, to record the
fixtures) and the product library (in the tests, to replay them); both
libraries export the same names with the same ctypes signatures.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

GENOME_TOTALS = (-3, 0, 1, 2, 3, 18, 35, 36, 64)
GENOME_BASE_K = (-2, 0, 1, 3, 9)

GEO_ALLOC, GEO_FREE = 0, 1
GEO_K_HINTS = (0, 1, 2, 3, 4, 5, 7, 255)


def genome_table(lib) -> np.ndarray:
    """Rows of (layer, total, base_k, rel, dist, crivo_k, hemisphere)."""
    rows = []
    outs = [C.c_int32() for _ in range(4)]
    for total in GENOME_TOTALS:
        for base_k in GENOME_BASE_K:
            for layer in range(-2, max(total, 1) + 3):
                for o in outs:
                    o.value = -99
                lib.gncx_genome_get_layer_coordinate(layer, total, base_k, *[C.addressof(o) for o in outs])
                rows.append([layer, total, base_k] + [o.value for o in outs])
    return np.array(rows, dtype=np.int32)


def _geo_step(lib, h, op) -> list[int]:
    kind, a, b, c, d = (int(v) for v in op)
    k, dd, r, idx = C.c_uint8(0), C.c_uint8(0), C.c_uint8(0), C.c_uint32(0)
    ret = -1
    if kind == GEO_ALLOC:
        ret = lib.gncx_geo_alloc(h, a, C.addressof(k), C.addressof(dd), C.addressof(r), C.addressof(idx))
    else:
        lib.gncx_geo_free(h, a, b, c, d)
    frag = np.float32(lib.gncx_geo_fragmentation(h)).view(np.uint32)
    return [ret, k.value, dd.value, r.value, idx.value, lib.gncx_geo_used(h), lib.gncx_geo_capacity(h), int(frag)]


def geo_generate(lib, min_frames: int, n_ops: int, seed: int) -> tuple[np.ndarray, np.ndarray]:
    """A random mix of allocations, frees of live slots and frees of
    arbitrary (k, d, R, index) values, run on `lib`; returns (ops, results)."""
    rng = np.random.default_rng(seed)
    h = lib.gncx_geo_mm_create(min_frames)
    live: list[tuple[int, int, int, int]] = []
    ops, res = [], []
    try:
        for _ in range(n_ops):
            u = rng.random()
            if u < 0.6 or not live:
                op = (GEO_ALLOC, int(rng.choice(GEO_K_HINTS)), 0, 0, 0)
            elif u < 0.92:
                k, d, r, idx = live.pop(int(rng.integers(len(live))))
                op = (GEO_FREE, k, d, r, idx)
            else:
                op = (GEO_FREE, int(rng.integers(256)), int(rng.integers(8)), int(rng.integers(8)),
                      int(rng.integers(700)))
            out = _geo_step(lib, h, op)
            if op[0] == GEO_ALLOC and out[0] == 1:
                live.append((out[1], out[2], out[3], out[4]))
            ops.append(op)
            res.append(out)
    finally:
        lib.gncx_geo_mm_destroy(h)
    return np.array(ops, dtype=np.int64), np.array(res, dtype=np.int64)


def geo_replay(lib, min_frames: int, ops: np.ndarray) -> np.ndarray:
    h = lib.gncx_geo_mm_create(min_frames)
    try:
        return np.array([_geo_step(lib, h, op) for op in ops], dtype=np.int64)
    finally:
        lib.gncx_geo_mm_destroy(h)


GEO_CASES = ((0, 120, 1), (1, 200, 2), (64, 300, 3), (72, 400, 4), (130, 500, 5), (512, 900, 6), (600, 900, 7),
             (4294967295, 100, 8))
