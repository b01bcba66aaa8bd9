"""The loader's host-side entry points, on the CPU: the weight-file mapping,
the coloured host buffers, the layer coordinate and the slot manager
(reference cpp:327-686, 2059-2111), and the exports the library does not
provide.  None of them needs a GPU; with one visible, the buffers are
page-locked (covered by the GPU tests)."""
from __future__ import annotations

import ctypes as C
import sys

import numpy as np
import pytest

from conftest import ROOT, gncx, ptr

sys.path.insert(0, str(ROOT / "tests" / "golden"))
import host_scripts  # noqa: E402


@pytest.fixture(scope="module")
def plib():
    lib = gncx.load()
    lib.gncx_hip_last_status()
    return lib


def test_genome_matches_reference_fixture(plib, golden):
    want = golden["genome_table"]
    got = host_scripts.genome_table(plib)
    assert np.array_equal(got, want)
    # the closed form at a few points: 36 layers -> origin 18
    row = {tuple(r[:3]): tuple(r[3:]) for r in got}
    assert row[(0, 36, 3)] == (-18, 18, 4, 1)
    assert row[(18, 36, 3)] == (0, 0, 2, 0)
    assert row[(27, 36, 3)] == (9, 9, 3, 0)
    assert row[(0, 1, 9)] == (0, 0, 4, 0)   # origin 0: base_k clamped to [1, 4]
    assert row[(0, 1, -2)] == (0, 0, 1, 0)


def test_genome_matches_live_reference(plib, ref):
    assert np.array_equal(host_scripts.genome_table(plib), host_scripts.genome_table(ref.lib))


@pytest.mark.parametrize("case", host_scripts.GEO_CASES, ids=lambda c: f"min_frames{c[0]}")
def test_geo_replays_reference_sequence(plib, golden, case):
    mf = case[0]
    ops, want = golden[f"geo_{mf}_ops"], golden[f"geo_{mf}_res"]
    got = host_scripts.geo_replay(plib, mf, ops)
    bad = np.nonzero((got != want).any(axis=1))[0]
    assert bad.size == 0, f"first mismatch at op {bad[0]}: {ops[bad[0]]} -> {got[bad[0]]} vs {want[bad[0]]}"


def test_geo_against_live_reference(plib, ref):
    for mf, n_ops, seed in ((64, 700, 91), (300, 1500, 92)):
        ops, want = host_scripts.geo_generate(ref.lib, mf, n_ops, seed)
        assert np.array_equal(host_scripts.geo_replay(plib, mf, ops), want)


def test_geo_invariants(plib):
    """Capacity is 64 frames per grid (1 to 8 grids); every successful
    allocation is a distinct frame of its grid; a full free restores zero
    use; the streamer's call pattern (k = 2..4 per layer pair) succeeds."""
    for mf, grids in ((0, 1), (64, 1), (65, 2), (512, 8), (10_000, 8)):
        h = plib.gncx_geo_mm_create(mf)
        assert plib.gncx_geo_capacity(h) == 64 * grids
        assert plib.gncx_geo_fragmentation(h) == 0.0
        plib.gncx_geo_mm_destroy(h)
    h = plib.gncx_geo_mm_create(72)
    k, d, r, idx = C.c_uint8(), C.c_uint8(), C.c_uint8(), C.c_uint32()
    seen = []
    for kh in (2, 3, 4, 2, 3, 4, 2, 2):
        assert plib.gncx_geo_alloc(h, kh, C.addressof(k), C.addressof(d), C.addressof(r), C.addressof(idx)) == 1
        assert k.value == kh and r.value == (1, 3, 5, 7)[kh & 3] and d.value < 8
        seen.append((k.value, d.value, r.value, idx.value))
    assert len({s[3] for s in seen}) == len(seen)
    assert plib.gncx_geo_used(h) == len(seen)
    for s in seen:
        plib.gncx_geo_free(h, *s)
    assert plib.gncx_geo_used(h) == 0
    plib.gncx_geo_mm_destroy(h)
    assert plib.gncx_geo_alloc(None, 2, None, None, None, None) == 0
    assert plib.gncx_geo_capacity(None) == 0


def _colour(k, d, r):
    r_odd = (r | 1) & 7
    return (d * r_odd + k) & 7, (d * r_odd * 3 + k * 7) & 63


def test_ram_alloc_colored_places_the_colour(plib):
    handles = []
    try:
        for size in (1, 64, 4096, 1 << 20, (1 << 20) + 1, 5 << 20):
            for k, d, r in ((0, 0, 1), (1, 3, 3), (2, 7, 5), (3, 63, 7), (1, 5, 4), (0, 17, 2)):
                h = plib.gncx_ram_alloc_colored(size, k, d, r)
                assert h
                handles.append(h)
                p = plib.gncx_ram_get_ptr(h)
                bank, l1 = _colour(k, d, r)
                assert p % 64 == 0
                assert (p >> 14) & 7 == bank == plib.gncx_ram_get_ddr3_bank(h)
                assert (p >> 6) & 63 == l1 == plib.gncx_ram_get_l1_set(h)
                buf = (C.c_uint8 * size).from_address(p)
                buf[size - 1], buf[0] = 0x5A, 0xA5    # writable end to end
                assert buf[0] == 0xA5 and buf[size - 1] == (0x5A if size > 1 else 0xA5)
        # above 64 MiB only the L1-set bits are placed (cpp:526-528)
        h = plib.gncx_ram_alloc_colored((64 << 20) + 4096, 2, 7, 5)
        handles.append(h)
        assert (plib.gncx_ram_get_ptr(h) >> 6) & 63 == _colour(2, 7, 5)[1]
    finally:
        for h in handles:
            plib.gncx_ram_free(h)
    assert plib.gncx_ram_get_ptr(None) is None
    plib.gncx_ram_free(None)


def test_ram_alloc_rotates_colours(plib):
    """gncx_ram_alloc's s-th call uses (s mod 4, s mod 64, {1,3,5,7}[s mod 4]);
    the sequence is process-wide, so only its pattern from some s0 is checked."""
    hs = [plib.gncx_ram_alloc(256) for _ in range(12)]
    try:
        got = [(plib.gncx_ram_get_ddr3_bank(h), plib.gncx_ram_get_l1_set(h)) for h in hs]
        matches = [s0 for s0 in range(64)
                   if all(got[i] == _colour((s0 + i) & 3, (s0 + i) & 63, (1, 3, 5, 7)[(s0 + i) & 3])
                          for i in range(12))]
        assert matches, got
        h0 = plib.gncx_ram_alloc(0)   # zero bytes still returns a buffer (of 64)
        assert plib.gncx_ram_get_ptr(h0) is not None
        plib.gncx_ram_free(h0)
    finally:
        for h in hs:
            plib.gncx_ram_free(h)


def test_ram_copy_chunk(plib):
    src = np.arange(1000, dtype=np.uint8)
    h = plib.gncx_ram_alloc_colored(4096, 1, 2, 3)
    try:
        p = plib.gncx_ram_get_ptr(h)
        view = np.ctypeslib.as_array((C.c_uint8 * 4096).from_address(p))
        view[:] = 7
        plib.gncx_ram_copy_chunk(h, 100, ptr(src), 10, 500)
        assert np.array_equal(view[100:600], src[10:510])
        assert (view[:100] == 7).all() and (view[600:] == 7).all()
        plib.gncx_ram_copy_chunk(h, 0, ptr(src), 0, 0)       # no-op
        plib.gncx_ram_copy_chunk(None, 0, ptr(src), 0, 10)   # no-op
    finally:
        plib.gncx_ram_free(h)


def test_gla_map_readonly(plib, tmp_path):
    data = np.random.default_rng(3).integers(0, 256, 3 * 4096 + 17, dtype=np.uint8)
    f = tmp_path / "weights.gguf"
    f.write_bytes(data.tobytes())
    size = C.c_size_t(0)
    h = plib.gncx_gla_map_readonly(str(f).encode(), C.addressof(size))
    assert h and size.value == data.size
    base = plib.gncx_gla_get_base_ptr(h)
    got = np.ctypeslib.as_array((C.c_uint8 * data.size).from_address(base))
    assert np.array_equal(got, data)
    plib.gncx_gla_prefetch_range(base, 4097, 5000)
    plib.gncx_gla_prefetch_range(base, 0, 0)
    plib.gncx_gla_unmap(h)
    assert plib.gncx_gla_map_readonly(str(tmp_path / "absent").encode(), None) is None
    empty = tmp_path / "empty"
    empty.write_bytes(b"")
    assert plib.gncx_gla_map_readonly(str(empty).encode(), None) is None
    assert plib.gncx_gla_get_base_ptr(None) is None
    plib.gncx_gla_unmap(None)


NOT_PROVIDED = [
    ("gncx_lora_init_adapter", lambda o: (ptr(o), ptr(o), 4, 4, 1, 1)),
    ("gncx_lora_forward_add", lambda o: (ptr(o), ptr(o), ptr(o), 4, 4, 1, 1.0, ptr(o))),
    ("gncx_lora_backward_step", lambda o: (ptr(o), ptr(o), ptr(o), ptr(o), ptr(o), 4, 4, 1, 1.0, 0.1, 0.0)),
    ("gncx_mezo_perturb_params", lambda o: (ptr(o), 16, 1, 0.1)),
    ("gncx_mezo_update_params", lambda o: (ptr(o), 16, 1, 0.5, 0.1, 0.0)),
    ("gncx_cross_entropy_loss", lambda o: (ptr(o), 16, 3, ptr(o))),
    ("gncx_project_layer_3d_point", lambda o: (1, 4, None, ptr(o), 16, ptr(o))),
    ("gncx_cosine_similarity", lambda o: (ptr(o), ptr(o), 16)),
    ("gncx_vector_l2_normalize", lambda o: (ptr(o), 16)),
    ("gncx_mean_pooling", lambda o: (ptr(o), 2, 8, ptr(o))),
    ("gncx_bidirectional_attention_gqa", lambda o: (ptr(o), ptr(o), ptr(o), 1, 2, 1, 8, 0.3, ptr(o))),
    ("gncx_bidirectional_attention", lambda o: (ptr(o), ptr(o), ptr(o), 1, 2, 8, 0.3, ptr(o))),
]


@pytest.mark.parametrize("name,args", NOT_PROVIDED, ids=[n for n, _ in NOT_PROVIDED])
def test_not_provided_exports_fail_loudly(plib, name, args):
    o = np.full(64, 3.0, dtype=np.float32)
    plib.gncx_hip_last_status()
    r = getattr(plib, name)(*args(o))
    assert plib.gncx_hip_last_status() != 0
    assert (o == 3.0).all(), "outputs must be left untouched"
    if r is not None:
        assert r == 0.0
