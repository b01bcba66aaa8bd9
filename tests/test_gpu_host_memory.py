"""GPU side of the loader's host-side entry points: GeGLU against the
reference's vectors, and weights / KV caches held in the library's host
buffers and file mappings, whose device copies must follow the host
memory through gncx_ram_copy_chunk, gncx_ram_free and gncx_gla_unmap."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import synth
from conftest import gncx, ptr, rel_l2

pytestmark = pytest.mark.gpu

Q4_K = 12
TOL = 1e-3  # relative L2 of fp32 matvec / attention outputs


def test_geglu_matches_reference(lib, golden, oracle):
    g, u = golden["geg_g"].copy(), golden["geg_u"].copy()
    out = np.zeros_like(g)
    lib.gncx_geglu_activation(ptr(g), ptr(u), g.size, ptr(out))
    gncx.check(lib)
    assert rel_l2(out, golden["geg_y"]) < 1e-6
    assert rel_l2(out, oracle.geglu(g, u)) < 1e-6
    assert out[7] == 0.0                               # GELU(0) = 0
    sat = np.abs(g) >= 10.0                            # tanh saturated: x * u above, 0 below
    assert np.allclose(out[sat & (g > 0)], (g * u)[sat & (g > 0)], rtol=1e-6, atol=0)
    assert np.all(np.abs(out[sat & (g < 0)]) < 1e-6)


def _changed_weights(w: np.ndarray) -> np.ndarray:
    """w with the super-block scales of its second half doubled or halved
    (one exponent bit of each Q4_K block's fp16 d) wherever the host-weight
    content signature does not sample (16 probes of 8 bytes at
    (nbytes - 8) * i / 15), so only the explicit drop of the device copy can
    make the change visible."""
    covered = set()
    for i in range(16):
        o = (w.size - 8) * i // 15
        covered.update(range(o, o + 8))
    w2 = w.copy()
    for p in range(w.size // 2, w.size):
        if p % 144 == 1 and p not in covered:
            w2[p] ^= 0x04
    assert all(w2[p] == w[p] for p in covered)
    return w2


def test_weights_in_ram_buffer_follow_copy_chunk(lib, oracle):
    k, n = 2048, 96
    w = synth.make_weights(Q4_K, n, k, seed=41)
    w2 = _changed_weights(w)
    x = synth.make_activations(1, k, seed=42)
    want1, want2 = oracle.matvec(Q4_K, w, x, k, n), oracle.matvec(Q4_K, w2, x, k, n)
    assert rel_l2(want1, want2) > 20 * TOL  # the planted change is visible in the result
    off = 4096 + 64
    h = lib.gncx_ram_alloc_colored(off + w.size, 1, 3, 3)
    assert h
    try:
        base = lib.gncx_ram_get_ptr(h)
        y = np.zeros(n, np.float32)
        lib.gncx_ram_copy_chunk(h, off, ptr(w), 0, w.size)
        lib.gncx_xfold_universal_matvec(base, off, Q4_K, ptr(x), None, k, n, ptr(y), None)
        gncx.check(lib)
        assert rel_l2(y, want1) < TOL
        lib.gncx_ram_copy_chunk(h, off, ptr(w2), 0, w2.size)
        lib.gncx_xfold_universal_matvec(base, off, Q4_K, ptr(x), None, k, n, ptr(y), None)
        gncx.check(lib)
        assert rel_l2(y, want2) < TOL
    finally:
        lib.gncx_ram_free(h)


def test_weights_in_ram_buffer_rewritten_by_plain_stores(lib, oracle):
    """A gncx_ram buffer is writable memory: weights rewritten there with plain
    stores (not gncx_ram_copy_chunk) are found changed by the content
    signature, as for any host memory.  A rewrite that touches none of the
    signature's probes is the caller's to announce with
    gncx_hip_weight_forget (weights are immutable in the reference's
    contract), after which the new bytes are used."""
    k, n = 2048, 96
    w = synth.make_weights(Q4_K, n, k, seed=43)
    w2 = synth.make_weights(Q4_K, n, k, seed=44)
    w3 = _changed_weights(w2)
    x = synth.make_activations(1, k, seed=45)
    want = [oracle.matvec(Q4_K, v, x, k, n) for v in (w, w2, w3)]
    assert rel_l2(want[1], want[2]) > 20 * TOL
    off = 4096 + 32
    h = lib.gncx_ram_alloc_colored(off + w.size, 2, 4, 3)
    assert h
    try:
        base = lib.gncx_ram_get_ptr(h)
        view = np.ctypeslib.as_array((C.c_uint8 * (off + w.size)).from_address(base))
        y = np.zeros(n, np.float32)
        for i, v in enumerate((w, w2)):
            view[off:off + v.size] = v  # plain stores into the buffer
            lib.gncx_xfold_universal_matvec(base, off, Q4_K, ptr(x), None, k, n, ptr(y), None)
            gncx.check(lib)
            assert rel_l2(y, want[i]) < TOL, i
        view[off:off + w3.size] = w3
        lib.gncx_hip_weight_forget(base + off)
        lib.gncx_xfold_universal_matvec(base, off, Q4_K, ptr(x), None, k, n, ptr(y), None)
        gncx.check(lib)
        assert rel_l2(y, want[2]) < TOL
    finally:
        lib.gncx_ram_free(h)


def test_weights_in_mapped_file_are_dropped_on_unmap(lib, oracle, tmp_path):
    k, n = 2048, 64
    w = synth.make_weights(Q4_K, n, k, seed=43)
    x = synth.make_activations(1, k, seed=44)
    off = 32
    w2 = _changed_weights(w)
    assert rel_l2(oracle.matvec(Q4_K, w, x, k, n), oracle.matvec(Q4_K, w2, x, k, n)) > 20 * TOL
    for i, ww in enumerate((w, w2)):
        f = tmp_path / f"model{i}.gguf"
        f.write_bytes(b"\0" * off + ww.tobytes())
        size = C.c_size_t(0)
        h = lib.gncx_gla_map_readonly(str(f).encode(), C.addressof(size))
        assert h and size.value == off + ww.size
        y = np.zeros(n, np.float32)
        lib.gncx_xfold_universal_matvec(lib.gncx_gla_get_base_ptr(h), off, Q4_K, ptr(x), None, k, n, ptr(y), None)
        gncx.check(lib)
        assert rel_l2(y, oracle.matvec(Q4_K, ww, x, k, n)) < TOL
        lib.gncx_gla_unmap(h)


def test_kv_cache_in_ram_buffers_is_dropped_on_free(lib, oracle):
    """Decode steps into caches held in ram buffers, the buffers freed and
    new ones filled with other rows, row 0 equal to the old buffers' final
    row 0 (the row the device copy's staleness check compares): the next
    steps must see the new rows."""
    H, KV, hd, rows = 8, 2, 64, 16
    kvd = KV * hd
    scale = 1.0 / np.sqrt(hd)
    rng = np.random.default_rng(45)
    nbytes = rows * kvd * 4
    first = {}
    for rnd in range(2):
        hk = lib.gncx_ram_alloc_colored(nbytes, 2, 5, 5)
        hv = lib.gncx_ram_alloc_colored(nbytes, 3, 6, 7)
        try:
            kc = np.ctypeslib.as_array((C.c_float * (rows * kvd)).from_address(lib.gncx_ram_get_ptr(hk)))
            vc = np.ctypeslib.as_array((C.c_float * (rows * kvd)).from_address(lib.gncx_ram_get_ptr(hv)))
            kc[:] = rng.standard_normal(kc.size).astype(np.float32)
            vc[:] = rng.standard_normal(vc.size).astype(np.float32)
            if rnd == 1:
                kc[:kvd], vc[:kvd] = first["k0"], first["v0"]
            start = 0 if rnd == 0 else 5
            for pos in range(start, start + 5):
                q = rng.standard_normal(H * hd).astype(np.float32)
                kn = rng.standard_normal(kvd).astype(np.float32)
                vn = rng.standard_normal(kvd).astype(np.float32)
                want, _, _ = oracle.attention(q, kn, vn, kc.reshape(rows, kvd).copy(), vc.reshape(rows, kvd).copy(),
                                              pos, H, KV, hd, scale, 0, 1)
                out = np.zeros(H * hd, np.float32)
                lib.gncx_mqa_attention_step_ext(ptr(q), ptr(kn), ptr(vn), kc.ctypes.data, vc.ctypes.data, pos, H,
                                                KV, hd, scale, 0, 1, ptr(out))
                gncx.check(lib)
                assert rel_l2(out, want) < TOL, (rnd, pos)
                assert np.array_equal(kc[pos * kvd:(pos + 1) * kvd], kn)
            first = {"k0": kc[:kvd].copy(), "v0": vc[:kvd].copy()}
        finally:
            lib.gncx_ram_free(hk)
            lib.gncx_ram_free(hv)
