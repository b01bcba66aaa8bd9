"""GPU: gncx_hip_decode_step_noalloc, the decode step that allocates nothing
(its scratch is a fixed device array per GPU), against gncx_hip_decode_step
through the C-ABI: logits, greedy tokens and KV caches bit for bit on two calls
in a row, the second at a smaller position (a smaller attention window, so a
smaller share of the scratch); free device memory unchanged across its calls;
a step that needs more scratch than the array holds is rejected before
anything is enqueued."""
from __future__ import annotations

import ctypes as C

import pytest

from conftest import gncx

pytestmark = pytest.mark.gpu


def _mem_free() -> int:
    hip = C.CDLL("libamdhip64.so")
    free, total = C.c_size_t(), C.c_size_t()
    assert hip.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


def _noalloc(lib, d, token, pos, greedy):
    if d._native is None:
        d._native_structs()
    _, model, _, _, state = d._native
    return lib.gncx_hip_decode_step_noalloc(C.byref(model), C.byref(state), int(token), int(pos), int(greedy))


def test_noalloc_step_equals_decode_step(lib, torch_mod):
    import gncx_amd.decode as dec

    torch = torch_mod
    shape = dec.Qwen3Shape(n_layers=2, embed=256, n_heads=4, n_kv=2, head_dim=64, ffn=512, vocab=600)
    model = dec.build_model(torch, shape, seed=31)
    a = dec.Decoder(lib, torch, model, max_seq=64, fused=True, native=True)
    b = dec.Decoder(lib, torch, model, max_seq=64, fused=True, native=True)
    toks = [3, 599, 17, 250, 0, 42, 511, 7, 9, 123]
    # identical caches on both sides: positions 0 .. 39 through the regular step
    for pos in range(40):
        for d in (a, b):
            d._step(toks[pos % len(toks)], pos, False)
    torch.cuda.synchronize()
    gncx.check(lib)
    # warm-up of the no-allocation path
    assert _noalloc(lib, b, 5, 40, 1) == 0, lib.gncx_hip_last_error().decode()
    a._step(5, 40, True)
    torch.cuda.synchronize()
    for pos, tok, greedy in ((41, 77, 1), (7, 300, 1)):  # the second call at a smaller position
        a._step(tok, pos, bool(greedy))
        torch.cuda.synchronize()
        # free device memory around the no-allocation call alone (torch's
        # comparisons below allocate through its own caching allocator)
        free0 = _mem_free()
        rc = _noalloc(lib, b, tok, pos, greedy)
        assert rc == 0, lib.gncx_hip_last_error().decode()
        torch.cuda.synchronize()
        assert _mem_free() == free0, pos
        assert torch.equal(a.logits, b.logits), (pos, (a.logits - b.logits).abs().max().item())
        assert torch.equal(a.token_dev, b.token_dev), pos
        assert torch.equal(a.token_log, b.token_log), pos
        for l in range(shape.n_layers):
            assert torch.equal(a.kc[l], b.kc[l]) and torch.equal(a.vc[l], b.vc[l]), (pos, l)
        print(f"noalloc pos={pos} token={int(b.token_dev.item())} logits equal", flush=True)
    gncx.check(lib)


def test_noalloc_first_call_on_fresh_model(lib, torch_mod):
    """The first call of a model and state the library has not seen (its plan
    is built inside that call) allocates nothing either, and equals the
    regular step.  A regular step on another model runs first, so every kernel
    has been launched once (the runtime loads code objects on first use)."""
    import gncx_amd.decode as dec

    torch = torch_mod
    warm_shape = dec.Qwen3Shape(n_layers=1, embed=256, n_heads=4, n_kv=2, head_dim=64, ffn=512, vocab=600)
    w = dec.Decoder(lib, torch, dec.build_model(torch, warm_shape, seed=40), max_seq=16, fused=True, native=True)
    w._step(1, 0, True)
    torch.cuda.synchronize()
    gncx.check(lib)
    shape = dec.Qwen3Shape(n_layers=3, embed=256, n_heads=8, n_kv=2, head_dim=64, ffn=512, vocab=700)
    model = dec.build_model(torch, shape, seed=41)
    a = dec.Decoder(lib, torch, model, max_seq=16, fused=True, native=True)
    b = dec.Decoder(lib, torch, model, max_seq=16, fused=True, native=True)
    b._native_structs()
    torch.cuda.synchronize()
    free0 = _mem_free()
    rc = _noalloc(lib, b, 123, 0, 1)
    assert rc == 0, lib.gncx_hip_last_error().decode()
    torch.cuda.synchronize()
    assert _mem_free() == free0
    a._step(123, 0, True)
    torch.cuda.synchronize()
    gncx.check(lib)
    assert torch.equal(a.logits, b.logits)
    assert torch.equal(a.token_dev, b.token_dev)


def test_noalloc_step_rejects_oversized_scratch(lib, torch_mod):
    """One KV head and 32 query heads at position 32767: the attention split
    plan has 1024 chunks, about 17 MB of partials, more than the fixed array."""
    import gncx_amd.decode as dec

    torch = torch_mod
    shape = dec.Qwen3Shape(n_layers=1, embed=256, n_heads=32, n_kv=1, head_dim=128, ffn=512, vocab=600)
    model = dec.build_model(torch, shape, seed=32)
    d = dec.Decoder(lib, torch, model, max_seq=32768, fused=True, native=True)
    d.logits.fill_(7.0)
    torch.cuda.synchronize()
    assert _noalloc(lib, d, 5, 32767, 1) == -1
    msg = lib.gncx_hip_last_error().decode()
    assert "scratch" in msg, msg
    assert lib.gncx_hip_last_status() != 0
    torch.cuda.synchronize()
    assert bool((d.logits == 7.0).all()), "a rejected step must enqueue nothing"
    # the same step through the regular entry point runs
    d._step(5, 32767, True)
    torch.cuda.synchronize()
    gncx.check(lib)
    assert 0 <= int(d.token_dev.item()) < shape.vocab
