"""GPU: the Qwen3-shaped replay driver (gnc-x_amd/decode.py) against the same
call sequence composed from the oracle on the CPU, at a small shape.

The oracle side restates GNCXStreamer:forward_token for the Qwen3 branch
(lua/gncx_streamer.lua:759-965): RMSNorm, Q/K/V matvecs, per-head Q/K RMSNorm,
NEOX RoPE, attention with a KV write at pos, output projection and residual,
RMSNorm, gate/up, SwiGLU, down and residual, then the final norm and the tied
Q6_K lm_head.  Bar: logits within 1e-3 relative L2 at every step, for decode
steps and for prefill (whose projections run through matbatch with fp16-pair
operands, within ~2e-7 of the integer block dots), teacher-forced on both
sides."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import gncx, rel_l2
from oracle_model import OracleModel

pytestmark = pytest.mark.gpu
TOL = 1e-3
TOL_PREFILL = 1e-3


def small_shape():
    import gncx_amd.decode as dec
    return dec.Qwen3Shape(n_layers=2, embed=256, n_heads=4, n_kv=2, head_dim=64, ffn=512, vocab=600)


@pytest.mark.parametrize("fused", [False, True])
def test_decode_steps_match_oracle(lib, oracle, torch_mod, fused):
    import gncx_amd.decode as dec
    lib.gncx_hip_set_stream(None)
    model = dec.build_model(torch_mod, small_shape(), seed=5)
    d = dec.Decoder(lib, torch_mod, model, max_seq=64, fused=fused)
    ref = OracleModel(oracle, model)
    tokens = [3, 599, 17, 250, 0, 42, 511, 7]
    for pos, tok in enumerate(tokens):
        got = d.forward_token(tok, pos).cpu().numpy()
        gncx.check(lib)
        want = ref.step(tok, pos)
        err = rel_l2(got, want)
        print(f"decode fused={fused} pos={pos} rel_l2={err:.2e}")
        assert err < TOL, (pos, err)


@pytest.mark.parametrize("fused,hd", [(False, 64), (True, 64), (True, 128)])
def test_prefill_then_decode_matches_oracle(lib, oracle, torch_mod, fused, hd):
    """prefill (matbatch projections on the matrix cores; per-token norms and
    attention, or with fused=True batched norms and one causal attention pass:
    the batched kernels at head_dim 128, one step per token at 64) then greedy
    decode steps, teacher-forced on both sides."""
    import gncx_amd.decode as dec
    shape = small_shape()
    if hd != shape.head_dim:
        shape = dec.Qwen3Shape(n_layers=2, embed=256, n_heads=4, n_kv=2, head_dim=hd, ffn=512, vocab=600)
    model = dec.build_model(torch_mod, shape, seed=9)
    d = dec.Decoder(lib, torch_mod, model, max_seq=64, fused=fused)
    ref = OracleModel(oracle, model)
    prompt = [11, 22, 33, 44, 55, 66, 77, 88, 99, 123, 321, 456]
    got = d.prefill(prompt).cpu().numpy()
    gncx.check(lib)
    for pos, tok in enumerate(prompt):
        want = ref.step(tok, pos)
    err = rel_l2(got, want)
    print(f"prefill fused={fused} rel_l2={err:.2e}")
    assert err < TOL_PREFILL
    tok = d.greedy(d.logits)
    for pos in range(len(prompt), len(prompt) + 3):
        got = d.forward_token(tok, pos).cpu().numpy()
        want = ref.step(tok, pos)
        err = rel_l2(got, want)
        print(f"decode after prefill pos={pos} rel_l2={err:.2e}")
        assert err < TOL_PREFILL
        tok = int(np.argmax(want))


def test_decode_from_gguf_file_host_pointers(lib, oracle, torch_mod, tmp_path):
    """The streamer's addressing (lua/gncx_gguf.lua:223-306, streamer.lua:664-696):
    a mapped GGUF file whose weights reach the library as host pointers
    (base, offset) and are uploaded once.  Logits equal those of the same
    bytes in device memory, bit for bit, and the oracle's within 1e-3."""
    import gncx_amd.decode as dec
    dec.write_model_gguf(tmp_path / "m.gguf", small_shape(), seed=21)
    mh = dec.load_model_gguf(tmp_path / "m.gguf")
    md = dec.Model(mh.shape, torch_mod.from_numpy(np.array(mh.blob)).cuda(), dict(mh.offsets))
    dh = dec.Decoder(lib, torch_mod, mh, max_seq=32)
    dd = dec.Decoder(lib, torch_mod, md, max_seq=32)
    ref = OracleModel(oracle, mh)
    try:
        for pos, tok in enumerate([5, 77, 599, 0]):
            a = dh.forward_token(tok, pos).cpu().numpy()
            gncx.check(lib)
            b = dd.forward_token(tok, pos).cpu().numpy()
            assert np.array_equal(a, b), pos
            err = rel_l2(a, ref.step(tok, pos))
            print(f"gguf decode pos={pos} rel_l2={err:.2e}")
            assert err < TOL
        assert lib.gncx_hip_weight_bytes() > 0
    finally:
        lib.gncx_hip_weight_forget(None)  # the mapping goes away with the test


@pytest.mark.parametrize("fused", [False, True])
def test_host_buffers_match_device_buffers(lib, torch_mod, tmp_path, fused):
    """The unchanged streamer's contract end to end: weights from a mapped GGUF
    file, and every activation buffer and KV cache in host memory (inputs
    staged, outputs written back before each call returns, caches mirrored on
    the device, residual adds on the host).  Prefill and decode logits equal
    those of device-resident buffers bit for bit."""
    import gncx_amd.decode as dec
    dec.write_model_gguf(tmp_path / "m.gguf", small_shape(), seed=33)
    m = dec.load_model_gguf(tmp_path / "m.gguf")
    dh = dec.Decoder(lib, torch_mod, m, max_seq=32, fused=fused, device="cpu")
    dd = dec.Decoder(lib, torch_mod, m, max_seq=32, fused=fused, device="cuda")
    try:
        prompt = [7, 8, 9, 300, 599, 1]
        a = dh.prefill(prompt).numpy().copy()
        gncx.check(lib)
        b = dd.prefill(prompt).cpu().numpy()
        assert np.array_equal(a, b)
        tok = int(np.argmax(a))
        for pos in range(len(prompt), len(prompt) + 3):
            a = dh.forward_token(tok, pos).numpy().copy()
            gncx.check(lib)
            b = dd.forward_token(tok, pos).cpu().numpy()
            assert np.array_equal(a, b), pos
            tok = int(np.argmax(a))
        assert np.array_equal(dh.kc[1].numpy()[:pos + 1], dd.kc[1].cpu().numpy()[:pos + 1])
    finally:
        lib.gncx_hip_weight_forget(None)
        lib.gncx_hip_kv_forget(None)


@pytest.mark.parametrize("layer_type", ["q4_k", "q8_0"])
def test_native_step_equals_fused_calls(lib, torch_mod, layer_type):
    """gncx_hip_decode_step (the whole token issued by the library, add+RMSNorm
    fused into the Q/K/V and gate/up launches, SwiGLU into gate/up) gives the
    logits of the Python-issued fused call sequence bit for bit.  The Q8_0 case
    has an FFN width (96) whose gate/up rows do not split evenly over the
    grid, so it also runs the separate-kernel fallback of the SwiGLU epilogue."""
    import gncx_amd.decode as dec
    if layer_type == "q4_k":
        shape = small_shape()
    else:
        shape = dec.Qwen3Shape(n_layers=2, embed=256, n_heads=4, n_kv=2, head_dim=64, ffn=96, vocab=600,
                               layer_type=gncx.Q8_0)
    model = _build_any(torch_mod, shape, seed=13)
    a = dec.Decoder(lib, torch_mod, model, max_seq=32, fused=True)
    b = dec.Decoder(lib, torch_mod, model, max_seq=32, fused=True, native=True)
    for pos, tok in enumerate([3, 599, 17, 250, 0, 42]):
        want = a.forward_token(tok, pos).cpu().numpy()
        gncx.check(lib)
        got = b.forward_token(tok, pos).cpu().numpy()
        gncx.check(lib)
        print(f"native {layer_type} pos={pos} equal={np.array_equal(got, want)}")
        assert np.array_equal(got, want), (pos, rel_l2(got, want))
    for l in range(shape.n_layers):
        assert torch_mod.equal(a.kc[l][:6], b.kc[l][:6]) and torch_mod.equal(a.vc[l][:6], b.vc[l][:6])


def _build_any(torch, shape, seed):
    """build_model for Q4_K layers, or Q8_0 layers (32-int8 blocks, fp16 d)."""
    import gncx_amd.decode as dec
    if shape.layer_type != gncx.Q8_0:
        return dec.build_model(torch, shape, seed=seed)
    q4 = dec.Qwen3Shape(**{**shape.__dict__, "layer_type": gncx.Q4_K})
    lay = dec._layout(shape)
    offsets, total = {}, 0
    for name, kind, rows, cols in lay:
        total = (total + 31) // 32 * 32
        offsets[name] = total
        total += dec._nbytes(kind, rows, cols)
    ref = dec.build_model(torch, q4, seed=seed)  # norms and the Q6_K table come from here
    blob = torch.empty(total, dtype=torch.uint8, device="cuda")
    g = torch.Generator(device="cuda").manual_seed(seed + 100)
    for name, kind, rows, cols in lay:
        o, n = offsets[name], dec._nbytes(kind, rows, cols)
        if kind == gncx.Q8_0:
            blk = blob[o:o + n].view(-1, 34)
            blk.copy_(torch.randint(0, 256, blk.shape, generator=g, device="cuda", dtype=torch.uint8))
            d = (0.02 * torch.randn(blk.shape[0], 1, generator=g, device="cuda")).abs().to(torch.float16)
            blk[:, 0:2].copy_(d.view(torch.uint8).view(-1, 2))
        else:
            ro = ref.offsets[name]
            blob[o:o + n].copy_(ref.blob[ro:ro + n])
    return dec.Model(shape, blob, offsets)


def test_native_greedy_loop(lib, oracle, torch_mod):
    """decode_greedy: steps that feed their own device argmax back (token_id
    -1) pick the tokens a host loop picks from the same logits, and match the
    oracle-composed model's greedy tokens; the log holds one token per position."""
    import gncx_amd.decode as dec
    model = dec.build_model(torch_mod, small_shape(), seed=17)
    a = dec.Decoder(lib, torch_mod, model, max_seq=32, fused=True, native=True)
    b = dec.Decoder(lib, torch_mod, model, max_seq=32, fused=True, native=True)
    got = a.decode_greedy(5, 0, 10)
    gncx.check(lib)
    want, tok = [], 5
    ref = OracleModel(oracle, model)
    ref_toks, rt = [], 5
    for pos in range(10):
        tok = int(torch_mod.argmax(b.forward_token(tok, pos)).item())
        want.append(tok)
        lg = ref.step(rt, pos)
        rt = int(np.argmax(lg))
        ref_toks.append(rt)
    print("native greedy", got, "host", want, "oracle", ref_toks)
    assert got == want
    assert got == ref_toks
    assert a.token_log[10:].eq(-1).all()
