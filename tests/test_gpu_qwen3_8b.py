"""GPU: the Qwen3-8B-shaped model end to end at its own widths, against the
oracle-composed model (tests/oracle_model.py).

Shape: hidden 4096, 32 query and 8 KV heads of 128, SwiGLU FFN 12288, vocab
151936, Q4_K layer matrices, and the tied Q6_K token_embd as both embedding
table and lm_head (lua/gncx_streamer.lua:951-962).  Each run prefills a prompt
through matbatch (lua/gncx_streamer.lua:968-1208), then decodes greedily
(:759-965), teacher-forced on both sides: the library is fed the tokens the
oracle's logits pick.  Bar: logits within 1e-3 relative L2 after the prompt
and after every decode step.

Both the streamer's own call sequence (per-token RMSNorm, heads-RMSNorm, RoPE
and attention calls) and the library's fused extensions (batched norms, one
causal attention pass) run over the same model and are held to the same bar.
All 36 layers run with a short prompt; a 300-token prompt, which takes the
256-token matbatch tiles and several causal attention blocks, runs 4 layers
at the full widths; and the decode workload's own 2048-token prompt (the
B = 2048 matbatch plans, causal attention over 2048 positions, then decode
steps at positions 2048-2050 whose attention spans the whole prefilled cache)
runs 4 layers at the full widths against the oracle's batched prefill.
The 36-layer model also runs from a GGUF file through host pointers and host
buffers, as the unchanged streamer drives it.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import gncx, rel_l2
from oracle_model import OracleModel

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _teacher_forced(lib, torch, oracle, model, prompt, n_decode, max_seq, batched_oracle=False):
    import gncx_amd.decode as dec

    ref = OracleModel(oracle, model, max_seq=max_seq)
    if batched_oracle:
        want = [ref.prefill(prompt, progress=lambda m: print(m, flush=True))]
    else:
        for pos, tok in enumerate(prompt[:-1]):
            ref.step(tok, pos, logits=False)
        want = [ref.step(prompt[-1], len(prompt) - 1)]
    toks = []
    for i in range(n_decode):
        toks.append(int(np.argmax(want[-1])))
        want.append(ref.step(toks[-1], len(prompt) + i))
    print(f"oracle tokens {toks}", flush=True)
    for fused in (False, True):
        d = dec.Decoder(lib, torch, model, max_seq=max_seq, fused=fused)
        got = d.prefill(prompt).cpu().numpy()
        gncx.check(lib)
        errs = [rel_l2(got, want[0])]
        picks = [int(np.argmax(got))]
        for i, tok in enumerate(toks):
            got = d.forward_token(tok, len(prompt) + i).cpu().numpy()
            gncx.check(lib)
            errs.append(rel_l2(got, want[i + 1]))
            picks.append(int(np.argmax(got)))
        print(f"layers={model.shape.n_layers} prompt={len(prompt)} fused={fused} rel_l2="
              + " ".join(f"{e:.2e}" for e in errs) + f" library picks {picks[:-1]}", flush=True)
        assert all(np.isfinite(errs)) and max(errs) < TOL, errs
        del d


def test_qwen3_8b_36_layers(lib, oracle, torch_mod):
    import gncx_amd.decode as dec

    torch = torch_mod
    model = dec.build_model(torch, dec.QWEN3_8B, seed=2024)
    try:
        rng = np.random.default_rng(11)
        prompt = [int(t) for t in rng.integers(0, dec.QWEN3_8B.vocab, 24)]
        _teacher_forced(lib, torch, oracle, model, prompt, n_decode=3, max_seq=32)
    finally:
        lib.gncx_hip_weight_forget(None)
        del model
        torch.cuda.empty_cache()


def test_qwen3_8b_widths_300_token_prompt(lib, oracle, torch_mod):
    import gncx_amd.decode as dec

    torch = torch_mod
    shape = dec.Qwen3Shape(n_layers=4)
    model = dec.build_model(torch, shape, seed=7)
    try:
        rng = np.random.default_rng(12)
        prompt = [int(t) for t in rng.integers(0, shape.vocab, 300)]
        _teacher_forced(lib, torch, oracle, model, prompt, n_decode=2, max_seq=320)
    finally:
        lib.gncx_hip_weight_forget(None)
        del model
        torch.cuda.empty_cache()


@pytest.mark.timeout(900)
def test_qwen3_8b_widths_2048_token_prompt(lib, oracle, torch_mod):
    """The decode workload's prompt length at the full widths (4 layers): the
    library's prefill through the streamer's call sequence and through the
    fused extensions (B = 2048 multi-matrix matbatch, one causal attention
    pass over 2048 positions), then 3 decode steps at positions 2048-2050,
    against the oracle's prefill (matbatch projections and the streamer's
    attention loop, lua/gncx_streamer.lua:968-1208) and its decode steps."""
    import gncx_amd.decode as dec

    torch = torch_mod
    shape = dec.Qwen3Shape(n_layers=4)
    model = dec.build_model(torch, shape, seed=2048)
    try:
        rng = np.random.default_rng(13)
        prompt = [int(t) for t in rng.integers(0, shape.vocab, 2048)]
        _teacher_forced(lib, torch, oracle, model, prompt, n_decode=3, max_seq=2048 + 4, batched_oracle=True)
    finally:
        lib.gncx_hip_weight_forget(None)
        del model
        torch.cuda.empty_cache()


@pytest.mark.timeout(900)
def test_qwen3_8b_36_layers_gguf_host_buffers(lib, oracle, torch_mod, tmp_path):
    """The unchanged streamer's contract at the full model: a 36-layer
    Qwen3-8B-shaped GGUF file mapped read-only (every weight reaches the
    library as a host pointer, base + offset, lua/gncx_gguf.lua:223-306), every
    activation buffer and KV cache from gncx_ram_alloc_colored (host memory,
    lua/gncx_streamer.lua:461-477), the streamer's own call sequence for an
    8-token prompt and 2 decode steps, synchronous and with lazy coherence;
    logits against the oracle's within 1e-3 after the prompt and each step."""
    import gncx_amd.decode as dec

    torch = torch_mod
    path = tmp_path / "qwen3_8b.gguf"
    dec.write_model_gguf(path, dec.QWEN3_8B, seed=2025)
    print(f"wrote {path.stat().st_size / 1e9:.2f} GB", flush=True)
    m = dec.load_model_gguf(path)
    assert m.shape.n_layers == 36 and m.shape.embed == 4096 and m.shape.vocab == dec.QWEN3_8B.vocab
    rng = np.random.default_rng(14)
    prompt = [int(t) for t in rng.integers(0, m.shape.vocab, 8)]
    ref = OracleModel(oracle, m, max_seq=16)
    for pos, tok in enumerate(prompt[:-1]):
        ref.step(tok, pos, logits=False)
        print(f"oracle position {pos}", flush=True)
    want = [ref.step(prompt[-1], len(prompt) - 1)]
    toks = []
    for i in range(2):
        toks.append(int(np.argmax(want[-1])))
        want.append(ref.step(toks[-1], len(prompt) + i))
    print(f"oracle tokens {toks}", flush=True)
    try:
        for lazy in (0, 1):
            lib.gncx_hip_set_host_coherence(lazy)
            d = dec.Decoder(lib, torch, m, max_seq=16, device="cpu", host="ram")
            try:
                got = d.prefill(prompt).numpy().copy()
                gncx.check(lib)
                errs = [rel_l2(got, want[0])]
                for i, tok in enumerate(toks):
                    got = d.forward_token(tok, len(prompt) + i).numpy().copy()
                    gncx.check(lib)
                    errs.append(rel_l2(got, want[i + 1]))
                print(f"36 layers, GGUF host pointers, host buffers, lazy={lazy}: rel_l2 "
                      + " ".join(f"{e:.2e}" for e in errs), flush=True)
                assert all(np.isfinite(errs)) and max(errs) < TOL, errs
            finally:
                lib.gncx_hip_set_host_coherence(0)
                d.close()
                lib.gncx_hip_kv_forget(None)
    finally:
        lib.gncx_hip_weight_forget(None)
        del m
