#!/usr/bin/env python3
"""Benchmark of the quantised decode GEMV on one MI355X.

Headline (`value`): gncx_xfold_universal_matvec on Q4_K 4096 -> 14336 (the
gate/up GEMV of Llama-3-8B / Qwen3-8B-sized models) with weights, x and y
resident in HBM, as whole-job throughput in GB/s of algorithmic bytes
(weights once + fp32 x + fp32 y per step), the back-to-back calls issued from
native code (gncx_bench_native.so) as an integrating C/C++ caller issues them.
One step is one matvec call (activation quantisation and the GEMV run in one
kernel).  Weight copies are rotated so the working set (> 512 MB) cannot sit
in the 256 MB Infinity Cache.

Also reported: `roofline` of that kernel (HIP-event durations on the
library's stream, beside the measured read ceiling of the same bytes),
`cpu_baseline` (the reference library compiled from its
own source, timed on this host on a bounded sample), and `extra` figures for
the other decode GEMV shapes, the decode-attention step, matbatch at B = 64,
256 and 512, and decode tok/s of a Qwen3-8B-shaped model (2048-token prompt
prefilled, then 256 greedy tokens) through the streamer's call sequence.

  python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--no-extra]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import pathlib
import platform
import sys
import time

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent
HBM_PEAK_GBPS = 8000.0
# sources the headline GEMV kernel is built from: a traffic figure measured on
# other sources is stale and is not reported
GEMV_SOURCES = ["gnc-x_amd/csrc/gemv.hip", "gnc-x_amd/csrc/gncx_slots.h", "gnc-x_amd/csrc/gncx_device.h",
                "gnc-x_amd/csrc/gncx_formats.h"]
TRAFFIC_JSON = ROOT / "profiles" / "traffic_gemv_q4k_4096x14336.json"
FETCH_SCALE, WRITE_SCALE = 2.0, 1.0  # profiles/hbm_counter_calibration.md
MFMA_FP16_PEAK = 2.5e15  # dense fp16 matrix-core FLOP/s of one MI355X
METRIC = "Q4_K GEMV HBM GB/s (% of peak); decode tok/s, Qwen3-8B-shaped, 1 GPU"


def import_pkg():
    import importlib.util
    root = ROOT / "gnc-x_amd"
    if "gncx_amd" not in sys.modules:
        spec = importlib.util.spec_from_file_location("gncx_amd", root / "__init__.py",
                                                      submodule_search_locations=[str(root)])
        mod = importlib.util.module_from_spec(spec)
        sys.modules["gncx_amd"] = mod
        spec.loader.exec_module(mod)
    import gncx_amd.synth  # noqa: F401
    return sys.modules["gncx_amd"]


class HipEvents:
    """hipEvent pairs recorded on the library's stream."""

    def __init__(self, stream: int):
        self.hip = C.CDLL("libamdhip64.so")
        self.stream = C.c_void_p(stream)

    def create(self, n: int):
        evs = []
        for _ in range(n):
            e = C.c_void_p()
            assert self.hip.hipEventCreate(C.byref(e)) == 0
            evs.append(e)
        return evs

    def record(self, e):
        assert self.hip.hipEventRecord(e, self.stream) == 0

    def elapsed_ms(self, a, b) -> float:
        ms = C.c_float()
        assert self.hip.hipEventSynchronize(b) == 0
        assert self.hip.hipEventElapsedTime(C.byref(ms), a, b) == 0
        return ms.value

    def destroy(self, evs):
        for e in evs:
            self.hip.hipEventDestroy(e)


def sources_sha256(paths) -> str:
    import hashlib
    h = hashlib.sha256()
    for p in paths:
        h.update(p.encode())
        h.update((ROOT / p).read_bytes())
    return h.hexdigest()


def headline_traffic():
    """(HBM bytes per launch or None, note): the figure of TRAFFIC_JSON when
    it was measured on the current GEMV sources."""
    if not TRAFFIC_JSON.exists():
        return None, "no counter measurement"
    t = json.loads(TRAFFIC_JSON.read_text())
    if t.get("source_sha256") != sources_sha256(GEMV_SOURCES):
        return None, "counter measurement is of other GEMV sources (stale)"
    return t.get("hbm_bytes_per_launch"), "FETCH_SIZE x %.1f + WRITE_SIZE x %.1f per dispatch, median" % (
        FETCH_SCALE, WRITE_SCALE)


def write_traffic_json(fetch_csv: str, write_csv: str, commands: list) -> dict:
    """profiles/traffic_*.json from the counter CSVs of two rocprofv3 --pmc
    runs (FETCH_SIZE, then WRITE_SIZE) of the headline loop: the median
    reading of the GEMV's dispatches, scaled to bytes, stamped with the hash
    of the GEMV sources it was measured on."""
    import csv

    def med(path, counter):
        v = sorted(float(r["Counter_Value"]) for r in csv.DictReader(open(path))
                   if r["Counter_Name"] == counter and "gemv" in r["Kernel_Name"])
        return v[len(v) // 2], len(v)
    f, nf = med(fetch_csv, "FETCH_SIZE")
    w, _ = med(write_csv, "WRITE_SIZE")
    hbm = int(round((f * FETCH_SCALE + w * WRITE_SCALE) * 1024))
    alg = 4096 // 256 * 144 * 14336 + 4 * 4096 + 4 * 14336
    out = {"kernel": "the headline GEMV (gemv_band_kernel, Q4_K 4096 -> 14336)",
           "workload": "gncx_xfold_universal_matvec Q4_K 4096->14336, device pointers, 16 rotated weight copies",
           "hbm_bytes_per_launch": hbm, "algorithmic_bytes_per_launch": alg, "ratio": round(hbm / alg, 4),
           "fetch_size_kib_per_dispatch_median": f, "write_size_kib_per_dispatch_median": w,
           "fetch_scale": FETCH_SCALE, "write_scale": WRITE_SCALE, "dispatches": nf, "commands": commands,
           "scale_from": "hbm_counter_calibration.md",
           "sources": GEMV_SOURCES, "source_sha256": sources_sha256(GEMV_SOURCES)}
    TRAFFIC_JSON.write_text(json.dumps(out, indent=1) + "\n")
    return out


def gemv_bytes(pkg, t: int, k: int, n: int) -> int:
    return pkg.row_bytes(t, k) * n + 4 * k + 4 * n


_NATIVE = None


def bench_native():
    """gnc-x_amd/bin/gncx_bench_native.so: the native matvec loop and the
    plain-read ceiling kernels (built with the library)."""
    global _NATIVE
    if _NATIVE is None:
        so = ROOT / "gnc-x_amd" / "bin" / "gncx_bench_native.so"
        if not so.exists():
            raise FileNotFoundError(f"{so} is not built (run __graft_entry__.build())")
        lib = C.CDLL(str(so))
        lib.gncx_bench_read_loop.restype = C.c_int
        lib.gncx_bench_read_loop.argtypes = [C.c_void_p, C.c_int32, C.c_size_t, C.c_uint32, C.c_int32, C.c_int32,
                                             C.c_void_p, C.POINTER(C.c_float)]
        lib.gncx_bench_matvec_loop.restype = C.c_int
        lib.gncx_bench_matvec_loop.argtypes = [C.c_void_p, C.c_int32, C.c_int32, C.c_void_p, C.c_int32, C.c_int32,
                                               C.c_void_p, C.c_int32, C.POINTER(C.c_double)]
        _NATIVE = lib
    return _NATIVE


def read_ceiling(ptrs, nbytes: int, row_bytes: int, steps: int, stream: int) -> dict:
    """Plain streaming reads of the same rotated weight buffers the GEMV is
    timed on (HIP events around back-to-back launches): the grid-stride
    pattern (the fastest found) and the GEMV's own row pattern."""
    nat = bench_native()
    arr = (C.c_void_p * len(ptrs))(*ptrs)
    out = {}
    for name, pattern in (("grid_stride", 0), ("gemv_row_pattern", 1)):
        us = C.c_float()
        rc = nat.gncx_bench_read_loop(arr, len(ptrs), nbytes, row_bytes, pattern, steps, C.c_void_p(stream),
                                      C.byref(us))
        if rc != 0:
            raise RuntimeError(f"gncx_bench_read_loop: HIP error {rc}")
        out[name] = {"us": round(us.value, 3), "gbps": round(nbytes / (us.value * 1e-6) / 1e9, 1),
                     "frac_of_peak": round(nbytes / (us.value * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)}
    return out


def time_gemv(pkg, lib, torch, t, k, n, steps, warmup, copies, seed=1):
    """Returns dict: wall ms/step, mean/median kernel us (events), GB/s."""
    w_host = pkg.synth.make_weights(t, n, k, seed=seed)
    x_host = pkg.synth.make_activations(1, k, seed=seed + 1)
    ws = [torch.from_numpy(w_host).cuda() for _ in range(copies)]
    x = torch.from_numpy(x_host).cuda()
    y = torch.zeros(n, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    fn = lib.gncx_xfold_universal_matvec
    wp = [w.data_ptr() for w in ws]
    xp, yp = x.data_ptr(), y.data_ptr()
    for i in range(warmup):
        fn(wp[i % copies], 0, t, xp, None, k, n, yp, None)
    torch.cuda.synchronize()
    pkg.check(lib)
    # wall-clock pass: K back-to-back steps
    t0 = time.perf_counter()
    for i in range(steps):
        fn(wp[i % copies], 0, t, xp, None, k, n, yp, None)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    pkg.check(lib)
    # the same loop issued from native code (gncx_bench_native.so calling the
    # C-ABI as an integrating C/C++ caller does): the host issue rate of
    # Python and ctypes (~9 us per call) is above the GPU's time per call
    nat = bench_native()
    us_native = C.c_double()
    rc = nat.gncx_bench_matvec_loop((C.c_void_p * copies)(*wp), copies, t, xp, k, n, yp, steps, C.byref(us_native))
    if rc != 0:
        raise RuntimeError(f"gncx_bench_matvec_loop failed: {rc} {lib.gncx_hip_last_error().decode()}")
    pkg.check(lib)
    # event pass: one event pair around the whole back-to-back loop on the
    # library stream; per-launch pairs would add the event overhead (~5 us)
    # to every launch
    ev = HipEvents(lib.gncx_hip_get_stream() or 0)
    e0, e1 = ev.create(2)
    ev.record(e0)
    for i in range(steps):
        fn(wp[i % copies], 0, t, xp, None, k, n, yp, None)
    ev.record(e1)
    kernel_us = ev.elapsed_ms(e0, e1) * 1e3 / steps
    ev.destroy([e0, e1])
    nbytes = gemv_bytes(pkg, t, k, n)
    ceiling = read_ceiling(wp, w_host.nbytes, pkg.row_bytes(t, k), steps, lib.gncx_hip_get_stream() or 0)
    del ws
    torch.cuda.empty_cache()
    return {
        "bytes": nbytes,
        "wall_ms": wall_ms,
        "wall_ms_native": us_native.value * 1e-3,
        "kernel_us_mean": kernel_us,
        "gbps_wall": nbytes / (wall_ms * 1e-3) / 1e9,
        "gbps_wall_native": nbytes / (us_native.value * 1e-6) / 1e9,
        "gbps_kernel": nbytes / (kernel_us * 1e-6) / 1e9,
        "read_ceiling": ceiling,
        "w_host": w_host,
        "x_host": x_host,
    }


ROTATE_BYTES = 512 << 20  # weight copies rotated per shape: twice the 256 MB Infinity Cache


def time_matbatch(pkg, lib, torch, t, k, n, b, steps):
    """gncx_xfold_universal_matbatch with device pointers; one HIP-event pair
    around `steps` back-to-back calls (act quantisation + the MFMA product),
    rotating weight copies of at least 512 MB in all."""
    w_host = pkg.synth.make_weights(t, n, k, seed=11)
    copies = max(2, -(-ROTATE_BYTES // w_host.nbytes))
    steps = max(steps, copies)
    ws = [torch.from_numpy(w_host).cuda() for _ in range(copies)]
    x = torch.from_numpy(pkg.synth.make_activations(b, k, seed=12).reshape(b, k)).cuda()
    y = torch.zeros(b, n, dtype=torch.float32, device="cuda")
    fn = lib.gncx_xfold_universal_matbatch
    args = lambda i: (ws[i % copies].data_ptr(), 0, t, x.data_ptr(), b, k, n, y.data_ptr(), None)  # noqa: E731
    for i in range(3):
        fn(*args(i))
    torch.cuda.synchronize()
    pkg.check(lib)
    ev = HipEvents(lib.gncx_hip_get_stream() or 0)
    e0, e1 = ev.create(2)
    ev.record(e0)
    for i in range(steps):
        fn(*args(i))
    ev.record(e1)
    us = ev.elapsed_ms(e0, e1) * 1e3 / steps
    ev.destroy([e0, e1])
    pkg.check(lib)
    flops = 2.0 * b * k * n
    nbytes = pkg.row_bytes(t, k) * n + 4 * b * k + 4 * b * n
    del ws
    torch.cuda.empty_cache()
    return {"us": round(us, 2), "tflops": round(flops / (us * 1e-6) / 1e12, 1),
            "frac_fp16_mfma_peak": round(flops / (us * 1e-6) / MFMA_FP16_PEAK, 4),
            "gbps": round(nbytes / (us * 1e-6) / 1e9, 1), "weight_copies": copies}


MATBATCH_SHAPES = {"q4k_4096x4096": (12, 4096, 4096), "q4k_4096x14336": (12, 4096, 14336),
                   "q6k_14336x4096": (14, 14336, 4096)}
PREFILL_SHAPES = {"q4k_4096x4096_b2048": (12, 4096, 4096), "q4k_4096x12288_b2048": (12, 4096, 12288),
                  "q4k_12288x4096_b2048": (12, 12288, 4096)}


def matbatch_extras(pkg, lib, torch, steps=20):
    """Matbatch at B = 64 / 256 / 512 on the prefill shapes, and the B = 2048
    prefill matrices of the Qwen3-8B-shaped model.  GFLOP/s count 2 B K N
    (the useful products); the kernel issues three fp16 MFMA products each."""
    mb = {}
    for name, (tt, kk, nn) in MATBATCH_SHAPES.items():
        for bb in (64, 256, 512):
            mb[f"{name}_b{bb}"] = time_matbatch(pkg, lib, torch, tt, kk, nn, bb, steps)
    for name, (tt, kk, nn) in PREFILL_SHAPES.items():
        mb[name] = time_matbatch(pkg, lib, torch, tt, kk, nn, 2048, 10)
    return mb


def time_attention(lib, torch, H, KV, hd, ctx, sw, steps, copies):
    """Device-resident KV caches (N(0,1)), one step at pos = ctx - 1."""
    g = torch.Generator(device="cuda").manual_seed(ctx + sw + KV)
    kcs = [torch.randn(ctx, KV * hd, device="cuda", generator=g) for _ in range(copies)]
    vcs = [torch.randn(ctx, KV * hd, device="cuda", generator=g) for _ in range(copies)]
    q = torch.randn(H * hd, device="cuda", generator=g)
    kn = torch.randn(KV * hd, device="cuda", generator=g)
    vn = torch.randn(KV * hd, device="cuda", generator=g)
    out = torch.zeros(H * hd, device="cuda")
    torch.cuda.synchronize()
    fn = lib.gncx_mqa_attention_step_ext
    args = lambda i: (q.data_ptr(), kn.data_ptr(), vn.data_ptr(), kcs[i % copies].data_ptr(),  # noqa: E731
                      vcs[i % copies].data_ptr(), ctx - 1, H, KV, hd, 1.0 / np.sqrt(hd), sw, 1, out.data_ptr())
    for i in range(5):
        fn(*args(i))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        fn(*args(i))
    torch.cuda.synchronize()
    wall_us = (time.perf_counter() - t0) * 1e6 / steps
    win = min(ctx, sw) if sw > 0 else ctx
    nbytes = 2 * 4 * KV * hd * win + 4 * (2 * H * hd + 2 * KV * hd)
    del kcs, vcs
    torch.cuda.empty_cache()
    return {"us_per_step": wall_us, "bytes": nbytes, "gbps": nbytes / (wall_us * 1e-6) / 1e9}


ATTENTION_SHAPES = {  # name: (query heads, KV heads, head_dim, context, sliding window, KV copies rotated)
    "gqa32x8_ctx512": (32, 8, 128, 512, 0, 160), "gqa32x8_ctx4096": (32, 8, 128, 4096, 0, 16),
    "gqa32x8_ctx32768": (32, 8, 128, 32768, 0, 3), "gqa32x8_swa1024": (32, 8, 128, 2048, 1024, 64),
    "mqa32x1_ctx32768": (32, 1, 128, 32768, 0, 16),
}


def attention_extras(lib, torch, steps=50):
    att = {}
    for name, (H, KV, hd, ctx, sw, cp) in ATTENTION_SHAPES.items():
        r = time_attention(lib, torch, H, KV, hd, ctx, sw, steps, cp)
        att[name] = {"us_per_step": round(r["us_per_step"], 2), "gbps": round(r["gbps"], 1)}
    return att


def time_decode(pkg, lib, torch, prompt_len, n_tokens, seed=1):
    """Qwen3-8B-shaped random-init model (decode.QWEN3_8B): prefill a random
    prompt through the streamer's prefill call sequence, then greedy decode
    steps through forward_token's; the unchanged call sequence and the fused
    one (the library's launch-saving extensions: attention with its Q/K norm
    and RoPE prologue, Q/K/V and gate/up as one GEMV each, residual add with
    the following RMSNorm) each decode n_tokens.  Wall-clock, synchronised
    around each timed loop (the greedy argmax synchronises every token anyway)."""
    import gncx_amd.decode as dec
    t0 = time.perf_counter()
    model = dec.build_model(torch, dec.QWEN3_8B, seed=seed)
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t0
    s = dec.QWEN3_8B
    g = torch.Generator().manual_seed(seed + 1)
    prompt = torch.randint(0, s.vocab, (prompt_len,), generator=g).tolist()
    # prefill through the library's batched extensions (own KV caches), timed
    # beside the streamer's per-token call sequence below
    d2 = dec.Decoder(lib, torch, model, max_seq=prompt_len + 1, fused=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    logits_f = d2.prefill(prompt).clone()
    torch.cuda.synchronize()
    prefill_fused_s = time.perf_counter() - t0
    pkg.check(lib)
    del d2
    torch.cuda.empty_cache()
    d = dec.Decoder(lib, torch, model, max_seq=prompt_len + 4 * n_tokens + 1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    logits = d.prefill(prompt)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    pkg.check(lib)
    prefill_rel = float(torch.linalg.vector_norm(logits_f - logits) / torch.linalg.vector_norm(logits))
    res = {}
    pos = prompt_len
    tok = d.greedy(logits)
    for mode in ("streamer", "fused", "native"):
        d.fused, d.native = mode != "streamer", mode == "native"
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n_tokens):
            tok = d.greedy(d.forward_token(tok, pos))
            pos += 1
        torch.cuda.synchronize()
        res[mode] = (time.perf_counter() - t0) / n_tokens
        pkg.check(lib)
    # the native step feeding its own device argmax back: no host round trip per token
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    toks = d.decode_greedy(tok, pos, n_tokens)
    res["native_greedy"] = (time.perf_counter() - t0) / n_tokens
    pkg.check(lib)
    pos += n_tokens
    assert len(toks) == n_tokens and all(0 <= t < s.vocab for t in toks)
    # the unchanged streamer's contract: every buffer and KV cache in host
    # memory from gncx_ram_alloc_colored, the 4-phase token array passed as
    # the streamer passes it (short prompt: its per-token prefill alone syncs
    # ~10 times per token and layer).  Synchronous: each call stages its
    # inputs and writes its outputs back before returning.  Lazy: the buffers
    # keep device copies and only the host's own accesses bring data back.
    host_prompt, host_tokens = 128, 32
    del d
    torch.cuda.empty_cache()
    host_runs = {}
    for lazy, driver in ((0, "python"), (1, "python"), (0, "c"), (1, "c")):
        lib.gncx_hip_set_host_coherence(lazy)
        dh = dec.Decoder(lib, torch, model, max_seq=host_prompt + host_tokens + 1, device="cpu", host="ram",
                         tokens=True, driver=driver)
        try:
            tok_h = dh.greedy(dh.prefill(prompt[:host_prompt]))
            seq = []
            t0 = time.perf_counter()
            for i in range(host_tokens):
                tok_h = dh.greedy(dh.forward_token(tok_h, host_prompt + i))
                seq.append(tok_h)
            host_runs[lazy, driver] = ((time.perf_counter() - t0) / host_tokens, seq)
            pkg.check(lib)
        finally:
            lib.gncx_hip_set_host_coherence(0)
            dh.close()
            del dh
            lib.gncx_hip_kv_forget(None)
    host_tok_s = {k: round(1.0 / v[0], 1) for k, v in host_runs.items()}
    assert all(v[1] == host_runs[0, "python"][1] for v in host_runs.values()), "host-buffer runs disagree"
    weight_bytes = model.blob.numel()
    kv_bytes = 2 * s.n_layers * s.kv_dim * 4 * (prompt_len + n_tokens)  # K and V rows read at the mid position
    del model
    torch.cuda.empty_cache()
    best = res["native_greedy"]
    return {"decode_tok_s": round(1.0 / res["streamer"], 1), "decode_ms_per_token": round(res["streamer"] * 1e3, 3),
            "decode_tok_s_fused": round(1.0 / res["fused"], 1),
            "decode_ms_per_token_fused": round(res["fused"] * 1e3, 3),
            "decode_tok_s_native": round(1.0 / res["native"], 1),
            "decode_ms_per_token_native": round(res["native"] * 1e3, 3),
            "decode_tok_s_native_device_greedy": round(1.0 / best, 1),
            "decode_ms_per_token_native_device_greedy": round(best * 1e3, 3),
            "hbm_gbps_effective_native_device_greedy": round((weight_bytes + kv_bytes) / best / 1e9, 1),
            "hbm_gbps_effective": round((weight_bytes + kv_bytes) / res["streamer"] / 1e9, 1),
            "prefill_tokens": prompt_len, "prefill_s": round(prefill_s, 3),
            "prefill_tok_s": round(prompt_len / prefill_s, 1),
            "prefill_s_fused": round(prefill_fused_s, 3), "prefill_tok_s_fused": round(prompt_len / prefill_fused_s, 1),
            "prefill_fused_vs_unfused_logits_rel_l2": round(prefill_rel, 7), "decode_tokens_each": n_tokens,
            "decode_tok_s_host_buffers": host_tok_s[0, "python"],
            "decode_tok_s_host_buffers_lazy": host_tok_s[1, "python"],
            "decode_tok_s_host_buffers_native_caller": host_tok_s[0, "c"],
            "decode_tok_s_host_buffers_native_caller_lazy": host_tok_s[1, "c"],
            "host_buffers_positions": f"{host_prompt}..{host_prompt + host_tokens - 1} (every call's inputs and "
                                      "outputs in host buffers from gncx_ram_alloc_colored and the 4-phase token "
                                      "array, as the unchanged streamer passes them, issued from Python or "
                                      "(_native_caller) from gncx_streamer_replay.so as LuaJIT's FFI issues "
                                      "them; _lazy: with gncx_hip_set_host_coherence(1); all four runs pick the "
                                      "same greedy tokens)",
            "weights_bytes": weight_bytes, "model_build_s": round(build_s, 2),
            "model": "Qwen3-8B-shaped random-init: 36 layers, hidden 4096, 32/8 heads x 128, FFN 12288, "
                     "vocab 151936; Q4_K attention/FFN, tied Q6_K token_embd as lm_head",
            "positions": f"{prompt_len}..{pos - 1}",
            "modes": "decode_tok_s: the streamer's call sequence issued from Python; _fused: the launch-saving "
                     "extensions from Python; _native: gncx_hip_decode_step (the library issues the token, "
                     "add+RMSNorm and SwiGLU fused into the matvecs), host argmax per token; "
                     "_native_device_greedy: the same steps feeding their own device argmax back"}


def decode_only(pkg, lib, torch, mode, prompt_len, n_tokens, seed=1):
    """The decode of time_decode in one call sequence: a fused prefill of the
    random prompt, then n_tokens greedy steps (the native mode feeds its
    device argmax back)."""
    import gncx_amd.decode as dec
    s = dec.QWEN3_8B
    model = dec.build_model(torch, s, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    prompt = torch.randint(0, s.vocab, (prompt_len,), generator=g).tolist()
    d = dec.Decoder(lib, torch, model, max_seq=prompt_len + n_tokens + 1, fused=True)
    tok = d.greedy(d.prefill(prompt))
    d.fused, d.native = mode != "streamer", mode == "native"
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    if mode == "native":
        d.decode_greedy(tok, prompt_len, n_tokens)
    else:
        for i in range(n_tokens):
            tok = d.greedy(d.forward_token(tok, prompt_len + i))
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / n_tokens
    pkg.check(lib)
    return {"decode_mode": mode, "decode_tok_s": round(1.0 / dt, 1), "ms_per_token": round(dt * 1e3, 3),
            "positions": f"{prompt_len}..{prompt_len + n_tokens - 1}"}


def cpu_baseline(pkg, t, k, n, w_host, x_host, seconds=10.0):
    """The reference's own matvec (compiled from its source) on this host's
    cores with its default pool size, clamp(hardware threads, 2, 12)
    (csrc/gncx_llm_kernels.cpp:139-141); the oracle restatement (1 thread)
    if the reference build is absent."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import pyoracle
    nbytes = gemv_bytes(pkg, t, k, n)
    try:
        impl, kind = pyoracle.Reference(), "reference"
        cores = min(max(os.cpu_count() or 1, 2), 12)
    except FileNotFoundError:
        impl, kind, cores = pyoracle.Oracle(), "port", 1
    for _ in range(3):
        impl.matvec(t, w_host, x_host, k, n)
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 5:
        t0 = time.perf_counter()
        impl.matvec(t, w_host, x_host, k, n)
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    cpu = platform.processor() or ""
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                cpu = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": kind,
            "sample": f"{len(times)} calls of the same Q4_K {k}->{n} matvec (median {med * 1e3:.2f} ms), "
                      f"{sum(times):.1f} s of CPU work, host '{cpu}', os.cpu_count()={os.cpu_count()}"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--copies", type=int, default=16, help="weight copies rotated to defeat the MALL")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--decode-prompt", type=int, default=2048)
    ap.add_argument("--decode-tokens", type=int, default=256)
    ap.add_argument("--decode-only", choices=["streamer", "fused", "native"], default=None,
                    help="only the decode measurement: prefill the prompt (fused), then --decode-tokens greedy "
                         "tokens through one call sequence, and print its rate (for kernel profiles)")
    ap.add_argument("--traffic-json", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="write profiles/traffic_gemv_q4k_4096x14336.json from the counter CSVs of two rocprofv3 "
                         "--pmc runs (FETCH_SIZE, then WRITE_SIZE) of 'bench.py --no-extra --no-cpu --no-decode' "
                         "and exit")
    ap.add_argument("--matbatch-only", action="store_true",
                    help="only the matbatch measurements (for kernel profiles)")
    ap.add_argument("--attention-only", action="store_true",
                    help="only the attention-step measurements (for kernel profiles)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 5 device copies of MIB MiB (the known-size kernel that scales the "
                         "FETCH_SIZE / WRITE_SIZE counters to bytes) and exit")
    args = ap.parse_args()
    if args.traffic_json:
        cmd = "rocprofv3 --pmc {c} --output-format csv -d rocprof_out/traffic -o {o} -- python3 bench.py " \
              "--steps 200 --warmup 20 --no-extra --no-cpu --no-decode"
        print(json.dumps(write_traffic_json(*args.traffic_json, [cmd.format(c="FETCH_SIZE", o="fetch"),
                                                                 cmd.format(c="WRITE_SIZE", o="write")])))
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: there is no multi-GPU path (GEMV would shard by output rows, "
              "attention by KV head)", file=sys.stderr)
        return 2

    import torch
    if args.copy_calibration > 0:
        n = args.copy_calibration << 20
        src = torch.ones(n // 4, dtype=torch.int32, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "launches": 5}), flush=True)
        return 0

    pkg = import_pkg()
    lib = pkg.load()
    assert lib.gncx_hip_init(0) == 0, lib.gncx_hip_last_error()
    lib.gncx_hip_set_stream(C.c_void_p(torch.cuda.current_stream().cuda_stream))
    if args.decode_only:
        print(json.dumps(decode_only(pkg, lib, torch, args.decode_only, args.decode_prompt, args.decode_tokens)),
              flush=True)
        return 0
    if args.matbatch_only:
        print(json.dumps({"matbatch": matbatch_extras(pkg, lib, torch)}), flush=True)
        return 0
    if args.attention_only:
        print(json.dumps({"attention": attention_extras(lib, torch)}), flush=True)
        return 0

    t, k, n = pkg.Q4_K, 4096, 14336
    head = time_gemv(pkg, lib, torch, t, k, n, args.steps, args.warmup, args.copies)
    achieved = head["bytes"] / (head["kernel_us_mean"] * 1e-6) / 1e9
    traffic, traffic_note = headline_traffic()

    extra = {}
    if not args.no_extra:
        gem = {}
        for name, (tt, kk, nn, cp) in {
            "q6k_14336x4096": (pkg.Q6_K, 14336, 4096, 12),
            "q8_0_4096x4096": (pkg.Q8_0, 4096, 4096, 32),
            "q4_0_4096x4096": (pkg.Q4_0, 4096, 4096, 64),
            "q6k_4096x128256_lm_head": (pkg.Q6_K, 4096, 128256, 2),
            "q4k_4096x4096": (pkg.Q4_K, 4096, 4096, 64),
        }.items():
            r = time_gemv(pkg, lib, torch, tt, kk, nn, max(50, args.steps // 2), 10, cp, seed=7)
            rc = r["read_ceiling"]["grid_stride"]
            gem[name] = {"gbps_wall": round(r["gbps_wall"], 1), "gbps_wall_native": round(r["gbps_wall_native"], 1),
                         "gbps_kernel": round(r["gbps_kernel"], 1), "kernel_us": round(r["kernel_us_mean"], 2),
                         "frac_kernel": round(r["gbps_kernel"] / HBM_PEAK_GBPS, 4),
                         "read_ceiling_us": rc["us"], "read_ceiling_frac_of_peak": rc["frac_of_peak"],
                         "frac_of_read_ceiling": round(rc["us"] / r["kernel_us_mean"], 4)}
        extra["gemv"] = gem
        extra["attention"] = attention_extras(lib, torch)
        extra["matbatch"] = matbatch_extras(pkg, lib, torch)
    if not args.no_decode:
        extra["decode_qwen3_8b"] = time_decode(pkg, lib, torch, args.decode_prompt, args.decode_tokens)

    cpu = None if args.no_cpu else cpu_baseline(pkg, t, k, n, head["w_host"], head["x_host"], args.cpu_seconds)
    line = {
        "metric": METRIC,
        "value": round(head["gbps_wall_native"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["wall_ms_native"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded GGUF Q4_K blocks, x ~ N(0,1))",
        "config": {"workload": "gncx_matvec Q4_K 4096->14336 (gate/up decode GEMV)", "in_dim": k, "out_dim": n,
                   "bytes_per_step": head["bytes"], "weight_copies_rotated": args.copies,
                   "inputs": "resident in HBM (device pointers through the reference C-ABI)",
                   "issued_from": "native code (gncx_bench_native.so calling the C-ABI, wall clock around the "
                                  "back-to-back loop)",
                   "value_issued_from_python_gbps": round(head["gbps_wall"], 2),
                   "ms_per_step_issued_from_python": round(head["wall_ms"], 5)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic, "traffic_note": traffic_note,
                     "kernel_us_mean": round(head["kernel_us_mean"], 3),
                     "timing": "HIP events around the back-to-back timed loop on the library stream",
                     "read_ceiling": head["read_ceiling"],
                     "frac_of_read_ceiling": round(head["read_ceiling"]["grid_stride"]["us"] / head["kernel_us_mean"], 4),
                     "read_ceiling_note": "plain streaming reads of the same 16 rotated weight copies, HIP events "
                                          "around back-to-back launches: the best pattern found (grid stride, "
                                          "512 x 1024 threads) and the GEMV's own row pattern; one launch of this "
                                          "size cannot read faster than grid_stride"},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
